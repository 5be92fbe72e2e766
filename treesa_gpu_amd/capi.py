"""ctypes binding of libtreesa_hip.so (include/treesa_hip.h) for tests and bench.py.

The product path of the drop-in is the C++ binary ``bin/treesa_gpu`` (the reference's CLI,
csrc/treesa_gpu.cu:1330-1406); this module exposes the same C ABI to Python so that tests can drive the
kernels directly.  It raises when the native library is missing: there is no Python fallback.
"""
import ctypes
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libtreesa_hip.so")
BIN_PATH = os.path.join(HERE, "bin", "treesa_gpu")
HOST_LIB_PATH = os.path.join(HERE, "lib", "libtreesa_host.so")

ORDER_PAR, ORDER_PREORDER = 0, 1
MODES = {"tc": 0, "gpu": 1, "h100": 2}
KERNEL_AUTO, KERNEL_LDS, KERNEL_GLOBAL, KERNEL_WIDE = 0, 1, 2, 3

# Default model constants of the reference's CLI (csrc/treesa_gpu.cu:1292-1295).
DEFAULT_GM = (11.9e15, 1.6e13, 6, 6, 8, 4e-6)
DEFAULT_H100 = (4e-6, 1.23e13, 5.44e-14, 7.68e-15, 6.37e-14, 2.02e-16, 1.77e-13, 14, 1e-12)

EXPORTS = ("tsa_layout", "tsa_create", "tsa_upload", "tsa_download", "tsa_sweeps", "tsa_sweeps_ms", "tsa_energy",
           "tsa_resample", "tsa_set_mode", "tsa_stats", "tsa_chunk_stats", "tsa_describe", "tsa_destroy", "tsa_last_error",
           "tsa_host_math", "tsa_host_alloc", "tsa_host_free", "tsa_track_begin", "tsa_track", "tsa_track_end",
           "tsa_sweeps_noalloc", "tsa_anneal", "tsa_download_async", "tsa_wait")


class Layout(ctypes.Structure):
    _fields_ = [("m", ctypes.c_int32), ("nint", ctypes.c_int32), ("nlab", ctypes.c_int32), ("W", ctypes.c_int32),
                ("runtime_width", ctypes.c_int32), ("ch_off", ctypes.c_int32), ("s_off", ctypes.c_int32),
                ("chain_words", ctypes.c_int32)]


class Select(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("slicing", ctypes.c_int32), ("select_sc", ctypes.c_int32),
                ("sc_target", ctypes.c_double), ("sc_weight", ctypes.c_double)]


TRACE_ROW = np.dtype([("lc", "<f4"), ("sc", "<i4"), ("ns", "<i4"), ("chain", "<i4"), ("score", "<f8"),
                      ("meanE", "<f8"), ("meanNs", "<f8"), ("ticks", "<u8")])


class Config(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("sc_target", ctypes.c_float), ("sc_weight", ctypes.c_float),
                ("key0", ctypes.c_uint32), ("key1", ctypes.c_uint32), ("slicing", ctypes.c_int32),
                ("slice_moves", ctypes.c_int32), ("slice_every", ctypes.c_int32), ("max_slices", ctypes.c_int32),
                ("par_follow", ctypes.c_int32), ("par_band", ctypes.c_int32), ("kernel", ctypes.c_int32),
                ("lpeak", ctypes.c_float), ("lbw", ctypes.c_float), ("llaunch", ctypes.c_float),
                ("m0", ctypes.c_int32), ("n0", ctypes.c_int32), ("k0", ctypes.c_int32),
                ("v2_l3launch", ctypes.c_float), ("v2_lperm2", ctypes.c_float), ("v2_lcc_bit", ctypes.c_float),
                ("v2_lcc_cell", ctypes.c_float), ("v2_ltc_bit", ctypes.c_float), ("v2_ltc_pad", ctypes.c_float),
                ("v2_ltc_out", ctypes.c_float), ("v2_lsmall_cell", ctypes.c_float), ("v2_small_rank", ctypes.c_int32),
                ("wide_waves", ctypes.c_int32), ("wide_wgs", ctypes.c_int32), ("fused_energy", ctypes.c_int32),
                ("sums", ctypes.c_int32), ("wide_lanes", ctypes.c_int32),
                ("track_overlap", ctypes.c_int32), ("draw_waves", ctypes.c_int32), ("wide_join", ctypes.c_int32),
                ("level_loop", ctypes.c_int32), ("level_blocks", ctypes.c_int32)]


_lib = None


def load():
    """The native library (loaded once).  Raises FileNotFoundError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(f"{LIB_PATH} is missing: build it with `make -C treesa_gpu_amd` "
                                "(or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    P, I32, U32, F32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint32, ctypes.c_float
    lib.tsa_layout.argtypes = [I32, I32, I32, ctypes.POINTER(Layout)]
    lib.tsa_create.argtypes = [ctypes.POINTER(Layout), P, I32, ctypes.POINTER(Config), I32, ctypes.POINTER(P)]
    lib.tsa_upload.argtypes = [P, P]
    lib.tsa_download.argtypes = [P, I32, I32, P]
    lib.tsa_download_async.argtypes = [P, I32, I32, P]
    lib.tsa_wait.argtypes = [P]
    lib.tsa_sweeps.argtypes = [P, I32, F32, U32, I32]
    lib.tsa_sweeps_ms.argtypes = [P, ctypes.POINTER(ctypes.c_double)]
    lib.tsa_energy.argtypes = [P, P, P, P]
    lib.tsa_resample.argtypes = [P, P]
    lib.tsa_set_mode.argtypes = [P, I32]
    lib.tsa_stats.argtypes = [P, P]
    lib.tsa_chunk_stats.argtypes = [P, P]
    lib.tsa_describe.argtypes = [P, ctypes.c_char_p, I32]
    lib.tsa_destroy.argtypes = [P]
    lib.tsa_last_error.argtypes = [P]
    lib.tsa_last_error.restype = ctypes.c_char_p
    lib.tsa_host_math.argtypes = [I32, F32]
    lib.tsa_host_math.restype = F32
    lib.tsa_host_alloc.argtypes = [ctypes.c_size_t]
    lib.tsa_host_alloc.restype = P
    lib.tsa_host_free.argtypes = [P]
    lib.tsa_host_free.restype = None
    lib.tsa_track_begin.argtypes = [P, ctypes.POINTER(Select), I32]
    lib.tsa_track.argtypes = [P, I32]
    lib.tsa_track_end.argtypes = [P, P, P, P, P, P, P, P]
    lib.tsa_anneal.argtypes = [P, I32, I32, I32, P, P, P, U32]
    lib.tsa_sweeps_noalloc.argtypes = [ctypes.POINTER(Layout), ctypes.POINTER(Config), I32, P, P, I32, I32, F32, U32,
                                       I32, P, P, P, P, P]
    _lib = lib
    return lib


class TsaError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"treesa_hip error {code}: {msg}")
        self.code = code


def splitmix64(x):
    m = (1 << 64) - 1
    x = (x + 0x9E3779B97F4A7C15) & m
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & m
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & m
    return x ^ (x >> 31)


def f32_log2(x):
    """(float)std::log2(x) as the reference's host computes the model constants."""
    return float(np.float32(math.log2(x)))


def layout(m, nlab, wide=False):
    lib = load()
    out = Layout()
    rc = lib.tsa_layout(m, nlab, 1 if wide else 0, ctypes.byref(out))
    if rc != 0:
        raise TsaError(rc, lib.tsa_last_error(None).decode())
    return out


def make_config(mode="tc", sc_target=20.0, sc_weight=1.0, seed=1, slicing=False, slice_moves=1, slice_every=1,
                max_slices=0, par_follow=False, par_band=0, kernel=KERNEL_AUTO, gm=DEFAULT_GM, h100=DEFAULT_H100,
                wide_waves=0, wide_wgs=0, fused_energy=False, sums=0, wide_lanes=0, track_overlap=0, draw_waves=0, wide_join=0,
                level_loop=0, level_blocks=0):
    """Config with the fields the reference's Runner derives from its options (csrc/treesa_gpu.cu:1449-1474)."""
    k = splitmix64(seed)
    c = Config()
    c.mode = MODES[mode] if isinstance(mode, str) else int(mode)
    c.sc_target, c.sc_weight = sc_target, sc_weight
    c.key0, c.key1 = k & 0xFFFFFFFF, k >> 32
    c.slicing = 1 if slicing else 0
    c.slice_moves = slice_moves if slicing else 0
    c.slice_every = max(1, slice_every)
    c.max_slices = max_slices
    c.par_follow = 1 if par_follow else 0
    c.par_band = par_band
    c.kernel = kernel
    c.lpeak, c.lbw = f32_log2(gm[0]), f32_log2(gm[1])
    c.m0, c.n0, c.k0 = int(gm[2]), int(gm[3]), int(gm[4])
    c.llaunch = f32_log2(gm[5])
    h = h100
    c.v2_l3launch, c.v2_lperm2 = f32_log2(3 * h[0]), f32_log2(2 / h[1])
    c.v2_lcc_bit, c.v2_lcc_cell = f32_log2(h[2]), f32_log2(h[3])
    c.v2_ltc_bit, c.v2_ltc_pad, c.v2_ltc_out = f32_log2(h[4]), f32_log2(h[5]), f32_log2(h[6])
    c.v2_small_rank, c.v2_lsmall_cell = int(h[7]), f32_log2(h[8])
    c.wide_waves, c.wide_wgs = wide_waves, wide_wgs
    c.fused_energy = int(fused_energy)  # 0 / False: none, 1 / True: automatic, 2: fold kernel always
    c.sums = int(sums)
    c.wide_lanes = int(wide_lanes)
    c.track_overlap = int(track_overlap)  # 0: automatic, -1: fold and selection on the sweep's stream
    c.draw_waves = int(draw_waves)  # pre-order: 0 automatic, 1 helper waves draw ahead, -1 each visit draws
    c.wide_join = int(wide_join)  # wide kernel, K > 1: check-in polls (0 default, -1 every chain swept alone)
    c.level_loop = int(level_loop)  # tsa_anneal: 0 automatic, 1 one launch whenever possible, -1 per-level launches
    c.level_blocks = int(level_blocks)  # tsa_anneal's per-level path: levels per sweep launch (0 automatic, 1 one)
    return c


class Context:
    """One device context: a population of nchains chain records on the GPU."""

    def __init__(self, lay, leaf, leaf_sc, cfg, nchains):
        self.lib = load()
        self.lay, self.cfg, self.nchains = lay, cfg, nchains
        self._leaf = np.ascontiguousarray(leaf, dtype=np.uint64)
        h = ctypes.c_void_p()
        rc = self.lib.tsa_create(ctypes.byref(lay), self._leaf.ctypes.data, leaf_sc, ctypes.byref(cfg), nchains,
                                 ctypes.byref(h))
        if rc != 0:
            raise TsaError(rc, self.lib.tsa_last_error(None).decode())
        self.h = h

    def _check(self, rc):
        if rc != 0:
            raise TsaError(rc, self.lib.tsa_last_error(self.h).decode())

    def upload(self, pop):
        pop = np.ascontiguousarray(pop, dtype=np.uint64)
        assert pop.shape == (self.nchains, self.lay.chain_words)
        self._check(self.lib.tsa_upload(self.h, pop.ctypes.data))

    def download(self, c0=0, count=None):
        count = self.nchains - c0 if count is None else count
        out = np.zeros((count, self.lay.chain_words), dtype=np.uint64)
        self._check(self.lib.tsa_download(self.h, c0, count, out.ctypes.data))
        return out

    def sweeps(self, order, beta, sweep0, nsweeps):
        self._check(self.lib.tsa_sweeps(self.h, order, beta, sweep0, nsweeps))

    def sweeps_ms(self):
        ms = ctypes.c_double()
        self._check(self.lib.tsa_sweeps_ms(self.h, ctypes.byref(ms)))
        return ms.value

    def energy(self):
        lc = np.zeros(self.nchains, np.float32)
        sc = np.zeros(self.nchains, np.int32)
        ns = np.zeros(self.nchains, np.int32)
        self._check(self.lib.tsa_energy(self.h, lc.ctypes.data, sc.ctypes.data, ns.ctypes.data))
        return lc, sc, ns

    def resample(self, anc):
        anc = np.ascontiguousarray(anc, dtype=np.int32)
        self._check(self.lib.tsa_resample(self.h, anc.ctypes.data))

    def wait(self):
        self._check(self.lib.tsa_wait(self.h))

    def set_mode(self, mode):
        self._check(self.lib.tsa_set_mode(self.h, MODES[mode] if isinstance(mode, str) else int(mode)))

    def stats(self):
        out = np.zeros(7, np.uint64)
        self._check(self.lib.tsa_stats(self.h, out.ctypes.data))
        return [int(x) for x in out]

    def chunk_stats(self):
        """Chunk positions loaded by proposals and written by accepts on the summary path."""
        out = np.zeros(2, np.uint64)
        self._check(self.lib.tsa_chunk_stats(self.h, out.ctypes.data))
        return [int(x) for x in out]

    def track_begin(self, mode="tc", slicing=False, select_sc=False, sc_target=20.0, sc_weight=1.0, max_levels=1):
        s = Select()
        s.mode = MODES[mode] if isinstance(mode, str) else int(mode)
        s.slicing, s.select_sc = int(bool(slicing)), int(bool(select_sc))
        s.sc_target, s.sc_weight = float(sc_target), float(sc_weight)
        self._max_levels = max_levels
        self._check(self.lib.tsa_track_begin(self.h, ctypes.byref(s), max_levels))

    def track(self, level):
        self._check(self.lib.tsa_track(self.h, level))

    def anneal(self, order, betas, niters, evaluated, level0=0, sweep0=0):
        """tsa_anneal over len(betas) levels."""
        b = np.ascontiguousarray(betas, dtype=np.float32)
        it = np.ascontiguousarray(niters, dtype=np.int32)
        ev = np.ascontiguousarray(evaluated, dtype=np.uint8)
        assert len(b) == len(it) == len(ev)
        self._check(self.lib.tsa_anneal(self.h, order, level0, len(b), b.ctypes.data, it.ctypes.data, ev.ctypes.data,
                                        sweep0))

    def track_end(self):
        """(best_chain, best_level, best_score, best_record, rows, ticks0, tick_hz)."""
        bc, bl = ctypes.c_int32(), ctypes.c_int32()
        bs, hz = ctypes.c_double(), ctypes.c_double()
        t0 = ctypes.c_uint64()
        rec = np.zeros(self.lay.chain_words, np.uint64)
        rows = np.zeros(self._max_levels, TRACE_ROW)
        self._check(self.lib.tsa_track_end(self.h, ctypes.byref(bc), ctypes.byref(bl), ctypes.byref(bs), rec.ctypes.data,
                                           rows.ctypes.data, ctypes.byref(t0), ctypes.byref(hz)))
        return bc.value, bl.value, bs.value, rec, rows, t0.value, hz.value

    def describe(self):
        buf = ctypes.create_string_buffer(256)
        self._check(self.lib.tsa_describe(self.h, buf, 256))
        return buf.value.decode()

    def close(self):
        if self.h:
            self.lib.tsa_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sweeps_noalloc(lay, cfg, leaf_sc, leaf_dev, pop_dev, nchains, order, beta, sweep0, nsweeps, lc_dev=None, sc_dev=None,
                   ns_dev=None, stats_dev=None, stream=None):
    """tsa_sweeps_noalloc on device pointers (ints); raises TsaError on a refused call."""
    lib = load()
    rc = lib.tsa_sweeps_noalloc(ctypes.byref(lay), ctypes.byref(cfg), leaf_sc, leaf_dev, pop_dev, nchains, order, beta,
                                sweep0, nsweeps, lc_dev, sc_dev, ns_dev, stats_dev, stream)
    if rc != 0:
        raise TsaError(rc, lib.tsa_last_error(None).decode())
