"""tsa_sweeps_noalloc (the allocation-free entry point) against tsa_sweeps + tsa_energy + tsa_stats (GPU).

The population, the leaf table and the outputs live in device memory this test allocates through the HIP
runtime itself; the library call allocates nothing and keeps its working memory in one static device buffer.
Two calls in a row on the same buffer, the second smaller and in another order and energy mode, must equal a
context's results bit for bit: every record, every chain's lc / sc / |S| and the seven counters; a third call,
a repeat of the second, leaves the device's free memory unchanged (hipMemGetInfo).  A call whose
chains would need more than the static buffer is refused on the host, before anything reaches the device.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

import common
from treesa_gpu_amd import capi

pytestmark = pytest.mark.gpu

_hip = None


def hip():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        _hip.hipFree.argtypes = [ctypes.c_void_p]
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipDeviceSynchronize.argtypes = []
        _hip.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    return _hip


def free_bytes():
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip().hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


H2D, D2H = 1, 2


class DeviceArray:
    """A device copy of a numpy array (or an uninitialised one of a shape and dtype)."""

    def __init__(self, host=None, shape=None, dtype=None):
        self.host = np.ascontiguousarray(host) if host is not None else np.zeros(shape, dtype)
        self.ptr = ctypes.c_void_p()
        assert hip().hipMalloc(ctypes.byref(self.ptr), max(1, self.host.nbytes)) == 0
        if host is not None:
            assert hip().hipMemcpy(self.ptr, self.host.ctypes.data, self.host.nbytes, H2D) == 0

    def get(self):
        out = np.empty_like(self.host)
        assert hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H) == 0
        return out

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()


def setup(inst, nchains, seed):
    m, nlab, ixs, iy = common.load_instance(inst)
    lay = capi.layout(m, nlab)
    from treesa_gpu_amd import host
    I = host.Instance(common.inst_path(inst))
    pop = I.population(lay, None, nchains, seed=seed)
    leaf = np.zeros((m, lay.W), np.uint64)
    for i, ix in enumerate(ixs):
        for l in ix:
            leaf[i, l >> 6] |= np.uint64(1) << np.uint64(l & 63)
    return lay, leaf, max(len(x) for x in ixs), pop


def with_context(lay, leaf, lsc, cfg, pop, order, beta, sweep0, nsweeps):
    with capi.Context(lay, leaf, lsc, cfg, pop.shape[0]) as ctx:
        ctx.upload(pop)
        ctx.sweeps(order, beta, sweep0, nsweeps)
        lc, sc, ns = ctx.energy()
        return ctx.download(), lc, sc, ns, ctx.stats()


def without_allocation(lay, leaf, lsc, cfg, pop, order, beta, sweep0, nsweeps, bufs, mem=None):
    """The same through tsa_sweeps_noalloc on device buffers made here; with mem (a list), the device's free
    bytes just before the call and after it has finished are appended to it."""
    n = pop.shape[0]
    d_leaf = DeviceArray(leaf)
    d_pop = DeviceArray(pop)
    bufs += [d_leaf, d_pop]
    lc, sc, ns, st = (DeviceArray(shape=n, dtype=np.float32), DeviceArray(shape=n, dtype=np.int32),
                      DeviceArray(shape=n, dtype=np.int32), DeviceArray(shape=7, dtype=np.uint64))
    bufs += [lc, sc, ns, st]
    print(f"[noalloc] {n} chains, order {order}, mode {cfg.mode}", flush=True)
    assert hip().hipDeviceSynchronize() == 0
    if mem is not None:
        mem.append(free_bytes())
    capi.sweeps_noalloc(lay, cfg, lsc, d_leaf.ptr.value, d_pop.ptr.value, n, order, beta, sweep0, nsweeps,
                        lc.ptr.value, sc.ptr.value, ns.ptr.value, st.ptr.value, None)
    assert hip().hipDeviceSynchronize() == 0
    if mem is not None:
        mem.append(free_bytes())
    return d_pop.get(), lc.get(), sc.get(), ns.get(), [int(x) for x in st.get()]


def test_noalloc_equals_context_on_two_calls():
    bufs = []
    try:
        # call 1: sat100 (W = 2, chains in LDS), par order, tc mode, 600 chains from random trees
        lay, leaf, lsc, pop = setup("sat100", 600, seed=3)
        cfg = capi.make_config(mode="tc", sc_target=20.0, seed=3)
        want = with_context(lay, leaf, lsc, cfg, pop, capi.ORDER_PAR, 1.5, 5, 3)
        got = without_allocation(lay, leaf, lsc, cfg, pop, capi.ORDER_PAR, 1.5, 5, 3, bufs)
        for k, what in enumerate(("records", "lc", "sc", "ns")):
            assert np.array_equal(got[k], want[k]), what
        assert got[4] == want[4] and got[4][0] > 0
        # call 2, on the same static buffer: fewer chains, pre-order, the gpu model energy (the float lse and the
        # log2f table), an instance of another width (sat40: W = 1)
        lay2, leaf2, lsc2, pop2 = setup("sat40", 70, seed=4)
        cfg2 = capi.make_config(mode="gpu", sc_target=24.0, seed=4)
        want2 = with_context(lay2, leaf2, lsc2, cfg2, pop2, capi.ORDER_PREORDER, 2.0, 11, 2)
        got2 = without_allocation(lay2, leaf2, lsc2, cfg2, pop2, capi.ORDER_PREORDER, 2.0, 11, 2, bufs)
        for k, what in enumerate(("records", "lc", "sc", "ns")):
            assert np.array_equal(got2[k], want2[k]), what
        assert got2[4] == want2[4]
        # call 3 repeats call 2 on fresh buffers: the device's free memory is the same before and after it (the
        # library's one-time set-up -- code objects, the symbol lookup -- happened in the calls before)
        mem = []
        got3 = without_allocation(lay2, leaf2, lsc2, cfg2, pop2, capi.ORDER_PREORDER, 2.0, 11, 2, bufs, mem)
        assert mem[0] == mem[1], f"free device memory {mem[0]} before the call, {mem[1]} after"
        for k, what in enumerate(("records", "lc", "sc", "ns")):
            assert np.array_equal(got3[k], want2[k]), what
        assert got3[4] == want2[4]
    finally:
        for b in bufs:
            b.free()


def test_noalloc_refuses_more_than_its_scratch():
    # the refusals happen on the host before any launch; the buffers are real and zero-filled all the same (zero
    # children words are leaves only: a sweep over them would read nothing out of bounds)
    lay = capi.layout(426, 100)
    cfg = capi.make_config()
    nint4 = (lay.nint + 3) & ~3
    too_many = (32 << 20) // (nint4 * 6) + 1
    bufs = [DeviceArray(np.zeros((too_many, lay.chain_words), np.uint64)), DeviceArray(np.zeros((426, lay.W), np.uint64)),
            DeviceArray(shape=too_many, dtype=np.float32), DeviceArray(shape=too_many, dtype=np.int32),
            DeviceArray(shape=too_many, dtype=np.int32)]
    try:
        pop, leaf, lc, sc, ns = (b.ptr.value for b in bufs)
        with pytest.raises(capi.TsaError, match="scratch"):
            capi.sweeps_noalloc(lay, cfg, 3, leaf, pop, too_many, capi.ORDER_PAR, 1.0, 0, 1, lc, sc, ns, None, None)
        wide = capi.layout(4096, 8064)
        with pytest.raises(capi.TsaError, match="register-width"):
            capi.sweeps_noalloc(wide, cfg, 4, leaf, pop, 8, capi.ORDER_PAR, 1.0, 0, 1, None, None, None, None, None)
    finally:
        for b in bufs:
            b.free()
