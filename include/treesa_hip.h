/* treesa_hip.h -- C ABI of the MI355X TreeSA sweep library (libtreesa_hip.so).
 *
 * The reference ships one CUDA binary whose host class Runner<W> drives the sweep kernels directly
 * (csrc/treesa_gpu.cu:1415-2062).  Here that device-facing half of Runner is a C ABI: the CLI host
 * (treesa_gpu_amd/bin/treesa_gpu, the drop-in for TREESA_GPU_BINARY, treesa_gpu/driver.py:45) and the
 * Python tests call these entry points with plain pointers and sizes.  Every call returns TSA_OK (0)
 * or a negative status; tsa_last_error() then holds a message.  No C++ exception crosses the ABI.
 * A context owns its device buffers and one HIP stream; calls on one context are synchronous with
 * respect to the host buffers passed in and must come from one host thread at a time.
 *
 * Chain record (what tsa_upload / tsa_download exchange), in 64-bit words, one record per chain,
 * records back to back (the layout is returned by tsa_layout):
 *   [0, nint*W)              labels of internal node m+i at i*W: the unsliced output-label set, bit l%64
 *                            of word l/64 for label l (W = words per set)
 *   [ch_off, ch_off+ceil(nint/2))  children, uint32 per internal node i: left | right << 16
 *                            (node ids: leaves 0..m-1, internal m..2m-2, root 2m-2)
 *   [s_off, s_off+W)         slice set S (sliced labels have log2 size 0 in every cost)
 *   padding up to chain_words (a multiple of 2, so records are 16-byte aligned)
 * Reference layout with 32-bit words: csrc/treesa_gpu.cu:15-20, 1439-1448.
 */
#ifndef TREESA_HIP_H
#define TREESA_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSA_OK 0
#define TSA_ERR_ARG (-1)     /* invalid argument or size */
#define TSA_ERR_HIP (-2)     /* HIP runtime error (message names the call) */
#define TSA_ERR_FIT (-3)     /* node arrays do not fit in LDS */
#define TSA_ERR_LIBM (-4)    /* the host libm disagrees with the restated expf/exp2f/log2f */

#define TSA_ORDER_PAR 0      /* random-priority independent-set phases (csrc/common.h:240-272) */
#define TSA_ORDER_PREORDER 1 /* the Julia pre-order sweep (csrc/cpu_ref.h:87-126) */

#define TSA_MODE_TC 0        /* tc + sc penalty (Julia tcscrw) */
#define TSA_MODE_GPU 1       /* modeled GPU time, roofline model v1 */
#define TSA_MODE_H100 2      /* modeled time, measured H100 model */

/* Kernel selection flags for tsa_create (results never depend on them). */
#define TSA_KERNEL_AUTO 0
#define TSA_KERNEL_LDS 1     /* chain staged in LDS (fails with TSA_ERR_FIT if it does not fit) */
#define TSA_KERNEL_GLOBAL 2  /* chain worked on in HBM, node arrays in LDS, one wave per chain */
#define TSA_KERNEL_WIDE 3    /* runtime-width chains, par order: G lanes per proposal, K workgroups per chain
                                (fails with TSA_ERR_FIT if the chain does not qualify); AUTO picks it for
                                runtime-width chains without slice moves */

typedef struct tsa_layout_t {
  int32_t m, nint, nlab;
  int32_t W;            /* 64-bit words per label set (1, 2, 4, 8 on the register path, else ceil(nlab/64)
                           rounded up to even, so that label sets and S are 16-byte aligned) */
  int32_t runtime_width;/* 1: kernels loop over W words at run time (wide path); 0: W is a register width */
  int32_t ch_off;       /* word offset of the children array */
  int32_t s_off;        /* word offset of S */
  int32_t chain_words;  /* words per chain record */
} tsa_layout_t;

/* Energy model and run parameters; the reference's Params (csrc/common.h:60-94) minus the layout. */
typedef struct tsa_config_t {
  int32_t mode;                 /* TSA_MODE_* */
  float sc_target, sc_weight;
  uint32_t key0, key1;          /* Philox key: low / high half of splitmix64(seed) (csrc/treesa_gpu.cu:1457-1459) */
  int32_t slicing;              /* 1: every cost uses label sets masked by ~S */
  int32_t slice_moves;          /* slice proposals after every slice_every-th global sweep (0: none) */
  int32_t slice_every;
  int32_t max_slices;           /* cap on |S| */
  int32_t par_follow;           /* par order: an accepted visit re-arms an already visited pivot */
  int32_t par_band;             /* par order: 0, or 2..16 = top-down priorities within bands of L levels */
  int32_t kernel;               /* TSA_KERNEL_* */
  /* GPU roofline model v1, log2 units (csrc/treesa_gpu.cu:1460-1465) */
  float lpeak, lbw, llaunch;
  int32_t m0, n0, k0;
  /* measured H100 model, log2 of the constants (csrc/treesa_gpu.cu:1466-1474) */
  float v2_l3launch, v2_lperm2, v2_lcc_bit, v2_lcc_cell, v2_ltc_bit, v2_ltc_pad, v2_ltc_out, v2_lsmall_cell;
  int32_t v2_small_rank;
  /* wide kernel plan (0 = automatic): waves per workgroup (1..16), workgroups per chain (1..16) */
  int32_t wide_waves, wide_wgs;
  /* 1: every tsa_sweeps on the register-width path also leaves the energies of the swept population ready,
   * so that tsa_energy / tsa_track launch no energy kernel; for callers that evaluate after every level.  The
   * sweep kernel computes every node's cost while the chain is still staged in LDS and folds it there, or,
   * with more than twice the chains that fit on the device at once (or with 2), leaves the costs to a fold
   * kernel that folds every chain in one round.  The wide path keeps a node-cost cache instead and its energy call
   * only folds it. */
  int32_t fused_energy;
  /* chunk summaries of the wide kernel (the reference's --sums / --no-sum, csrc/treesa_gpu.cu:1444-1448):
   * 0 = automatic (on from 64 words per label set, 4096 labels), 1 = on, -1 = off.  With summaries a
   * visit loads only the 16-byte chunks that are nonzero in one of its label sets; results do not change */
  int32_t sums;
  /* wide kernel: lanes per proposal (4, 8, 16, 32 or 64; 0 = automatic) */
  int32_t wide_lanes;
  /* tsa_track after a sweep whose node costs are folded apart (the wide path, or fused_energy with the fold
   * kernel, without slice moves): 0 = automatic, the fold and the selection of that sweep's snapshot run on
   * a second stream beside the next sweep; -1 = never, they run on the sweep's stream.  Results do not change */
  int32_t track_overlap;
  /* pre-order sweeps: one chain per workgroup, whose three helper waves draw every internal node's random
   * numbers (the rule word and the Metropolis threshold) for the next sweep while the first wave sweeps, instead
   * of each visit drawing its own: 0 = automatic (on for at most one chain per compute unit, where the sweeping
   * wave's dependent steps bound the sweep and three SIMDs idle), 1 = on, -1 = off.  Results do not change */
  int32_t draw_waves;
  /* wide kernel with several workgroups per chain: polls a workgroup waits at the chain's check-in for the
   * others before it sweeps the chain alone (0 = default, about a millisecond; -1 = at once, every chain swept
   * by one workgroup -- for tests).  Results do not change */
  int32_t wide_join;
  /* tsa_anneal: 0 = automatic (the level loop in one launch when every chain of it is resident on the device
   * at once, else one sweep launch and one selection per level), 1 = the level loop in one launch whenever the
   * context's kernels run it, -1 = per-level launches.  Results do not change */
  int32_t level_loop;
  /* tsa_anneal without the one-launch level loop, on the one-wave LDS kernels whose selection overlaps the next
   * sweep with the fold apart (more than twice the chains the device holds at once, par order, no slicing):
   * levels per sweep launch, each evaluated level leaving its own snapshot for the fold and the selection
   * (0 = automatic: 8, the most; 1 = one level per launch).  Results do not change */
  int32_t level_blocks;
} tsa_config_t;

typedef struct tsa_ctx tsa_ctx;

/* Record layout for an instance with m tensors and nlab labels.  wide != 0 forces the runtime-width
 * path (the reference's --wide).  Pure host function: needs no GPU.
 * Replaces the layout set-up of Runner<W>::Runner, csrc/treesa_gpu.cu:1439-1448, 2078-2085. */
int tsa_layout(int32_t m, int32_t nlab, int32_t wide, tsa_layout_t* out);

/* Create a context for nchains chains on the current HIP device.  leaf: m*W words, the label sets of
 * the input tensors in the layout's word format; leaf_sc = largest leaf tensor (log2).
 * Replaces Runner<W>::Runner + alloc, csrc/treesa_gpu.cu:1435-1548, 1564-1578. */
int tsa_create(const tsa_layout_t* lay, const uint64_t* leaf, int32_t leaf_sc, const tsa_config_t* cfg,
               int32_t nchains, tsa_ctx** out);

/* Upload the whole population (nchains * chain_words words).  Synchronous.  On the wide path it also builds
 * the population's derived data before it returns: the chunk summaries (as init_chains builds them with the
 * labels, csrc/treesa_gpu.cu:1604-1612) and, in tc mode, the node-cost cache and the energies.  Replaces the
 * H2D copy of init_chains, csrc/treesa_gpu.cu:1629. */
int tsa_upload(tsa_ctx* ctx, const uint64_t* population);

/* Download count chain records starting at chain c0.  Replaces the best-chain and --check copies,
 * csrc/treesa_gpu.cu:1823, 1948-1949. */
int tsa_download(tsa_ctx* ctx, int32_t c0, int32_t count, uint64_t* out);
/* tsa_download enqueued on the context's stream without waiting: out (page-locked, tsa_host_alloc) holds the
 * records, as they are at this point of the stream, once a later synchronizing call returns (tsa_download,
 * tsa_energy, tsa_track_end, tsa_wait).  No counterpart in the reference (its best-chain copy waits,
 * csrc/treesa_gpu.cu:1823); for a host-side level loop that keeps the best chain's record without stopping
 * the device for it. */
int tsa_download_async(tsa_ctx* ctx, int32_t c0, int32_t count, uint64_t* out);
/* Wait until everything enqueued on the context has run.  No counterpart in the reference (its calls are
 * synchronous); pairs with tsa_download_async. */
int tsa_wait(tsa_ctx* ctx);

/* Enqueue nsweeps sweeps of every chain at inverse temperature beta, global sweep counter sweep0
 * (the RNG counter), in TSA_ORDER_*; slice moves follow every sweep s with (sweep0+s+1) % slice_every
 * == 0 when slice_moves > 0.  Asynchronous (with overlapped tracking, see track_overlap, it first waits
 * on the host for the selection of three launches back to finish); event-timed.  Replaces Runner::sweeps / sweeps_mode,
 * csrc/treesa_gpu.cu:1659-1716. */
int tsa_sweeps(tsa_ctx* ctx, int32_t order, float beta, uint32_t sweep0, int32_t nsweeps);

/* Wait for every tsa_sweeps since the previous call and return their summed event-timed kernel time in
 * ms (0 if none pending).
 * Replaces the cudaEventElapsedTime bookkeeping of run_anneal, csrc/treesa_gpu.cu:1799-1809, 1870-1876. */
int tsa_sweeps_ms(tsa_ctx* ctx, double* ms);

/* Per-chain energy: lc = log2 of the per-slice cost (lse fold of node costs), sc = largest tensor
 * (masked by S, leaves included), ns = |S|.  Synchronous.  Replaces Runner::energy + k_energy,
 * csrc/treesa_gpu.cu:999-1014, 1717-1729. */
int tsa_energy(tsa_ctx* ctx, float* lc, int32_t* sc, int32_t* ns);

/* Population step: chain c <- chain anc[c] for every c.  Asynchronous (anc is copied before the call
 * returns); later calls on the context see the new population.  The copy itself is made by the next sweep
 * launch of the kernels that stage a chain in LDS (each chain starts from its ancestor's record) or, before
 * any other call's work, by a copy kernel.  Replaces Runner::resample + k_copy, csrc/treesa_gpu.cu:1016-1022,
 * 1925-1933. */
int tsa_resample(tsa_ctx* ctx, const int32_t* anc);

/* Switch the energy mode (stage 2 of a two-stage run, csrc/treesa_gpu.cu:1790-1798). */
int tsa_set_mode(tsa_ctx* ctx, int32_t mode);

/* Counters since creation: proposals, accepts, phases (par) or frontier steps (preorder), node
 * visits, slice proposals, slice accepts, busy lanes.  Replaces the d_stats copy,
 * csrc/treesa_gpu.cu:1880-1881. */
int tsa_stats(tsa_ctx* ctx, uint64_t out[7]);

/* Counters of the wide kernel with chunk summaries since creation: out[0] = 16-byte chunk positions a
 * proposal loaded (one per set bit of the union of its summaries; each is read from the label sets of the
 * visited node, the other child and the two grandchildren, and from the pivot's too in the gpu / h100 modes),
 * out[1] = chunk positions written by accepted rotations.  Both stay 0 without summaries.  No counterpart in
 * the reference: it is the measured byte count of the summary path's roofline. */
int tsa_chunk_stats(tsa_ctx* ctx, uint64_t out[2]);

/* Device-side best tracking for runs without population steps (scheme indep): after a level's sweeps,
 * tsa_track enqueues the energy kernel and a selection kernel that scores every chain (lower is better,
 * the reference's score, csrc/treesa_gpu.cu:1737-1748, evaluated with the restated double log2 / exp2 of
 * tsa_select.h), keeps the lowest score over all tracked levels (first chain and first level on ties, as
 * the reference's loop at csrc/treesa_gpu.cu:1810-1824) and copies that chain's tree (children words and
 * S) on the device, and writes one trace row per tracked level.  On the wide path each sweep launch leaves
 * a snapshot of the trees and node costs, and the energy fold and selection of a level run on a second
 * stream beside the next level's sweep.  Nothing synchronizes until tsa_track_end. */
typedef struct tsa_select_t {
  int32_t mode, slicing, select_sc;
  double sc_target, sc_weight;
} tsa_select_t;

typedef struct tsa_trace_row_t {
  float lc;             /* lcost of the level's best chain */
  int32_t sc, ns;       /* its sc and |S| */
  int32_t chain;        /* its index (-1: no finite score) */
  double score;         /* its score */
  double meanE, meanNs; /* population means of the energy and of |S| */
  uint64_t ticks;       /* device wall clock when the row was written */
} tsa_trace_row_t;

/* Start tracking: best score +inf, room for max_levels rows.  Replaces the best-tracking state of
 * run_anneal, csrc/treesa_gpu.cu:1777-1779. */
int tsa_track_begin(tsa_ctx* ctx, const tsa_select_t* sel, int32_t max_levels);
/* Enqueue energy + selection for level (0 <= level < max_levels).  Asynchronous.  With overlapped tracking
 * (tsa_config_t.track_overlap) they run on a second stream beside the next tsa_sweeps, on the snapshot the
 * last sweep launch left.  Replaces the per-level energy call and score loop of run_anneal,
 * csrc/treesa_gpu.cu:1805-1832. */
int tsa_track(tsa_ctx* ctx, int32_t level);
/* Wait and return the best over the tracked levels (best_chain -1 if none), its tree in best_record (a
 * chain_words record of which the children words and S are written; its label words are a function of the
 * tree and are left as they were), max_levels trace rows (rows of untracked levels are zero) and the device
 * wall-clock rate in Hz; ticks0 = device wall clock when the session started on the device (the session's
 * start is enqueued with its first launch after tsa_track_begin). */
int tsa_track_end(tsa_ctx* ctx, int32_t* best_chain, int32_t* best_level, double* best_score, uint64_t* best_record,
                  tsa_trace_row_t* rows, uint64_t* ticks0, double* tick_hz);

/* The level loop of a run without population steps (scheme indep), levels level0 .. level0 + nlevels - 1:
 * niters[l] >= 1 sweeps at betas[l], the sweep counter running on from sweep0, and after every level with
 * evaluated[l] != 0 the energies and selection of tsa_track.  Exactly tsa_sweeps for each level followed by
 * tsa_track at the evaluated ones: the same population, statistics, trace rows and, at tsa_track_end, the
 * same best chain, level, score and tree.  It replaces the level loop of run_anneal
 * (csrc/treesa_gpu.cu:1788-1832), which the reference runs as one sweep launch and one host-side selection per
 * level.  On the LDS kernels with every chain resident at once (tsa_config_t.level_loop) the call is ONE
 * launch: each chain stays staged from its first level to its last, folds its energy and keeps its own best
 * tree after every evaluated level, and the last chain to finish a level selects while the others sweep on, so
 * no level waits for the host or for a launch (the trace row's ticks: the device clock of that selection).
 * Else it runs those per-level launches itself.  Needs tsa_track_begin (max_levels >= level0 + nlevels); a
 * session that has called tsa_track runs per-level launches, and tsa_track after a one-launch tsa_anneal in the
 * same session fails.  tsa_describe names the way the last call ran.  The kernel time counts in
 * tsa_sweeps_ms.  Asynchronous. */
int tsa_anneal(tsa_ctx* ctx, int32_t order, int32_t level0, int32_t nlevels, const float* betas,
               const int32_t* niters, const uint8_t* evaluated, uint32_t sweep0);

/* Human-readable description of the kernels this context launches (name, lanes, LDS bytes). */
int tsa_describe(tsa_ctx* ctx, char* buf, int32_t len);

/* Page-locked host memory for buffers the library copies chain records into (tsa_download,
 * tsa_track_end): copies into it run at the link's full speed instead of through the runtime's staging of
 * pageable memory.  NULL on failure; tsa_host_free(NULL) is a no-op.  No counterpart in the reference (it
 * copies into pageable memory); for callers that time the whole level loop. */
void* tsa_host_alloc(size_t bytes);
void tsa_host_free(void* p);

/* Allocation-free sweeps for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.  It runs what tsa_sweeps
 * + tsa_energy + tsa_stats do on a context, on buffers the caller owns, and allocates nothing: no context, no
 * hipMalloc / hipFree, no events.  The caller passes device pointers: leaf_dev (m * W words, the layout's leaf
 * table), population_dev (nchains records, swept in place; every record must hold a valid tree, as written by
 * tsa_download or an earlier call: nothing is checked on the host), and optionally lc_dev / sc_dev / ns_dev
 * (all or none: the energies after the last sweep) and stats_dev (7 words: the call's counters, as tsa_stats).
 * Register-width layouts only (at most 512 labels, no --wide).  stream: a hipStream_t (NULL: the null stream);
 * everything is enqueued on it and the call returns without waiting.
 * Its working memory is one static device buffer of 32 MiB per GPU (held until the process ends): the
 * counters plus, when energies are asked for, 6 bytes per internal node per chain; a call that would need more
 * fails with TSA_ERR_ARG.  The first call on a device fills the library's log2f table there with one
 * synchronous copy (make it before any graph capture).  Calls on one GPU share that buffer: calls that overlap
 * in time on one GPU (several host threads or streams) race and must be serialized by the caller. */
int tsa_sweeps_noalloc(const tsa_layout_t* lay, const tsa_config_t* cfg, int32_t leaf_sc, const uint64_t* leaf_dev,
                       uint64_t* population_dev, int32_t nchains, int32_t order, float beta, uint32_t sweep0,
                       int32_t nsweeps, float* lc_dev, int32_t* sc_dev, int32_t* ns_dev, uint64_t* stats_dev,
                       void* stream);

/* Release everything.  Replaces Runner::release, csrc/treesa_gpu.cu:1579-1582. */
int tsa_destroy(tsa_ctx* ctx);

/* Message of the last failed call on ctx (or of the last failed tsa_create / tsa_layout when ctx is
 * NULL).  Never NULL. */
const char* tsa_last_error(const tsa_ctx* ctx);

/* Single-float math shared with the kernels (host side), for tests: expf, exp2f and log2f on [1, 2]
 * exactly as the device computes them.  which: 0 expf, 1 exp2f, 2 log2f.  Returns the float. */
float tsa_host_math(int32_t which, float x);

#ifdef __cplusplus
}
#endif
#endif /* TREESA_HIP_H */
