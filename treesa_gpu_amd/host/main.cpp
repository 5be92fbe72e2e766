// main.cpp -- bin/treesa_gpu: the MI355X drop-in for the reference's treesa_gpu binary.
//
// Same command line (csrc/treesa_gpu.cu:1279-1406), same instance / tree / betas files, same JSON result
// (csrc/treesa_gpu.cu:1896-1920) and exit codes (0 ok, 1 usage / input / device error, 2 invalid final
// tree, 3 failed --check), so treesa_gpu/driver.py runs it through TREESA_GPU_BINARY unchanged.  The level
// loop (csrc/treesa_gpu.cu:1756-1933) runs here on the host; every device step goes through the C ABI of
// libtreesa_hip.so (include/treesa_hip.h).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <random>
#include <string>
#include <vector>

#include "treesa_hip.h"
#include <new>
#include "tsa_host.h"
#include "tsa_select.h"

// Page-locked host memory from the library: device-to-host copies of chain records into it run at the link's
// full speed (the best record of a 64 x 64 lattice chain is 4 MB).
template <typename T>
struct PinnedAlloc {
  using value_type = T;
  PinnedAlloc() = default;
  template <typename U>
  PinnedAlloc(const PinnedAlloc<U>&) {}
  T* allocate(size_t n) {
    void* p = tsa_host_alloc(n * sizeof(T));
    if (!p) throw std::bad_alloc();
    return static_cast<T*>(p);
  }
  void deallocate(T* p, size_t) { tsa_host_free(p); }
  bool operator==(const PinnedAlloc&) const { return true; }
  bool operator!=(const PinnedAlloc&) const { return false; }
};
using PinnedRecord = std::vector<uint64_t, PinnedAlloc<uint64_t>>;

using namespace tsa;

namespace {

struct Opts {
  std::string inst, tree, out, kernel = "auto", scheme = "indep", betas = "0.01:0.05:15", order = "par";
  std::string betas2, init_slices, init = "tree";
  int spectral_k = 4, greedy_repeat = 10;
  int niters2 = -1;
  int nchains = 1024, niters = 50, block = 0, wpb = 0, lpc = 32, eval_every = 1, ref_chains = 8, mode = 0;
  bool check = false, quiet = false, cross = true, wide = false, slicing = false, no_sum = false, force_sum = false;
  bool select_sc = false, no_overlap = false;
  int slice_moves = 1, slice_every = 1, max_slices = 0, random_slices = 0;
  int coop_max = 0, coop_min_units = -1, coop_min = 1, coop_full = 0, coop_cpl = 2, par_follow = 0, par_band = 0, wpc = 0, wide_wgs = 0, wide_lanes = 0;
  double sc_target = 20.0, sc_weight = 1.0, trunc_frac = 0.25;
  uint64_t seed = 1;
  ModelConsts mc;
  int mode2 = 1;
  int max_levels = -1;
  int bench_warmup = 0;  // untimed levels before the level loop (then the population is re-uploaded)
  bool host_select = false;  // select on the host every level even for indep runs
};

double now_s() { return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count(); }

std::string jnum(double x) {
  if (!std::isfinite(x)) return "null";
  char b[64];
  snprintf(b, sizeof b, "%.6e", x);
  return b;
}

[[noreturn]] void usage() {
  fprintf(stderr,
          "usage: treesa_gpu -i instance.txt [--tree init_tree.txt] [--nchains N] [--niters K]\n"
          "  [--betas a:step:b | --betas file:PATH | --betas b1,b2,..] [--mode tc|gpu|h100]\n"
          "  [--gm peak,bw,m0,n0,k0,launch] [--h100-model launch,perm_bw,cc_bit,cc_cell,tc_bit,tc_pad,tc_out,small_rank,small_cell]\n"
          "  [--stage2-betas SPEC [--stage2-niters K] [--stage2-mode gpu|h100]]  (continue the population)\n"
          "  [--sc-target x] [--sc-weight y] [--scheme indep|pa|trunc] [--trunc-frac f]\n"
          "  [--slicing [--slice-moves k] [--slice-every s] [--max-slices n] [--init-slices l1,l2,..]]\n"
          "  [--order par|preorder] [--kernel auto|seq|seqsm|warp|warpsm|block|par [--wpc n]] [--lpc 32|16|8] [--coop-max G] [--coop-min G0] [--coop-full G1] [--par-follow] [--par-band L] [--coop-min-units u] [--wide] [--sums|--no-sum] [--select-sc] [--block B] [--wpb W] [--seed s] [--wide-wgs K] [--wide-lanes G]\n"
          "  [--eval-every k] [--out result.json] [--check [--ref-chains R] [--random-slices k]] [--quiet]\n"
          "  [--bench-warmup W]  (W untimed levels first, then the initial population again)\n"
          "  [--host-select]  (select the best chain on the host at every level, also for --scheme indep)\n"
          "  [--no-overlap]  (device-side selection on the sweep's stream, not beside the next sweep)\n"
          "  [--init tree|spectral|greedy [--spectral-k K] [--greedy-repeat R]]  (start trees made natively when no --tree\n"
          "   is given: the K best spectral path trees, chain c from tree c %% K, or the best of R greedy runs)\n");
  exit(1);
}

[[noreturn]] void die(const std::string& msg, int code = 1) {
  fprintf(stderr, "%s\n", msg.c_str());
  exit(code);
}

Opts parse(int argc, char** argv) {
  Opts o;
  try {
    for (int i = 1; i < argc; i++) {
      const std::string a = argv[i];
      auto nx = [&]() -> std::string {
        if (i + 1 >= argc) usage();
        return argv[++i];
      };
      if (a == "-i") o.inst = nx();
      else if (a == "--tree") o.tree = nx();
      else if (a == "--init") {
        o.init = nx();
        if (o.init != "tree" && o.init != "spectral" && o.init != "greedy") usage();
      } else if (a == "--spectral-k") o.spectral_k = std::stoi(nx());
      else if (a == "--greedy-repeat") o.greedy_repeat = std::stoi(nx());
      else if (a == "--out") o.out = nx();
      else if (a == "--nchains") o.nchains = std::stoi(nx());
      else if (a == "--niters") o.niters = std::stoi(nx());
      else if (a == "--betas") o.betas = nx();
      else if (a == "--stage2-betas") o.betas2 = nx();
      else if (a == "--stage2-niters") o.niters2 = std::stoi(nx());
      else if (a == "--mode") {
        const std::string s = nx();
        o.mode = (s == "gpu") ? 1 : (s == "h100" || s == "gpu2") ? 2 : 0;
      } else if (a == "--stage2-mode") {
        const std::string s = nx();
        o.mode2 = (s == "h100" || s == "gpu2") ? 2 : 1;
      } else if (a == "--h100-model" || a == "--gm2") {
        const std::string s = nx();
        double* h = o.mc.h100;
        if (sscanf(s.c_str(), "%lf,%lf,%lf,%lf,%lf,%lf,%lf,%lf,%lf", &h[0], &h[1], &h[2], &h[3], &h[4], &h[5], &h[6],
                   &h[7], &h[8]) != 9)
          usage();
      } else if (a == "--sc-target") o.sc_target = std::stod(nx());
      else if (a == "--sc-weight") o.sc_weight = std::stod(nx());
      else if (a == "--scheme") o.scheme = nx();
      else if (a == "--trunc-frac") o.trunc_frac = std::stod(nx());
      else if (a == "--kernel") o.kernel = nx();
      else if (a == "--order") o.order = nx();
      else if (a == "--block") o.block = std::stoi(nx());
      else if (a == "--wpb") o.wpb = std::stoi(nx());
      else if (a == "--lpc") o.lpc = std::stoi(nx());
      else if (a == "--seed") o.seed = std::stoull(nx());
      else if (a == "--eval-every") o.eval_every = std::stoi(nx());
      else if (a == "--ref-chains") o.ref_chains = std::stoi(nx());
      else if (a == "--max-levels") o.max_levels = std::stoi(nx());
      else if (a == "--bench-warmup") o.bench_warmup = std::stoi(nx());
      else if (a == "--host-select") o.host_select = true;
      else if (a == "--slicing") o.slicing = true;
      else if (a == "--slice-moves") o.slice_moves = std::stoi(nx());
      else if (a == "--slice-every") o.slice_every = std::stoi(nx());
      else if (a == "--max-slices") o.max_slices = std::stoi(nx());
      else if (a == "--init-slices") {
        o.init_slices = nx();
        o.slicing = true;
      } else if (a == "--random-slices") {
        o.random_slices = std::stoi(nx());
        o.slicing = true;
      } else if (a == "--coop-max") o.coop_max = std::stoi(nx());
      else if (a == "--coop-min-units") o.coop_min_units = std::stoi(nx());
      else if (a == "--coop-min") o.coop_min = std::stoi(nx());
      else if (a == "--coop-full") o.coop_full = std::stoi(nx());
      else if (a == "--coop-chunks") o.coop_cpl = std::max(1, std::stoi(nx()));
      else if (a == "--par-follow") o.par_follow = 1;
      else if (a == "--par-band") o.par_band = std::stoi(nx());
      else if (a == "--wpc") o.wpc = std::stoi(nx());
      else if (a == "--wide-wgs") o.wide_wgs = std::stoi(nx());
      else if (a == "--wide-lanes") o.wide_lanes = std::stoi(nx());
      else if (a == "--wide") o.wide = true;
      else if (a == "--no-sum") o.no_sum = true;
      else if (a == "--select-sc") o.select_sc = true;
      else if (a == "--no-overlap") o.no_overlap = true;
      else if (a == "--sums") o.force_sum = true;
      else if (a == "--check") o.check = true;
      else if (a == "--no-cross") o.cross = false;
      else if (a == "--quiet") o.quiet = true;
      else if (a == "--gm") {
        const std::string s = nx();
        double* g = o.mc.gm;
        if (sscanf(s.c_str(), "%lf,%lf,%lf,%lf,%lf,%lf", &g[0], &g[1], &g[2], &g[3], &g[4], &g[5]) != 6) usage();
      } else usage();
    }
  } catch (const std::logic_error&) {  // std::stoi / std::stod on a malformed number
    usage();
  }
  if (o.inst.empty()) usage();
  return o;
}

class Runner {
 public:
  std::vector<std::vector<uint32_t>> trees_;
  std::vector<double> init_tcs;  // tc of each start tree made by --init spectral / greedy
  double t_trees = 0.0;
  bool have_trees = false;
  Runner(const Inst& I, const Opts& O) : I(I), O(O) {
    if (tsa_layout(I.m, I.nlab, O.wide ? 1 : 0, &lay) != TSA_OK) die(tsa_last_error(nullptr));
    G = Geometry{lay.W, lay.ch_off, lay.s_off, lay.chain_words};
    leaf = leaf_sets(I, lay.W);
    lsc = leaf_sc(I);
    ML = model_log2(O.mc);
    mode = O.mode;
    if (O.order != "par" && O.order != "preorder") die("--order par|preorder");
    // order "par" (default) runs the par kernel; an explicit --kernel other than auto/par means the
    // pre-order sweep (csrc/treesa_gpu.cu:1480-1483)
    kernel = O.kernel;
    if (kernel == "auto" && O.order == "par" && O.lpc == 32) kernel = "par";
    const bool known = kernel == "auto" || kernel == "par" || kernel == "seq" || kernel == "seqsm" ||
                       kernel == "warp" || kernel == "warpsm" || kernel == "block";
    if (!known) die("unknown --kernel " + kernel);
    order = kernel == "par" ? TSA_ORDER_PAR : TSA_ORDER_PREORDER;
    if (O.par_band == 1 || O.par_band > 16 || O.par_band < 0) die("--par-band L: 0 (off) or 2..16");
    const int slice_moves = (O.slicing && O.random_slices == 0) ? O.slice_moves : 0;
    if (slice_moves > 0 && (kernel == "seq" || kernel == "seqsm" || O.lpc != 32))
      die("slice moves need the warp kernels with --lpc 32");
    if (O.nchains < 1) die("--nchains must be at least 1");
    memset(&cfg, 0, sizeof cfg);
    cfg.mode = mode;
    cfg.sc_target = (float)O.sc_target;
    cfg.sc_weight = (float)O.sc_weight;
    const uint64_t k = splitmix64(O.seed);
    cfg.key0 = (uint32_t)k;
    cfg.key1 = (uint32_t)(k >> 32);
    cfg.slicing = O.slicing ? 1 : 0;
    cfg.slice_moves = slice_moves;
    cfg.slice_every = std::max(1, O.slice_every);
    cfg.max_slices = O.max_slices > 0 ? O.max_slices : I.nlab;
    cfg.par_follow = O.par_follow;
    cfg.par_band = O.par_band;
    cfg.kernel = (kernel == "warpsm" || kernel == "seqsm") ? TSA_KERNEL_LDS
                 : (kernel == "warp" || kernel == "seq" || kernel == "block") ? TSA_KERNEL_GLOBAL
                                                                               : TSA_KERNEL_AUTO;
    cfg.lpeak = ML.lpeak;
    cfg.lbw = ML.lbw;
    cfg.llaunch = ML.llaunch;
    cfg.m0 = ML.m0;
    cfg.n0 = ML.n0;
    cfg.k0 = ML.k0;
    cfg.v2_l3launch = ML.v2_l3launch;
    cfg.v2_lperm2 = ML.v2_lperm2;
    cfg.v2_lcc_bit = ML.v2_lcc_bit;
    cfg.v2_lcc_cell = ML.v2_lcc_cell;
    cfg.v2_ltc_bit = ML.v2_ltc_bit;
    cfg.v2_ltc_pad = ML.v2_ltc_pad;
    cfg.v2_ltc_out = ML.v2_ltc_out;
    cfg.v2_lsmall_cell = ML.v2_lsmall_cell;
    cfg.v2_small_rank = ML.v2_small_rank;
    cfg.wide_waves = O.wpc > 0 ? (O.wpc + 1) / 2 : 0;  // --wpc counts 32-lane warps
    cfg.wide_wgs = O.wide_wgs;
    cfg.wide_lanes = O.wide_lanes;
    cfg.fused_energy = O.eval_every == 1 ? 1 : 0;  // every level is evaluated: the sweep kernel evaluates too
    cfg.sums = O.no_sum ? -1 : (O.force_sum ? 1 : 0);
    cfg.track_overlap = O.no_overlap ? -1 : 0;
  }
  ~Runner() {
    if (ctx) tsa_destroy(ctx);
  }

  int run_anneal();
  int run_check();

 private:
  const Inst& I;
  const Opts& O;
  tsa_layout_t lay{};
  tsa_config_t cfg{};
  Geometry G{};
  tsa_ctx* ctx = nullptr;
  std::vector<uint64_t> leaf;
  int lsc = 0;
  ModelLog2 ML{};
  int mode = 0;
  std::string kernel;
  int order = TSA_ORDER_PAR;
  double kernel_ms = 0;

  void ck(int rc) {
    if (rc != TSA_OK) die(std::string("treesa_hip: ") + tsa_last_error(ctx));
  }
  void create(tsa_ctx** c, int kflag) {
    tsa_config_t c2 = cfg;
    c2.kernel = kflag;
    if (tsa_create(&lay, leaf.data(), lsc, &c2, O.nchains, c) != TSA_OK) {
      const std::string msg = tsa_last_error(nullptr);
      if (msg.find("fit") != std::string::npos)
        die("chains do not fit in shared memory (try --kernel warp / --lpc 32)");
      die("treesa_hip: " + msg);
    }
  }
  // start trees: the --tree file, else (--init spectral / greedy) made once here on the host
  const std::vector<std::vector<uint32_t>>& start_trees() {
    if (have_trees) return trees_;
    const double t = now_s();
    if (!O.tree.empty()) trees_ = read_trees(O.tree, I.m);
    else if (O.init == "spectral") {
      for (const SpectralOrder& so : spectral_orders(I, std::max(1, O.spectral_k), 24, 24, O.seed)) {
        trees_.push_back(path_tree(so.order));
        init_tcs.push_back(so.tc);
      }
    } else if (O.init == "greedy") {
      double tc = 0.0;
      trees_.push_back(greedy_tree(I, std::max(1, O.greedy_repeat), O.seed, &tc));
      init_tcs.push_back(tc);
    }
    t_trees = now_s() - t;
    have_trees = true;
    return trees_;
  }
  std::vector<uint64_t> init_population() {
    const std::vector<std::vector<uint32_t>>& trees = start_trees();
    std::vector<uint64_t> S0(lay.W, 0);
    if (!O.init_slices.empty()) {
      const char* p = O.init_slices.c_str();
      while (*p) {
        char* q;
        const long l = strtol(p, &q, 10);
        if (q == p) break;
        if (l < 0 || l >= I.nlab) die("bad --init-slices label");
        S0[l >> 6] |= 1ull << (l & 63);
        p = q;
        while (*p == ',' || *p == ' ') p++;
      }
    }
    std::vector<uint64_t> pop;
    build_population(I, G, trees, O.nchains, O.seed, S0, O.random_slices, pop);
    return pop;
  }
  const uint64_t* chS(const uint64_t* base) const { return O.slicing ? base + lay.s_off : nullptr; }
  const uint32_t* chCh(const uint64_t* base) const { return reinterpret_cast<const uint32_t*>(base + lay.ch_off); }

  // Selection score and population energy (tsa_select.h, the same functions the device-side tracking
  // evaluates).
  TsaSelect select_params() const {
    TsaSelect S;
    S.mode = mode;
    S.slicing = O.slicing ? 1 : 0;
    S.select_sc = O.select_sc ? 1 : 0;
    S.sc_target = O.sc_target;
    S.sc_weight = O.sc_weight;
    return S;
  }
  double score(float lc, int sc, int ns) const { return tsa_score(lc, sc, ns, select_params()); }
  double energyE(float lc, int sc, int ns) const { return tsa_energyE(lc, sc, ns, select_params()); }
  int run_levels_tracked(const std::vector<float>& betas, const std::vector<int>& lniters, uint32_t& sweep_ctr,
                         PinnedRecord& best, std::string& trace, double t0);
  void resample(const std::vector<int>& anc, std::vector<int>& family) {
    ck(tsa_resample(ctx, anc.data()));
    std::vector<int> nfm(O.nchains);
    for (int c = 0; c < O.nchains; c++) nfm[c] = family[anc[c]];
    family.swap(nfm);
  }
  std::string kernel_name() const {
    if (order == TSA_ORDER_PAR) return "par";
    char b[256] = {0};
    tsa_describe(ctx, b, sizeof b);
    return strncmp(b, "lds", 3) == 0 ? "warpsm" : "warp";
  }
};

// The level loop of an indep run with device-side selection: every level enqueues its sweeps and, at
// evaluated levels, the energy and selection kernels; the host waits once at the end.  The selected chain,
// the trace rows and the kernel time are those of the synchronous loop below (same score function, same
// first-chain / first-level tie rule); only the trace's time column comes from the device clock.
int Runner::run_levels_tracked(const std::vector<float>& betas, const std::vector<int>& lniters, uint32_t& sweep_ctr,
                               PinnedRecord& best, std::string& trace, double t0) {
  const TsaSelect S = select_params();
  tsa_select_t sel;
  sel.mode = S.mode;
  sel.slicing = S.slicing;
  sel.select_sc = S.select_sc;
  sel.sc_target = S.sc_target;
  sel.sc_weight = S.sc_weight;
  const int nlev = (int)betas.size();
  ck(tsa_track_begin(ctx, &sel, nlev));
  std::vector<char> evaluated(nlev, 0);
  for (int lev = 0; lev < nlev; lev++) {
    ck(tsa_sweeps(ctx, order, betas[lev], sweep_ctr, lniters[lev]));
    sweep_ctr += (uint32_t)lniters[lev];
    const bool last = lev + 1 == nlev;
    if (lev % O.eval_every == O.eval_every - 1 || last) {
      ck(tsa_track(ctx, lev));
      evaluated[lev] = 1;
    }
  }
  double ms = 0;
  ck(tsa_sweeps_ms(ctx, &ms));
  kernel_ms += ms;
  std::vector<tsa_trace_row_t> rows(nlev);
  int32_t bc = -1, bl = -1;
  double bs = 0, hz = 1;
  uint64_t tk0 = 0;
  ck(tsa_track_end(ctx, &bc, &bl, &bs, best.data(), rows.data(), &tk0, &hz));
  const double t_dev0 = now_s() - t0;  // the level loop has finished; device times are scaled to it
  const double span = std::max(1.0, (double)(rows[nlev - 1].ticks - tk0));
  for (int lev = 0; lev < nlev; lev++) {
    if (!evaluated[lev]) continue;
    const tsa_trace_row_t& r = rows[lev];
    const double t = t_dev0 * (double)(r.ticks - tk0) / span;
    char buf[320];
    snprintf(buf, sizeof buf, "%s[%.4f,%d,%.4f,%.6f,%d,%.6f,%d,%d,%d,%.3f]", trace.empty() ? "" : ",", t, lev,
             betas[lev], (double)r.lc, r.sc, r.meanE, O.nchains, mode, r.ns, r.meanNs);
    trace += buf;
    if (!O.quiet && (lev % 25 == 0 || lev + 1 == nlev))
      fprintf(stderr, "lev %4d beta %7.3f  best(l2cost/slice %.3f sc %d |S| %d)  meanE %.3f  mean|S| %.2f  families %d  t=%.2fs\n",
              lev, betas[lev], (double)r.lc, r.sc, r.ns, r.meanE, r.meanNs, O.nchains, t);
  }
  (void)hz;
  return bc;
}

int Runner::run_anneal() {
  std::vector<float> betas = parse_betas(O.betas);
  if (O.max_levels > 0 && (int)betas.size() > O.max_levels) betas.resize(O.max_levels);
  std::vector<int> lmode(betas.size(), O.mode), lniters(betas.size(), O.niters);
  if (!O.betas2.empty()) {
    for (float b : parse_betas(O.betas2)) {
      betas.push_back(b);
      lmode.push_back(O.mode2);
      lniters.push_back(O.niters2 > 0 ? O.niters2 : O.niters);
    }
  }
  HostEnergy H1;
  bool staged = false;
  uint32_t sweep_ctr = 0;
  const double t_start = now_s();
  uint64_t stats0[7] = {0, 0, 0, 0, 0, 0, 0}, chunks0[2] = {0, 0};
  {
    const std::vector<uint64_t> pop = init_population();  // input errors surface before the device is touched
    create(&ctx, cfg.kernel);
    ck(tsa_upload(ctx, pop.data()));
    if (O.bench_warmup > 0 && !betas.empty()) {
      // untimed warm-up levels (clocks, code objects, the tracking buffers of the level loop), then the same
      // initial population again
      std::vector<float> l(O.nchains);
      std::vector<int> s(O.nchains), n(O.nchains);
      const bool track = O.scheme == "indep" && O.betas2.empty() && !O.host_select;
      tsa_select_t sel{};
      if (track) {
        const TsaSelect S = select_params();
        sel.mode = S.mode;
        sel.slicing = S.slicing;
        sel.select_sc = S.select_sc;
        sel.sc_target = S.sc_target;
        sel.sc_weight = S.sc_weight;
        ck(tsa_track_begin(ctx, &sel, (int)betas.size()));
      }
      for (int k = 0; k < O.bench_warmup; k++) {
        ck(tsa_sweeps(ctx, order, betas[k % betas.size()], (uint32_t)k, lniters[k % betas.size()]));
        if (track) ck(tsa_track(ctx, k % (int)betas.size()));
        ck(tsa_energy(ctx, l.data(), s.data(), n.data()));
      }
      if (track) {  // the end of a tracked loop too (first use of its copies and of the second stream)
        std::vector<uint64_t> rec(lay.chain_words);
        std::vector<tsa_trace_row_t> rows(betas.size());
        int32_t bc = -1, bl = -1;
        double bs = 0, hz = 0;
        uint64_t tk = 0;
        ck(tsa_track_end(ctx, &bc, &bl, &bs, rec.data(), rows.data(), &tk, &hz));
      }
      double ms = 0;
      ck(tsa_sweeps_ms(ctx, &ms));
      ck(tsa_upload(ctx, pop.data()));
      ck(tsa_stats(ctx, stats0));
      ck(tsa_chunk_stats(ctx, chunks0));
    }
  }
  PinnedRecord best(lay.chain_words, 0);  // allocated (and its pages touched) before the clock starts
  const double t_init = now_s() - t_start;
  const double t0 = now_s();
  const int nc = O.nchains;
  std::vector<float> lc(nc);
  std::vector<int> sc(nc), ns(nc);
  std::vector<double> E(nc);  // energyE of every chain at the last evaluated level
  double best_score = INFINITY;
  int best_chain = -1;
  std::vector<int> family(nc), nfam(nc);
  std::iota(family.begin(), family.end(), 0);
  std::string trace;
  std::mt19937_64 hrng(splitmix64(O.seed + 777));
  float beta_last_resample = betas.empty() ? 0.f : betas[0];
  int nresample = 0;
  // independent chains in one energy mode: selection runs on the device, no host round trip per level
  const bool tracked = O.scheme == "indep" && O.betas2.empty() && !betas.empty() && !O.host_select;
  if (tracked) best_chain = run_levels_tracked(betas, lniters, sweep_ctr, best, trace, t0);
  for (size_t lev = 0; lev < (tracked ? 0 : betas.size()); lev++) {
    if (lmode[lev] != mode) {
      // stage switch: the stage-1 best stays the incumbent, scored in the new energy
      H1 = host_energy(I, lay.W, ML, best.data(), chCh(best.data()), leaf, chS(best.data()));
      staged = true;
      mode = lmode[lev];
      ck(tsa_set_mode(ctx, mode));
      best_score = score((float)std::log2(mode == 1 ? H1.time : H1.time2), H1.sc, H1.ns);
      beta_last_resample = betas[lev];
    }
    ck(tsa_sweeps(ctx, order, betas[lev], sweep_ctr, lniters[lev]));
    sweep_ctr += (uint32_t)lniters[lev];
    const bool last = lev + 1 == betas.size();
    const bool switching = !last && lmode[lev + 1] != mode;
    if ((int)(lev % O.eval_every) == O.eval_every - 1 || last || switching) {
      ck(tsa_energy(ctx, lc.data(), sc.data(), ns.data()));
      double ms = 0;
      ck(tsa_sweeps_ms(ctx, &ms));
      kernel_ms += ms;
      int bi = 0;
      double bs = INFINITY, meanE = 0, meanNs = 0;
      for (int c = 0; c < nc; c++) {
        const double s = score(lc[c], sc[c], ns[c]);
        if (s < bs) {
          bs = s;
          bi = c;
        }
        E[c] = energyE(lc[c], sc[c], ns[c]);  // the population step below reuses it
        meanE += E[c];
        meanNs += ns[c];
      }
      meanE /= nc;
      meanNs /= nc;
      if (bs < best_score) {
        best_score = bs;
        best_chain = bi;
        ck(tsa_download(ctx, bi, 1, best.data()));
      }
      std::fill(nfam.begin(), nfam.end(), 0);
      int nf = 0;
      for (int c = 0; c < nc; c++)
        if (nfam[family[c]]++ == 0) nf++;
      char buf[320];
      snprintf(buf, sizeof buf, "%s[%.4f,%zu,%.4f,%.6f,%d,%.6f,%d,%d,%d,%.3f]", trace.empty() ? "" : ",", now_s() - t0,
               lev, betas[lev], (double)lc[bi], sc[bi], meanE, nf, mode, ns[bi], meanNs);
      trace += buf;
      if (!O.quiet && (lev % 25 == 0 || last))
        fprintf(stderr, "lev %4zu beta %7.3f  best(l2cost/slice %.3f sc %d |S| %d)  meanE %.3f  mean|S| %.2f  families %d  t=%.2fs\n",
                lev, betas[lev], (double)lc[bi], sc[bi], ns[bi], meanE, meanNs, nf, now_s() - t0);
      if (!last && !switching && O.scheme == "pa") {
        // population annealing: systematic resampling with weights exp(-(beta_next - beta_prev) * E)
        const double db = betas[lev + 1] - beta_last_resample;
        beta_last_resample = betas[lev + 1];
        std::vector<double> w(nc);
        double Emin = INFINITY;
        for (int c = 0; c < nc; c++) Emin = std::min(Emin, E[c]);
        double wsum = 0;
        for (int c = 0; c < nc; c++) {
          w[c] = std::exp(-db * (E[c] - Emin));
          wsum += w[c];
        }
        std::vector<int> anc(nc);
        const double u = std::uniform_real_distribution<double>(0, 1)(hrng);
        double acc = 0;
        int j = 0;
        for (int c = 0; c < nc; c++) {
          acc += w[c] / wsum * nc;
          while (j < nc && j + u < acc) anc[j++] = c;
        }
        while (j < nc) anc[j++] = nc - 1;
        resample(anc, family);
        nresample++;
      } else if (!last && !switching && O.scheme == "trunc") {
        // truncation selection: the worst trunc_frac are replaced by copies of the best
        std::vector<int> idx(nc);
        std::iota(idx.begin(), idx.end(), 0);
        std::sort(idx.begin(), idx.end(), [&](int a, int b) { return E[a] < E[b]; });
        std::vector<int> anc(nc);
        std::iota(anc.begin(), anc.end(), 0);
        const int nrep = (int)(O.trunc_frac * nc);
        for (int k = 0; k < nrep; k++) anc[idx[nc - 1 - k]] = idx[k];
        resample(anc, family);
        nresample++;
      }
    } else {
      double ms = 0;
      ck(tsa_sweeps_ms(ctx, &ms));
      kernel_ms += ms;
    }
  }
  const double t_anneal = now_s() - t0;
  uint64_t stats[7], chunks[2];
  ck(tsa_stats(ctx, stats));
  for (int k = 0; k < 7; k++) stats[k] -= stats0[k];
  ck(tsa_chunk_stats(ctx, chunks));
  for (int k = 0; k < 2; k++) chunks[k] -= chunks0[k];

  // final best tree: verified from scratch; with slicing, sc > sc_target is repaired greedily
  const uint32_t* bch = chCh(best.data());
  std::vector<uint64_t> lab2((size_t)lay.nint * lay.W, 0);
  const bool valid = labels_from_topology(I, lay.W, bch, lab2.data());
  bool labels_ok = valid && std::equal(lab2.begin(), lab2.end(), best.begin());
  if (tracked && best_chain >= 0) {
    // device-side tracking returns the best tree only; the label sets the device maintains are checked on
    // that chain's final record instead, and the best record gets the sets of its own tree
    std::vector<uint64_t> live(lay.chain_words), lab3((size_t)lay.nint * lay.W, 0);
    ck(tsa_download(ctx, best_chain, 1, live.data()));
    labels_ok = valid && labels_from_topology(I, lay.W, chCh(live.data()), lab3.data()) &&
                std::equal(lab3.begin(), lab3.end(), live.begin());
    std::copy(lab2.begin(), lab2.end(), best.begin());
  }
  int n_repair = 0;
  if (O.slicing && valid) n_repair = greedy_repair(I, lay.W, lab2.data(), leaf, best.data() + lay.s_off, O.sc_target);
  const HostEnergy HE = host_energy(I, lay.W, ML, lab2.data(), bch, leaf, chS(best.data()));
  const double ks = kernel_ms / 1e3;
  if (!O.quiet)
    fprintf(stderr,
            "done: best tc %.4f sc %d |S| %d (repair +%d) time %.4e s time2 %.4e s (per slice) | anneal %.2fs init %.2fs "
            "kernel %.2fs | %.3e proposals/s | %.3e node visits/s | slice moves %llu/%llu accepted\n",
            HE.tc, HE.sc, HE.ns, n_repair, HE.time, HE.time2, t_anneal, t_init, ks, ks > 0 ? stats[0] / ks : 0.0,
            ks > 0 ? (double)sweep_ctr * nc * (I.m - 1) / ks : 0.0, (unsigned long long)stats[5],
            (unsigned long long)stats[4]);
  FILE* f = O.out.empty() ? stdout : fopen(O.out.c_str(), "w");
  if (!f) die("cannot open " + O.out);
  char desc[256] = {0};
  tsa_describe(ctx, desc, sizeof desc);
  // summary words per label set in the reference's 32-bit count (one bit per 16-byte chunk)
  const char* sp = strstr(desc, " sums=");
  const int nsum = (sp && atoi(sp + 6) > 0) ? (lay.W / 2 + 31) / 32 : 0;
  fprintf(f, "{\"tc\": %.6f, \"sc\": %d, \"gpu_time\": %s, \"h100_time\": %s, \"valid\": %s, \"labels_ok\": %s, \"best_chain\": %d,\n",
          HE.tc, HE.sc, jnum(HE.time).c_str(), jnum(HE.time2).c_str(), valid ? "true" : "false",
          labels_ok ? "true" : "false", best_chain);
  fprintf(f, " \"slicing\": %s, \"nsliced\": %d, \"n_repair\": %d, \"tc_total\": %.6f, \"gpu_time_total\": %s, \"h100_time_total\": %s, \"sliced\": [",
          O.slicing ? "true" : "false", HE.ns, n_repair, HE.tc + HE.ns, jnum(HE.time * std::exp2((double)HE.ns)).c_str(),
          jnum(HE.time2 * std::exp2((double)HE.ns)).c_str());
  {
    int k = 0;
    const uint64_t* S = best.data() + lay.s_off;
    for (int l = 0; l < I.nlab; l++)
      if (O.slicing && (S[l >> 6] >> (l & 63) & 1u)) fprintf(f, "%s%d", k++ ? "," : "", l);
  }
  fprintf(f, "],\n \"t_anneal\": %.6f, \"t_init\": %.6f, \"kernel_s\": %.6f, \"proposals\": %llu, \"accepts\": %llu, \"warp_steps\": %llu, \"node_visits\": %llu, \"slice_proposals\": %llu, \"slice_accepts\": %llu, \"busy_lanes\": %llu, \"coop_max\": %d, \"coop_min\": %d, \"coop_full\": %d, \"par_follow\": %d, \"par_band\": %d, \"nsum\": %d, \"wpc\": %d, \"order\": \"%s\",\n",
          t_anneal, t_init, ks, (unsigned long long)stats[0], (unsigned long long)stats[1], (unsigned long long)stats[2],
          (unsigned long long)stats[3], (unsigned long long)stats[4], (unsigned long long)stats[5],
          (unsigned long long)stats[6], 1, 1, 1, O.par_follow, O.par_band, nsum, 1,
          order == TSA_ORDER_PAR ? "par" : "preorder");
  fprintf(f, " \"nchains\": %d, \"niters\": %d, \"nlevels\": %zu, \"total_sweeps\": %u, \"W\": %d, \"nw\": %d, \"word_bits\": 64, \"lpc\": 64, \"kernel\": \"%s\", \"hip_kernel\": \"%s\", \"scheme\": \"%s\", \"mode\": %d, \"nresample\": %d,\n",
          nc, O.niters, betas.size(), sweep_ctr, lay.runtime_width ? 0 : lay.W, lay.W, kernel_name().c_str(), desc,
          O.scheme.c_str(), O.mode, nresample);
  fprintf(f, " \"sum_chunks\": %llu, \"sum_xchunks\": %llu,\n", (unsigned long long)chunks[0],
          (unsigned long long)chunks[1]);
  if (!init_tcs.empty()) {
    fprintf(f, " \"init\": \"%s\", \"t_start_trees\": %.6f, \"init_tcs\": [", O.init.c_str(), t_trees);
    for (size_t i = 0; i < init_tcs.size(); i++) fprintf(f, "%s%.4f", i ? ", " : "", init_tcs[i]);
    fprintf(f, "],\n");
  }
  if (staged)
    fprintf(f, " \"stage1_tc\": %.6f, \"stage1_sc\": %d, \"stage1_nsliced\": %d, \"stage1_gpu_time\": %s, \"stage1_h100_time\": %s, \"stage1_h100_time_total\": %s,\n",
            H1.tc, H1.sc, H1.ns, jnum(H1.time).c_str(), jnum(H1.time2).c_str(),
            jnum(H1.time2 * std::exp2((double)H1.ns)).c_str());
  fprintf(f, " \"trace_cols\": [\"t\", \"level\", \"beta\", \"best_lcost_per_slice\", \"best_sc\", \"mean_E\", \"families\", \"mode\", \"best_nsliced\", \"mean_nsliced\"],\n");
  fprintf(f, " \"trace\": [%s],\n \"tree\": [", trace.c_str());
  for (int i = 0; i < lay.nint; i++) fprintf(f, "%s[%u,%u]", i ? "," : "", bch[i] & 0xFFFFu, bch[i] >> 16);
  fprintf(f, "]}\n");
  if (f != stdout) fclose(f);
  return valid && labels_ok ? 0 : 2;
}

// Validation on the device (csrc/treesa_gpu.cu:1940-2061): [1] every chain is a valid tree whose labels
// equal the topology's, [2] the energy kernel agrees with the host double computation, [3] the other
// kernel mapping (chain in LDS vs in HBM) is bit-identical.  The CPU-reference comparison [4] needs the
// oracle, which this binary does not link; the test suite runs it through the C ABI.
int Runner::run_check() {
  std::vector<float> betas = parse_betas(O.betas);
  if (O.max_levels > 0 && (int)betas.size() > O.max_levels) betas.resize(O.max_levels);
  const std::vector<uint64_t> init = init_population();
  create(&ctx, cfg.kernel);
  ck(tsa_upload(ctx, init.data()));
  for (size_t lev = 0; lev < betas.size(); lev++)
    ck(tsa_sweeps(ctx, order, betas[lev], (uint32_t)(lev * O.niters), O.niters));
  std::vector<uint64_t> fin(init.size());
  ck(tsa_download(ctx, 0, O.nchains, fin.data()));
  uint64_t stats[7];
  ck(tsa_stats(ctx, stats));
  char desc[256] = {0};
  tsa_describe(ctx, desc, sizeof desc);
  printf("check: %d chains, %zu levels x %d sweeps, kernel %s (%s), mode %d, W=%d (64-bit words), slicing %d (moves %d): "
         "%llu proposals, %llu accepted, %llu/%llu slice moves accepted\n",
         O.nchains, betas.size(), O.niters, kernel_name().c_str(), desc, O.mode, lay.W, cfg.slicing, cfg.slice_moves,
         (unsigned long long)stats[0], (unsigned long long)stats[1], (unsigned long long)stats[5],
         (unsigned long long)stats[4]);
  int bad_tree = 0, bad_lab = 0, changed = 0, Schanged = 0;
  std::vector<uint64_t> lab2((size_t)lay.nint * lay.W);
  for (int c = 0; c < O.nchains; c++) {
    const uint64_t* base = &fin[(size_t)c * lay.chain_words];
    const uint64_t* b0 = &init[(size_t)c * lay.chain_words];
    if (!labels_from_topology(I, lay.W, chCh(base), lab2.data())) {
      bad_tree++;
      continue;
    }
    if (!std::equal(lab2.begin(), lab2.end(), base)) bad_lab++;
    if (!std::equal(base, base + lay.s_off, b0)) changed++;
    if (!std::equal(base + lay.s_off, base + lay.s_off + lay.W, b0 + lay.s_off)) Schanged++;
  }
  printf("  [1] invalid trees: %d, chains with label mismatch vs recomputation: %d (chains changed by SA: %d/%d, "
         "slice set changed: %d)\n",
         bad_tree, bad_lab, changed, O.nchains, Schanged);
  std::vector<float> lc(O.nchains);
  std::vector<int> sc(O.nchains), ns(O.nchains);
  ck(tsa_energy(ctx, lc.data(), sc.data(), ns.data()));
  double maxd = 0;
  int scbad = 0;
  for (int c = 0; c < O.nchains; c++) {
    const uint64_t* base = &fin[(size_t)c * lay.chain_words];
    const HostEnergy HE = host_energy(I, lay.W, ML, base, chCh(base), leaf, chS(base));
    const double ref = O.mode == 0 ? HE.tc : std::log2(O.mode == 1 ? HE.time : HE.time2);
    maxd = std::max(maxd, std::fabs(ref - (double)lc[c]));
    if (HE.sc != sc[c] || HE.ns != ns[c]) scbad++;
  }
  printf("  [2] GPU energy kernel vs host double: max |dlog2cost| = %.3g, sc/|S| mismatches %d\n", maxd, scbad);
  int xdiff = -1;
  const bool is_lds = strncmp(desc, "lds", 3) == 0, is_wide = strncmp(desc, "wide", 4) == 0;
  if (O.cross && cfg.slice_moves == 0 && (is_lds || (is_wide && order == TSA_ORDER_PAR))) {
    tsa_ctx* c2 = nullptr;
    create(&c2, TSA_KERNEL_GLOBAL);
    ck(tsa_upload(c2, init.data()));
    for (size_t lev = 0; lev < betas.size(); lev++)
      ck(tsa_sweeps(c2, order, betas[lev], (uint32_t)(lev * O.niters), O.niters));
    std::vector<uint64_t> fin2(fin.size());
    ck(tsa_download(c2, 0, O.nchains, fin2.data()));
    tsa_destroy(c2);
    xdiff = 0;
    for (int c = 0; c < O.nchains; c++)
      if (!std::equal(fin.begin() + (size_t)c * lay.chain_words, fin.begin() + (size_t)(c + 1) * lay.chain_words,
                      fin2.begin() + (size_t)c * lay.chain_words))
        xdiff++;
    printf("  [3] kernel %s vs global: chains differing: %d/%d\n", is_lds ? "lds" : "wide", xdiff, O.nchains);
  }
  printf("  [4] CPU reference: not linked into this binary\n");
  const bool ok = bad_tree == 0 && bad_lab == 0 && scbad == 0 && maxd < 1e-3 && xdiff <= 0;
  printf("CHECK %s\n", ok ? "PASSED" : "FAILED");
  return ok ? 0 : 3;
}

}  // namespace

int main(int argc, char** argv) {
  const Opts O = parse(argc, argv);
  try {
    const Inst I = read_instance(O.inst);
    if (I.m < 3) die("need at least 3 tensors");
    if (2 * I.m - 1 > 65535) die("too many tensors (node ids are 16-bit)");
    Runner R(I, O);
    return O.check ? R.run_check() : R.run_anneal();
  } catch (const InputError& e) {
    die(e.what());
  }
}
