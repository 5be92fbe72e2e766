// tsa_cli.cpp -- the command line of bin/treesa_gpu as one table: each entry names a flag, its value (if any),
// a line of help and how it sets Options; parsing, validation of numbers and the usage text all come from it.
#include "tsa_cli.h"

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <vector>

namespace tsa {

namespace {

using Setter = std::function<void(Options&, const std::string&)>;

struct Flag {
  const char* name;
  const char* value;  // placeholder of the value, nullptr for a switch
  const char* help;
  Setter set;
};

long to_long(const std::string& s) {
  char* e = nullptr;
  errno = 0;
  const long v = strtol(s.c_str(), &e, 10);
  if (s.empty() || *e != 0 || errno != 0) throw UsageError("not an integer: " + s);
  return v;
}
int to_int(const std::string& s) {
  const long v = to_long(s);
  if (v < -2147483647L || v > 2147483647L) throw UsageError("out of range: " + s);
  return (int)v;
}
double to_real(const std::string& s) {
  char* e = nullptr;
  const double v = strtod(s.c_str(), &e);
  if (s.empty() || *e != 0) throw UsageError("not a number: " + s);
  return v;
}
uint64_t to_u64(const std::string& s) {
  char* e = nullptr;
  errno = 0;
  const unsigned long long v = strtoull(s.c_str(), &e, 10);
  if (s.empty() || *e != 0 || errno != 0) throw UsageError("not an unsigned integer: " + s);
  return (uint64_t)v;
}
// n comma-separated numbers into out
void to_reals(const std::string& s, double* out, int n) {
  size_t p = 0;
  for (int k = 0; k < n; k++) {
    const size_t q = k + 1 < n ? s.find(',', p) : s.size();
    if (q == std::string::npos) throw UsageError("expected " + std::to_string(n) + " comma-separated values: " + s);
    out[k] = to_real(s.substr(p, q - p));
    p = q + 1;
  }
}
// energy modes: "gpu" -> 1, "h100" (old name "gpu2") -> 2, anything else tc (csrc/treesa_gpu.cu:1358)
int mode_of(const std::string& s) { return s == "gpu" ? 1 : (s == "h100" || s == "gpu2") ? 2 : 0; }

#define INT_FIELD(f) [](Options& o, const std::string& v) { o.f = to_int(v); }
#define REAL_FIELD(f) [](Options& o, const std::string& v) { o.f = to_real(v); }
#define TEXT_FIELD(f) [](Options& o, const std::string& v) { o.f = v; }
#define SWITCH(f, x) [](Options& o, const std::string&) { o.f = x; }

const std::vector<Flag>& flags() {
  static const std::vector<Flag> table = {
      {"-i", "FILE", "instance file: m nlab / m tensors 'k l1..lk' / 'ny y1..yny'", TEXT_FIELD(instance)},
      {"--tree", "FILE", "start trees: K trees of m-1 'left right' lines, chain c from tree c % K", TEXT_FIELD(tree_file)},
      {"--init", "tree|spectral|greedy", "start trees without --tree (tree: random trees per chain)",
       [](Options& o, const std::string& v) {
         if (v != "tree" && v != "spectral" && v != "greedy") throw UsageError("--init tree|spectral|greedy");
         o.init = v;
       }},
      {"--spectral-k", "K", "--init spectral: the K best spectral path trees", INT_FIELD(spectral_k)},
      {"--greedy-repeat", "R", "--init greedy: the best of R greedy runs", INT_FIELD(greedy_repeat)},
      {"--out", "FILE", "JSON result (default: stdout)", TEXT_FIELD(out_file)},
      {"--nchains", "N", "chains (default 1024)", INT_FIELD(nchains)},
      {"--niters", "K", "sweeps per level (default 50)", INT_FIELD(niters)},
      {"--betas", "SPEC", "levels: a:step:b | file:PATH | b1,b2,.. (default 0.01:0.05:15)", TEXT_FIELD(betas)},
      {"--max-levels", "L", "use only the first L levels", INT_FIELD(max_levels)},
      {"--stage2-betas", "SPEC", "stage 2: continue the population on these levels in --stage2-mode",
       TEXT_FIELD(stage2_betas)},
      {"--stage2-niters", "K", "sweeps per stage-2 level (default --niters)", INT_FIELD(stage2_niters)},
      {"--stage2-mode", "gpu|h100", "energy of stage 2 (default gpu)",
       [](Options& o, const std::string& v) { o.stage2_mode = (v == "h100" || v == "gpu2") ? 2 : 1; }},
      {"--mode", "tc|gpu|h100", "energy: tc + sc penalty, or a modeled time", [](Options& o, const std::string& v) {
         o.mode = mode_of(v);
       }},
      {"--gm", "peak,bw,m0,n0,k0,launch", "GPU roofline model constants",
       [](Options& o, const std::string& v) { to_reals(v, o.model.gm, 6); }},
      {"--h100-model", "launch,perm_bw,cc_bit,cc_cell,tc_bit,tc_pad,tc_out,small_rank,small_cell",
       "measured H100 model constants", [](Options& o, const std::string& v) { to_reals(v, o.model.h100, 9); }},
      {"--gm2", "(9 values)", "old name of --h100-model", [](Options& o, const std::string& v) {
         to_reals(v, o.model.h100, 9);
       }},
      {"--sc-target", "x", "space-complexity target (default 20)", REAL_FIELD(sc_target)},
      {"--sc-weight", "y", "weight of the sc excess (default 1)", REAL_FIELD(sc_weight)},
      {"--scheme", "indep|pa|trunc", "population scheme (default indep)", TEXT_FIELD(scheme)},
      {"--trunc-frac", "f", "trunc: fraction of chains replaced per level (default 0.25)", REAL_FIELD(trunc_frac)},
      {"--seed", "s", "random seed (default 1)", [](Options& o, const std::string& v) { o.seed = to_u64(v); }},
      {"--eval-every", "k", "evaluate (select, resample) every k-th level (default 1)", INT_FIELD(eval_every)},
      {"--select-sc", nullptr, "report the lowest sc excess first, then tc", SWITCH(select_sc, true)},
      {"--slicing", nullptr, "anneal a slice set together with the tree", SWITCH(slicing, true)},
      {"--slice-moves", "k", "slice proposals per slice step (default 1)", INT_FIELD(slice_moves)},
      {"--slice-every", "s", "a slice step after every s-th sweep (default 1)", INT_FIELD(slice_every)},
      {"--max-slices", "n", "cap on the number of sliced labels", INT_FIELD(max_slices)},
      {"--init-slices", "l1,l2,..", "labels sliced in every chain at the start (implies --slicing)",
       [](Options& o, const std::string& v) {
         o.init_slices = v;
         o.slicing = true;
       }},
      {"--order", "par|preorder", "sweep order (default par)", TEXT_FIELD(order)},
      {"--kernel", "auto|par|seq|seqsm|warp|warpsm|block", "kernel family (other than auto / par: pre-order)",
       TEXT_FIELD(kernel)},
      {"--par-follow", nullptr, "par: an accepted move re-visits its pivot", SWITCH(par_follow, 1)},
      {"--par-band", "L", "par: priorities top-down within bands of L levels (2..16)", INT_FIELD(par_band)},
      {"--wide", nullptr, "runtime-width label sets whatever the label count", SWITCH(wide, true)},
      {"--sums", nullptr, "chunk summaries on", SWITCH(force_sum, true)},
      {"--no-sum", nullptr, "chunk summaries off", SWITCH(no_sum, true)},
      {"--wpc", "n", "wide kernel: 32-lane warps per workgroup (waves = n / 2)", INT_FIELD(wpc)},
      {"--wide-wgs", "K", "wide kernel: workgroups per chain", INT_FIELD(wide_wgs)},
      {"--wide-lanes", "G", "wide kernel: lanes per proposal", INT_FIELD(wide_lanes)},
      {"--draw-waves", "1|-1|0",
       "pre-order: helper waves draw the next sweep's random numbers (1), each visit draws its own (-1), automatic (0)",
       INT_FIELD(draw_waves)},
      {"--lpc", "32|16|8", "lanes per chain of the reference's warp kernels (not 32: pre-order)", INT_FIELD(lpc)},
      {"--wpb", "W", "accepted, no effect here", INT_FIELD(wpb)},
      {"--block", "B", "accepted, no effect here", INT_FIELD(block)},
      {"--coop-max", "G", "accepted, no effect here", INT_FIELD(coop_max)},
      {"--coop-min", "G0", "accepted, no effect here", INT_FIELD(coop_min)},
      {"--coop-full", "G1", "accepted, no effect here", INT_FIELD(coop_full)},
      {"--coop-min-units", "u", "accepted, no effect here", INT_FIELD(coop_min_units)},
      {"--coop-chunks", "c", "accepted, no effect here",
       [](Options& o, const std::string& v) { o.coop_chunks = std::max(1, to_int(v)); }},
      {"--check", nullptr, "validate the kernels instead of annealing", SWITCH(check, true)},
      {"--ref-chains", "R", "--check: chains of the CPU comparison (run by the test suite here)",
       INT_FIELD(ref_chains)},
      {"--random-slices", "k", "--check: a fixed random slice set of k labels per chain (implies --slicing)",
       [](Options& o, const std::string& v) {
         o.random_slices = to_int(v);
         o.slicing = true;
       }},
      {"--no-cross", nullptr, "--check: skip the comparison with the other kernel mapping", SWITCH(cross, false)},
      {"--quiet", nullptr, "no progress on stderr", SWITCH(quiet, true)},
      {"--bench-warmup", "W", "W untimed levels first, then the start population again", INT_FIELD(bench_warmup)},
      {"--dump-population", "FILE",
       "after the level loop (outside its timing), every chain's record as raw little-endian 64-bit words",
       TEXT_FIELD(dump_population)},
      {"--host-select", nullptr, "select on the host at every level, also for --scheme indep",
       SWITCH(host_select, true)},
      {"--no-overlap", nullptr, "device-side selection on the sweep's stream", SWITCH(no_overlap, true)},
      {"--level-launches", nullptr, "scheme indep: one sweep launch and one selection per level, not the level loop "
       "in one launch", SWITCH(level_launches, true)},
      {"--level-loop", nullptr, "scheme indep: the level loop in one launch also with more chains than are resident "
       "at once", SWITCH(level_loop, true)},
      {"--level-blocks", "K", "scheme indep, par order, more than twice the chains the device holds at once: levels "
       "per sweep launch (0: automatic, 1: one)", INT_FIELD(level_blocks)},
      {"--level-log", "FILE", "one JSON line per evaluated level: best chain, score, energies, ancestors",
       TEXT_FIELD(level_log)},
  };
  return table;
}

}  // namespace

Options parse_options(int argc, char** argv) {
  Options o;
  for (int i = 1; i < argc; i++) {
    const std::string a = argv[i];
    const Flag* f = nullptr;
    for (const Flag& x : flags())
      if (a == x.name) f = &x;
    if (!f) throw UsageError("unknown flag " + a);
    std::string v;
    if (f->value) {
      if (i + 1 >= argc) throw UsageError(a + " needs a value");
      v = argv[++i];
    }
    f->set(o, v);
  }
  if (o.instance.empty()) throw UsageError("no instance (-i FILE)");
  return o;
}

std::string usage_text() {
  std::string s = "usage: treesa_gpu -i instance.txt [flags]\n";
  for (const Flag& f : flags()) {
    std::string left = std::string("  ") + f.name + (f.value ? std::string(" ") + f.value : "");
    if (left.size() < 34) left.resize(34, ' ');
    else left += "\n" + std::string(34, ' ');
    s += left + f.help + "\n";
  }
  return s;
}

}  // namespace tsa
