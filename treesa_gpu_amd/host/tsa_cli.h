// tsa_cli.h -- command line of bin/treesa_gpu: every flag of the reference binary (csrc/treesa_gpu.cu:1330-1406,
// as treesa_gpu/driver.py:252-296 builds them), with its defaults, plus this build's own diagnostics.
#pragma once
#include <cstdint>
#include <stdexcept>
#include <string>

#include "tsa_host.h"

namespace tsa {

// A malformed command line; the binary prints the usage text and exits 1.
struct UsageError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

struct Options {
  // inputs and outputs
  std::string instance, tree_file, out_file;
  std::string init = "tree";  // start trees without --tree: tree (random trees), spectral, greedy
  int spectral_k = 4, greedy_repeat = 10;
  // schedule
  std::string betas = "0.01:0.05:15", stage2_betas;
  int nchains = 1024, niters = 50, stage2_niters = -1, max_levels = -1, eval_every = 1;
  int mode = 0, stage2_mode = 1;  // 0 tc, 1 gpu, 2 h100
  ModelConsts model;
  // energy, selection and population
  double sc_target = 20.0, sc_weight = 1.0, trunc_frac = 0.25;
  std::string scheme = "indep";
  uint64_t seed = 1;
  bool select_sc = false;
  // slicing
  bool slicing = false;
  int slice_moves = 1, slice_every = 1, max_slices = 0, random_slices = 0;
  std::string init_slices;
  // sweep order and kernel choice (results never depend on the kernel flags)
  std::string order = "par", kernel = "auto";
  int par_follow = 0, par_band = 0;
  bool wide = false, no_sum = false, force_sum = false;
  int wpc = 0, wide_wgs = 0, wide_lanes = 0;
  int draw_waves = 0;  // pre-order: 1 helper waves draw the next sweep's random numbers, -1 each visit, 0 automatic
  int lpc = 32, wpb = 0, block = 0, coop_max = 0, coop_min_units = -1, coop_min = 1, coop_full = 0, coop_chunks = 2;
  // validation mode
  bool check = false, cross = true;
  int ref_chains = 8;
  // diagnostics of this build
  bool quiet = false, host_select = false, no_overlap = false, level_launches = false, level_loop = false;
  int bench_warmup = 0;
  int level_blocks = 0;  // tsa_config_t.level_blocks
  std::string level_log, dump_population;
};

// Parses argv; throws UsageError on an unknown flag, a missing or malformed value, or no -i.
Options parse_options(int argc, char** argv);

// The usage text, generated from the flag table.
std::string usage_text();

}  // namespace tsa
