// Launch planning shared by the fused kernels: per-n tile shapes, thread
// counts, occupancy (cached) and tuning overrides.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>

#include "mhc_host.hpp"

namespace mhc {

// Forward tile: V consecutive channels per chunk, up to CH chunks per thread
// held in registers.  NMAX is n rounded up to {4, 8, 16, 32, 64}.
template <int NMAX>
struct FwdCfg {
  // n = 16 takes 2-channel chunks: with 4 the 16 streams' x (64 fp32 values) and the per-stream
  // branches of a runtime n spilled at the 1024-thread bound (128 VGPRs)
  static constexpr int V = NMAX <= 8 ? 8 : 32 / NMAX;
  static constexpr int CH = NMAX <= 4 ? 2 : 1;
};

// Register-tiled kernels exist for NMAX in {4, 8, 16}; 0 selects the
// runtime-n kernels of generic.hip (16 < n <= 64).
inline int nmax_for(int n) { return n <= 4 ? 4 : (n <= 8 ? 8 : (n <= 16 ? 16 : 0)); }
inline int fwd_vec_width(int nmax) { return nmax <= 8 ? 8 : 64 / nmax; }
inline int bwd_vec_width(int nmax) { return nmax <= 4 ? 8 : (nmax == 8 ? 4 : (nmax == 16 ? 2 : 1)); }

inline int dtype_bytes(int code) {
  switch (code) {
    case MHC_DTYPE_F32: return 4;
    case MHC_DTYPE_BF16: return 2;
    case MHC_DTYPE_F16: return 2;
    default: return 0;
  }
}

struct ThreadPlan {
  int tpb;     // threads per block
  int ch;      // chunks per thread held in registers
  int reload;  // 1: tile does not fit, two passes over the inputs
};

// Smallest block (multiple of 64, <= max_tpb) holding nchunks with at most
// `chmax` chunks per thread; `tpb_pref` > 0 forces the block size (capped at
// max_tpb).  Above max_tpb * chmax chunks the kernel reloads (reload = 1).
inline ThreadPlan plan_threads(int nchunks, int chmax, int tpb_pref, int max_tpb) {
  ThreadPlan p{};
  if (tpb_pref > 0) {
    p.tpb = std::min(max_tpb, std::max(64, round_up(tpb_pref, 64)));
    p.ch = (int)ceil_div(nchunks, p.tpb);
    p.reload = p.ch > chmax ? 1 : 0;
    if (p.reload) p.ch = 0;
    return p;
  }
  int tpb = round_up((int)ceil_div(nchunks, chmax), 64);
  if (tpb <= max_tpb) {
    p.tpb = std::max(64, tpb);
    p.ch = (int)ceil_div(nchunks, p.tpb);
    p.reload = 0;
  } else {
    p.tpb = max_tpb;
    p.ch = 0;
    p.reload = 1;
  }
  return p;
}

// Resident blocks per CU for a kernel at a block size (cached).
int occupancy_blocks(const void* kernel, int tpb, size_t smem);

// Launch-shape tuning knobs (names in capi.hip; set through mhc_set_knob,
// initialised from the environment once at load).
enum Knob : int {
  kKnobFwdMfma, kKnobFwdSpw, kKnobFwdCh, kKnobFwdTpb, kKnobFwdGrid, kKnobFwdSkf,
  kKnobBwdGrid, kKnobBwdMfma, kKnobBwdSpw, kKnobBwdLegacy, kKnobBwdTpb,
  kKnobSk16, kKnobSk16Cpl, kKnobSk16Record,
  kKnobResGrid, kKnobMixFwdGrid, kKnobMixBwdGrid, kKnobScaleFwdGrid, kKnobScaleBwdGrid,
  kKnobBwdPipe, kKnobMix32, kKnobMf32Waves, kKnobSkBlkRecord, kKnobFwdLoop, kKnobMf32FwdWaves,
  kKnobFwdPipe, kKnobScaleFwdFlat, kKnobScaleBwdFlat, kKnobGenMfma, kKnobSkWg,
  kNumKnobs
};

// The knob's value, or `dflt` when it is unset.
int knob(Knob k, int dflt);

// Upper bound on a one-dimensional grid; larger token counts are covered by
// the kernels' grid-stride loops.
constexpr int64_t kMaxGrid = 1 << 24;

}  // namespace mhc
