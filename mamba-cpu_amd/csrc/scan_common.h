// Selective-scan kernel parameters and the shared lane layout.
//
// Lane layout (forward and backward): a workgroup is 4 waves; each wave holds
// 4 channels (rows r = lane / 16) x 16 state lanes (j = lane % 16); lane j owns
// states n = j + 16 * s for s < SPL (SPL = ceil(dstate / 16)). Time is walked
// in blocks of 16 steps; within a block lane j also "owns" step t0 + j for the
// per-step scalar work (loading u/delta/z/dout, softplus, gating, stores), and
// the other lanes of its row read those scalars through DPP row broadcasts.
// A workgroup covers 16 consecutive channels of one (batch, group) slice, so
// all its rows share the same B/C rows.
#pragma once

#include "mcpu_common.h"

namespace mcpu {

constexpr int kScanBlockT = 16;       // time steps per block
constexpr int kScanRowsPerWave = 4;   // channels per wave
constexpr int kScanWaves = 4;         // waves per workgroup
constexpr int kScanChannelsPerWG = kScanRowsPerWave * kScanWaves;
constexpr int kScanThreads = 64 * kScanWaves;

struct ScanParams {
  const void* u;
  const void* delta;
  const float* A;
  const float* B;
  const float* C;
  const float* D;
  const void* z;
  const float* delta_bias;
  void* out;
  float* last_state;
  float* ckpt;          // (batch, dim, nblk, dstate): state at the start of each block
  const void* dout;
  const float* dlast_state;
  void* du;
  void* ddelta;
  void* dz;
  float* dA_part;       // (batch, dim, dstate)
  float* dB_part;       // (batch, ngroups, nblk_c, seqlen, dstate)
  float* dC_part;
  float* dD_part;       // (batch, dim)
  float* dbias_part;    // (batch, dim)
  int64_t batch, dim, seqlen, dstate, ngroups, dpg;
  int64_t nblk;         // ceil(seqlen / 16)
  int64_t nblk_c;       // ceil(dpg / 16)
  int64_t su[3], sdl[3], sz[3], sB[3], sC[3], sdo[3];
  int softplus;
};

struct RowCtx {
  int64_t b, g, d;     // batch, group, channel (clamped into range)
  bool active;         // channel exists (rows past the slice end are padding)
};

__device__ __forceinline__ RowCtx scan_row_ctx(const ScanParams& p, int wave, int r) {
  int64_t bid = blockIdx.x;
  const int64_t cblk = bid % p.nblk_c;
  bid /= p.nblk_c;
  RowCtx c;
  c.g = bid % p.ngroups;
  c.b = bid / p.ngroups;
  const int64_t cl = cblk * kScanChannelsPerWG + wave * kScanRowsPerWave + r;
  c.active = cl < p.dpg;
  c.d = c.g * p.dpg + (c.active ? cl : p.dpg - 1);
  return c;
}

}  // namespace mcpu
