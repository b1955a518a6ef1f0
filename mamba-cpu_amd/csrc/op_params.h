// Kernel parameter blocks for the conv1d and state-update kernels, shared by
// the kernels and the C-ABI layer that fills them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mcpu {

constexpr int kConvT = 8;      // conv steps per chunk
constexpr int kConvMaxW = 16;  // widest conv of the register-window kernels
constexpr int64_t kConvWideMaxW = 1 << 16;  // widest conv (the per-element kernels above kConvMaxW)
constexpr int kConvWideSeg = 256;  // steps per dweight partial of the per-element backward
constexpr int kConvRMax = 16;  // most threads walking one (batch, channel) row
constexpr int kConvVTSteps = 8;  // steps per thread of the time-contiguous fast path
constexpr int kConvClG = 8;      // unrolled steps per group of the channel-contiguous fast path

struct ConvParams {
  const void* x;
  const float* w;
  const float* bias;
  const void* init;
  void* out;
  void* final_states;
  const void* dout;
  const void* dfinal;
  void* dx;
  void* dinit;
  float* dw_part;   // (batch, R, dim, W + 1): per-thread partial dw and dbias
  float* dpre;      // widths above kConvMaxW: (batch, dim, seqlen) float32 dout * act'(pre)
  int64_t batch, dim, seqlen, width;
  int64_t nchunks, R;
  int64_t sx[3], sinit[3], sout[3], sdo[3], sdx[3];
  int silu;
  const int32_t* seq_idx;  // (batch, seqlen) packed-sequence ids, or null
  int channels_last;  // thread index decomposed channel-fastest
  // Time-contiguous fast path (conv_*_vt_kernel): vt = steps per thread (8 or
  // 16), 0 when the path does not apply.
  int vt;
  int tpr;            // threads per row segment: 64, 128 or 256
  int rpw;            // row segments per workgroup: 256 / tpr
  int64_t nseg;       // segments per row (rows longer than 2048 steps)
  // Channel-contiguous fast path (conv_*_cl_kernel): cl = 1 when it applies;
  // a wave's time segment is cl_ng groups of kConvClG steps; cl_gy segment
  // groups of four per row (the grid's y).
  int cl, cl_ng;
  int64_t cl_gy;
};

struct ConvUpdateParams {
  const void* x;
  void* state;
  const float* w;
  const float* bias;
  void* out;
  int64_t batch, dim, seqlen, width, state_len;
  int64_t sx[3], sst[3], sout[3];
  int silu;
  const int32_t* cache_seqlens;  // ring-buffer write positions, or null
  const int32_t* state_idx;      // conv_state row per batch row, or null
  int64_t state_batch;           // rows of conv_state
};

struct StateUpdateParams {
  void* state;
  const void* x;
  const void* dt;
  const float* A;
  const float* B;
  const float* C;
  const float* D;
  const void* z;
  const float* dt_bias;
  void* out;
  int64_t batch, nheads, headdim, dstate, ngroups;
  int64_t sst[3], sx[3], sdt[3], sz[3], sB[2], sC[2];
  int64_t sA[3], sD[2], sbias[2];  // A over (head, headdim, dstate); D, dt_bias over (head, headdim)
  int softplus;
  const int32_t* state_idx;  // state row per batch row, or null
  int64_t state_batch;       // rows of state
};

hipError_t conv_fwd_launch(const ConvParams& p, int dtype, hipStream_t st);
hipError_t conv_bwd_launch(const ConvParams& p, int dtype, float* dweight, float* dbias,
                           hipStream_t st);
hipError_t conv_update_launch(const ConvUpdateParams& p, int dtype, hipStream_t st);
hipError_t state_update_launch(const StateUpdateParams& p, int dtype, int state_dtype,
                               hipStream_t st);

}  // namespace mcpu
