// Kernel parameters of the Mamba-2 SSD scan (csrc/ssd.hip) and its launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mcpu {

constexpr int kSsdQ = 64;         // steps per chunk
constexpr int kSsdMaxP = 64;      // largest headdim
constexpr int kSsdMaxN = 128;     // largest dstate
constexpr int kSsdSlice = 256;    // state elements per workgroup of the chunk-passing kernels
constexpr int kSsdMaxHeadBlock = 8;  // heads one workgroup of the chunk kernels walks through
constexpr int kSsdPassCols = 64;  // state columns per workgroup of the in-order passing kernels
constexpr int kSsdCUs = 256;      // compute units of an MI355X (workgroups of the chunk kernels per round)

// Layouts (all contiguous): x, z, out, ysave, dx, dz (batch, seqlen, nheads,
// headdim) in the storage type; dt, ddt (batch, seqlen, nheads) float32;
// B, C (batch, seqlen, ngroups, dstate) in the storage type; states
// (batch, nheads, headdim, dstate) float32; heads split into ngroups
// contiguous groups sharing B and C. The chunk kernels give each workgroup
// one chunk of `hb` consecutive heads of one group (head block; nhb = nheads
// / hb of them), so B, C and C B^T are staged and formed once per block.
struct SsdParams {
  const void* x;
  const float* dt;
  const float* A;
  const void* B;
  const void* C;
  const float* D;           // (nheads, headdim) or null
  const void* z;
  const float* dt_bias;
  const float* init;
  const int32_t* seq_idx;   // (batch, seqlen) packed-sequence ids, or null
  void* out;
  float* final_states;
  void* ysave;              // y before the z gate, written when the backward will need it
  // Saved by the forward for the backward.
  float* cs;                // (batch, nheads, nchunks, Q): running sum of dt*A within the chunk,
  float* cs_lo;             // as a float pair cs + cs_lo (the rounding error of the float sum),
                            // so that differences cs_t - cs_s keep their own precision
  float* step;              // (batch, nheads, nchunks, Q): the effective dt, 0 past the sequence
  float* states;            // (batch, nchunks, nheads, headdim, dstate): chunk-end states from
                            // zero, then (after the passing kernel) the state entering each chunk
  // Backward.
  const void* dout;
  const float* dfinal;
  void* dx;
  float* ddt;
  void* dz;
  float* dinit;
  float* dstates;           // like states: first the chunk's seed dL/dH_in from its own outputs,
                            // then dL/d(state leaving the chunk)
  float* dB_part;           // (batch, seqlen, nhb, dstate): dB summed over a head block
  float* dC_part;
  float* dcsL;              // (batch, nheads, nchunks, nslices): dL/dcs_last from the passing, per slice
                            // (slices of kSsdSlice state elements, or of kSsdPassCols columns when
                            // the passing walks the chunks in order)
  float* dA_part;           // (batch * nchunks, nheads)
  float* dbias_part;        // (batch * nchunks, nheads)
  float* dD_part;           // (batch * nchunks, nheads, headdim)
  int64_t batch, seqlen, nheads, headdim, ngroups, dstate, nchunks, nslices;
  int hb, nhb;              // heads per block, blocks over the heads
  int in_order;             // chunk states carried by the in-order kernels (one launch per
                            // direction, no chunk-end states stored) instead of two launches
  int softplus;
  float dt_lo, dt_hi;       // the step is clamped to [dt_lo, dt_hi]
};

hipError_t ssd_fwd_launch(const SsdParams& p, int dtype, hipStream_t st);
hipError_t ssd_bwd_launch(const SsdParams& p, int dtype, hipStream_t st);
// Per-sequence final states (nseqs, nheads, headdim, dstate) of batch row 0
// after the forward; cu holds nseqs + 1 sequence offsets.
hipError_t ssd_varlen_launch(const SsdParams& p, const int32_t* cu, int64_t nseqs, float* out, int dtype,
                             hipStream_t st);

}  // namespace mcpu
