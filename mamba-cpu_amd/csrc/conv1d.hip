// Causal depthwise conv1d on gfx950: forward, backward and the decode update.
//
// Forward (reference src/mamba_cpu/ops/causal_conv1d.py:16-53 and the tap loop
// of src/mamba_cpu/reference.py:65-75):
//   out[b,d,t] = act(bias[d] + sum_{k<W} w[d,k] * X[b,d,t-(W-1)+k])
// where X[s] = x[s] for s >= 0 and initial_states[W-1+s] (or 0) for s < 0.
// Arithmetic is float32 whatever the storage type; the result is rounded once.
//
// Work split: a "row" is one (batch, channel); each row is cut into chunks of
// kConvT consecutive steps and walked by kConvR threads, thread r taking
// chunks r, r + R, r + 2R, ... The thread index is decomposed channel-fastest
// when the channel stride is 1 (the transposed views Hugging Face passes) and
// time-fastest otherwise, so that neighbouring lanes touch neighbouring
// addresses in both layouts.
#include "mcpu_common.h"
#include "op_params.h"

namespace mcpu {

struct ConvRow {
  int64_t b, d, r;
};

__device__ __forceinline__ ConvRow conv_row(const ConvParams& p, int64_t tid) {
  ConvRow c;
  if (p.channels_last) {
    c.d = tid % p.dim;
    tid /= p.dim;
    c.r = tid % p.R;
    c.b = tid / p.R;
  } else {
    c.r = tid % p.R;
    tid /= p.R;
    c.d = tid % p.dim;
    c.b = tid / p.dim;
  }
  return c;
}

// X[s] for s in [-(W-1), L): input or initial state (zero when absent).
template <typename T>
__device__ __forceinline__ float conv_x(const ConvParams& p, const ConvRow& c, int64_t s) {
  if (s >= 0) return ld<T>(p.x, c.b * p.sx[0] + c.d * p.sx[1] + s * p.sx[2]);
  if (p.init == nullptr || s < -(p.width - 1)) return 0.f;
  return ld<T>(p.init, c.b * p.sinit[0] + c.d * p.sinit[1] + (p.width - 1 + s) * p.sinit[2]);
}

template <typename T>
__global__ void __launch_bounds__(256) conv_fwd_kernel(const ConvParams p) {
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim * p.R) return;
  const ConvRow c = conv_row(p, tid);
  const int W = static_cast<int>(p.width);
  float w[kConvMaxW];
#pragma unroll
  for (int k = 0; k < kConvMaxW; ++k) w[k] = k < W ? p.w[c.d * W + k] : 0.f;
  const float bias = p.bias ? p.bias[c.d] : 0.f;
  for (int64_t ch = c.r; ch < p.nchunks; ch += p.R) {
    const int64_t t0 = ch * kConvT;
    float win[kConvT + kConvMaxW - 1];
#pragma unroll
    for (int i = 0; i < kConvT + kConvMaxW - 1; ++i) {
      const int64_t s = t0 - (W - 1) + i;
      win[i] = (i < kConvT + W - 1 && s < p.seqlen) ? conv_x<T>(p, c, s) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kConvT; ++i) {
      const int64_t t = t0 + i;
      if (t >= p.seqlen) break;
      float acc = bias;
#pragma unroll
      for (int k = 0; k < kConvMaxW; ++k)
        if (k < W) acc = fmaf(w[k], win[i + k], acc);
      if (p.silu) acc = acc * sigmoid(acc);
      st<T>(p.out, c.b * p.sout[0] + c.d * p.sout[1] + t * p.sout[2], acc);
    }
  }
}

// final_states[b, d, i] = X[L - (W-1) + i], i < W-1 (the last W-1 columns of
// [initial_states, x]).
template <typename T>
__global__ void __launch_bounds__(256) conv_final_states_kernel(const ConvParams p) {
  const int64_t W1 = p.width - 1;
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim * W1) return;
  const int64_t i = tid % W1;
  ConvRow c;
  c.d = (tid / W1) % p.dim;
  c.b = tid / (W1 * p.dim);
  c.r = 0;
  st<T>(p.final_states, tid, conv_x<T>(p, c, p.seqlen - W1 + i));
}

// Backward. For the outputs s this thread owns:
//   dpre[t] = dout[t] * act'(pre[t])
//   dX[s]   = sum_k w[k] dpre[s + (W-1) - k]  (+ dfinal for the last W-1 columns)
// dX[s] goes to dx for s >= 0 and to dinitial_states for s < 0 (handled by the
// thread of chunk 0). dw/dbias accumulate dpre[t] X[t-(W-1)+k] over this
// thread's steps and are written as one partial per thread.
template <typename T>
__global__ void __launch_bounds__(256) conv_bwd_kernel(const ConvParams p) {
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim * p.R) return;
  const ConvRow c = conv_row(p, tid);
  const int W = static_cast<int>(p.width);
  const int64_t L = p.seqlen;
  float w[kConvMaxW], dw[kConvMaxW];
#pragma unroll
  for (int k = 0; k < kConvMaxW; ++k) {
    w[k] = k < W ? p.w[c.d * W + k] : 0.f;
    dw[k] = 0.f;
  }
  const float bias = p.bias ? p.bias[c.d] : 0.f;
  float dbias = 0.f;
  const int64_t fin0 = L - (W - 1);  // first column copied into final_states

  // The thread of chunk 0 also produces dX[s] for s in [-(W-1), 0).
  const int64_t first = (c.r == 0) ? -1 : c.r;
  for (int64_t ch = first; ch < p.nchunks; ch = (ch < 0 ? 0 : ch + p.R)) {
    const bool pre_chunk = ch < 0;
    const int64_t s0 = pre_chunk ? -(W - 1) : ch * kConvT;
    const int nout = pre_chunk ? W - 1 : kConvT;
    // dpre for t in [s0, s0 + nout + W - 1), which needs X on
    // [s0 - (W-1), s0 + nout + W - 1).
    float xw[kConvT + 2 * (kConvMaxW - 1)];
    float dp[kConvT + kConvMaxW - 1];
#pragma unroll
    for (int i = 0; i < kConvT + 2 * (kConvMaxW - 1); ++i) {
      const int64_t s = s0 - (W - 1) + i;
      xw[i] = (i < nout + 2 * (W - 1) && s < L) ? conv_x<T>(p, c, s) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kConvT + kConvMaxW - 1; ++i) {
      const int64_t t = s0 + i;
      float v = 0.f;
      if (i < nout + W - 1 && t >= 0 && t < L) {
        float pre = bias;
#pragma unroll
        for (int k = 0; k < kConvMaxW; ++k)
          if (k < W) pre = fmaf(w[k], xw[i + k], pre);
        const float go = ld<T>(p.dout, c.b * p.sdo[0] + c.d * p.sdo[1] + t * p.sdo[2]);
        if (p.silu) {
          const float sg = sigmoid(pre);
          v = go * sg * (1.f + pre * (1.f - sg));
        } else {
          v = go;
        }
      }
      dp[i] = v;
    }
    // Parameter gradients from the steps this chunk owns (t in [s0, s0+nout), t >= 0).
    if (!pre_chunk) {
#pragma unroll
      for (int i = 0; i < kConvT; ++i) {
        if (i < nout && s0 + i < L) {
          dbias += dp[i];
#pragma unroll
          for (int k = 0; k < kConvMaxW; ++k)
            if (k < W) dw[k] = fmaf(dp[i], xw[i + k], dw[k]);
        }
      }
    }
    // Input gradients for s in [s0, s0 + nout).
#pragma unroll
    for (int i = 0; i < kConvT; ++i) {
      const int64_t s = s0 + i;
      if (i >= nout || s >= L) break;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < kConvMaxW; ++k)
        if (k < W) acc = fmaf(w[k], dp[i + (W - 1) - k], acc);
      if (p.dfinal != nullptr && s >= fin0)
        acc += ld<T>(p.dfinal, (c.b * p.dim + c.d) * (W - 1) + (s - fin0));
      if (s >= 0) {
        st<T>(p.dx, c.b * p.sdx[0] + c.d * p.sdx[1] + s * p.sdx[2], acc);
      } else if (p.dinit != nullptr) {
        st<T>(p.dinit, (c.b * p.dim + c.d) * (W - 1) + (s + W - 1), acc);
      }
    }
  }
  float* part = p.dw_part + ((c.b * p.R + c.r) * p.dim + c.d) * (W + 1);
#pragma unroll
  for (int k = 0; k < kConvMaxW; ++k)
    if (k < W) part[k] = dw[k];
  part[W] = dbias;
}

// dweight[d, k] / dbias[d] = sum over (batch, R) partials.
__global__ void __launch_bounds__(256) conv_reduce_dw_kernel(const float* __restrict__ part,
                                                             float* __restrict__ dw,
                                                             float* __restrict__ dbias,
                                                             int64_t nparts, int64_t dim,
                                                             int64_t width) {
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  const int64_t per = dim * (width + 1);
  if (i >= per) return;
  float acc = 0.f;
  for (int64_t q = 0; q < nparts; ++q) acc += part[q * per + i];
  const int64_t d = i / (width + 1), k = i % (width + 1);
  if (k < width) dw[d * width + k] = acc;
  else if (dbias != nullptr) dbias[d] = acc;
}

// Decode update (reference src/mamba_cpu/ops/causal_conv1d.py:56-85): one
// thread per (batch, channel). x_full = [state, x]; out[s] = act(bias +
// sum_k w[k] x_full[state_len-(W-1)+s+k]); state <- last state_len columns.
template <typename T>
__global__ void __launch_bounds__(256) conv_update_kernel(const ConvUpdateParams p) {
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim) return;
  const int64_t d = tid % p.dim, b = tid / p.dim;
  const int W = static_cast<int>(p.width);
  const int64_t S = p.state_len, L = p.seqlen;
  const int64_t xb = b * p.sx[0] + d * p.sx[1];
  const int64_t sb = b * p.sst[0] + d * p.sst[1];
  auto full = [&](int64_t i) -> float {  // x_full[i], i in [0, S + L)
    return i < S ? ld<T>(p.state, sb + i * p.sst[2]) : ld<T>(p.x, xb + (i - S) * p.sx[2]);
  };
  float w[kConvMaxW];
#pragma unroll
  for (int k = 0; k < kConvMaxW; ++k) w[k] = k < W ? p.w[d * W + k] : 0.f;
  const float bias = p.bias ? p.bias[d] : 0.f;
  for (int64_t s = 0; s < L; ++s) {
    float acc = bias;
#pragma unroll
    for (int k = 0; k < kConvMaxW; ++k)
      if (k < W) acc = fmaf(w[k], full(S - (W - 1) + s + k), acc);
    if (p.silu) acc = acc * sigmoid(acc);
    st<T>(p.out, b * p.sout[0] + d * p.sout[1] + s * p.sout[2], acc);
  }
  // Shift: new_state[i] = x_full[L + i]; ascending i never reads a slot it
  // has already overwritten (reads are at index L + i >= i).
  for (int64_t i = 0; i < S; ++i) {
    const float v = full(L + i);
    st<T>(p.state, sb + i * p.sst[2], v);
  }
}

static unsigned blocks_for(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

hipError_t conv_fwd_launch(const ConvParams& p, int dtype, hipStream_t st) {
  const int64_t n = p.batch * p.dim * p.R;
  if (n > 0) {
    switch (dtype) {
      case MCPU_F32: hipLaunchKernelGGL(conv_fwd_kernel<float>, dim3(blocks_for(n)), dim3(256), 0, st, p); break;
      case MCPU_BF16: hipLaunchKernelGGL(conv_fwd_kernel<bf16>, dim3(blocks_for(n)), dim3(256), 0, st, p); break;
      default: hipLaunchKernelGGL(conv_fwd_kernel<f16>, dim3(blocks_for(n)), dim3(256), 0, st, p); break;
    }
    if (hipError_t e = hipGetLastError()) return e;
  }
  const int64_t nf = p.final_states ? p.batch * p.dim * (p.width - 1) : 0;
  if (nf > 0) {
    switch (dtype) {
      case MCPU_F32: hipLaunchKernelGGL(conv_final_states_kernel<float>, dim3(blocks_for(nf)), dim3(256), 0, st, p); break;
      case MCPU_BF16: hipLaunchKernelGGL(conv_final_states_kernel<bf16>, dim3(blocks_for(nf)), dim3(256), 0, st, p); break;
      default: hipLaunchKernelGGL(conv_final_states_kernel<f16>, dim3(blocks_for(nf)), dim3(256), 0, st, p); break;
    }
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t conv_bwd_launch(const ConvParams& p, int dtype, float* dweight, float* dbias, hipStream_t st) {
  const int64_t n = p.batch * p.dim * p.R;
  if (n > 0) {
    switch (dtype) {
      case MCPU_F32: hipLaunchKernelGGL(conv_bwd_kernel<float>, dim3(blocks_for(n)), dim3(256), 0, st, p); break;
      case MCPU_BF16: hipLaunchKernelGGL(conv_bwd_kernel<bf16>, dim3(blocks_for(n)), dim3(256), 0, st, p); break;
      default: hipLaunchKernelGGL(conv_bwd_kernel<f16>, dim3(blocks_for(n)), dim3(256), 0, st, p); break;
    }
    if (hipError_t e = hipGetLastError()) return e;
  }
  const int64_t per = p.dim * (p.width + 1);
  hipLaunchKernelGGL(conv_reduce_dw_kernel, dim3(blocks_for(per)), dim3(256), 0, st, p.dw_part,
                     dweight, dbias, p.batch * p.R, p.dim, p.width);
  return hipGetLastError();
}

hipError_t conv_update_launch(const ConvUpdateParams& p, int dtype, hipStream_t st) {
  const int64_t n = p.batch * p.dim;
  if (n == 0) return hipSuccess;
  switch (dtype) {
    case MCPU_F32: hipLaunchKernelGGL(conv_update_kernel<float>, dim3(blocks_for(n)), dim3(256), 0, st, p); break;
    case MCPU_BF16: hipLaunchKernelGGL(conv_update_kernel<bf16>, dim3(blocks_for(n)), dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL(conv_update_kernel<f16>, dim3(blocks_for(n)), dim3(256), 0, st, p); break;
  }
  return hipGetLastError();
}

}  // namespace mcpu
