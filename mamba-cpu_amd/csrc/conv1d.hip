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

// Packed-sequence id of step s of row b, or a value no id equals outside the
// sequence (the taps there read zeros anyway: seq_idx excludes initial states).
__device__ __forceinline__ int64_t conv_seq(const ConvParams& p, int64_t b, int64_t s) {
  return (s >= 0 && s < p.seqlen) ? static_cast<int64_t>(p.seq_idx[b * p.seqlen + s]) : INT64_MIN;
}

// WT: the width as a compile-time constant (2..5), or 0 for any width up to
// kConvMaxW read from the parameters. With a fixed width the window and tap
// loops unroll to exactly the taps that exist. SEQ: packed sequences (seq_idx);
// a tap reading another sequence's input counts as zero.
template <typename T, int WT, bool SEQ>
__global__ void __launch_bounds__(256) conv_fwd_kernel(const ConvParams p) {
  constexpr int MW = WT > 0 ? WT : kConvMaxW;
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim * p.R) return;
  const ConvRow c = conv_row(p, tid);
  const int W = WT > 0 ? WT : static_cast<int>(p.width);
  float w[MW];
#pragma unroll
  for (int k = 0; k < MW; ++k) w[k] = k < W ? p.w[c.d * W + k] : 0.f;
  const float bias = p.bias ? p.bias[c.d] : 0.f;
  for (int64_t ch = c.r; ch < p.nchunks; ch += p.R) {
    const int64_t t0 = ch * kConvT;
    float win[kConvT + MW - 1];
    int64_t sq[SEQ ? kConvT + MW - 1 : 1];
#pragma unroll
    for (int i = 0; i < kConvT + MW - 1; ++i) {
      const int64_t s = t0 - (W - 1) + i;
      win[i] = (i < kConvT + W - 1 && s < p.seqlen) ? conv_x<T>(p, c, s) : 0.f;
      if constexpr (SEQ) sq[i] = conv_seq(p, c.b, s);
    }
#pragma unroll
    for (int i = 0; i < kConvT; ++i) {
      const int64_t t = t0 + i;
      if (t >= p.seqlen) break;
      float acc = bias;
#pragma unroll
      for (int k = 0; k < MW; ++k) {
        if (k >= W) continue;
        float xk = win[i + k];
        if constexpr (SEQ) xk = sq[i + k] == sq[i + W - 1] ? xk : 0.f;
        acc = fmaf(w[k], xk, acc);
      }
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
template <typename T, int WT, bool SEQ>
__global__ void __launch_bounds__(256) conv_bwd_kernel(const ConvParams p) {
  constexpr int MW = WT > 0 ? WT : kConvMaxW;
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim * p.R) return;
  const ConvRow c = conv_row(p, tid);
  const int W = WT > 0 ? WT : static_cast<int>(p.width);
  const int64_t L = p.seqlen;
  float w[MW], dw[MW];
#pragma unroll
  for (int k = 0; k < MW; ++k) {
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
    float xw[kConvT + 2 * (MW - 1)];
    float dp[kConvT + MW - 1];
    int64_t sq[SEQ ? kConvT + 2 * (MW - 1) : 1];  // ids of the xw positions
    // Tap mask: input at xw index a feeds the output whose own xw index is o.
    auto same = [&](int a, int o) { if constexpr (SEQ) return sq[a] == sq[o]; else return true; };
#pragma unroll
    for (int i = 0; i < kConvT + 2 * (MW - 1); ++i) {
      const int64_t s = s0 - (W - 1) + i;
      xw[i] = (i < nout + 2 * (W - 1) && s < L) ? conv_x<T>(p, c, s) : 0.f;
      if constexpr (SEQ) sq[i] = conv_seq(p, c.b, s);
    }
#pragma unroll
    for (int i = 0; i < kConvT + MW - 1; ++i) {
      const int64_t t = s0 + i;
      float v = 0.f;
      if (i < nout + W - 1 && t >= 0 && t < L) {
        float pre = bias;
#pragma unroll
        for (int k = 0; k < MW; ++k)
          if (k < W) pre = fmaf(w[k], same(i + k, i + W - 1) ? xw[i + k] : 0.f, pre);
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
          for (int k = 0; k < MW; ++k)
            if (k < W) dw[k] = fmaf(same(i + k, i + W - 1) ? dp[i] : 0.f, xw[i + k], dw[k]);
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
      for (int k = 0; k < MW; ++k)
        if (k < W)
          acc = fmaf(w[k], same(i + W - 1, i + 2 * (W - 1) - k) ? dp[i + (W - 1) - k] : 0.f, acc);
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
  for (int k = 0; k < MW; ++k)
    if (k < W) part[k] = dw[k];
  part[W] = dbias;
}

// Widths above kConvMaxW (the reference's F.conv1d takes any width): per-element
// kernels whose tap loops read the weights from memory. Forward: one thread per
// output. Backward: dpre = dout * act'(pre) per element into the workspace,
// then dX per input position (W taps of dpre, plus dfinal_states), and
// dweight/dbias partials over segments of kConvWideSeg steps, summed by
// conv_reduce_dw_kernel. Threads run along the contiguous dimension (channel
// or time) of x.

// (b, d, i) of thread tid over a (batch, dim, span) index space.
__device__ __forceinline__ ConvRow wide_index(const ConvParams& p, int64_t tid, int64_t span, int64_t& i) {
  ConvRow c;
  c.r = 0;
  if (p.channels_last) {
    c.d = tid % p.dim;
    tid /= p.dim;
    i = tid % span;
    c.b = tid / span;
  } else {
    i = tid % span;
    tid /= span;
    c.d = tid % p.dim;
    c.b = tid / p.dim;
  }
  return c;
}

// The pre-activation at step t: bias + sum_k w[k] X[t-(W-1)+k], taps from
// another packed sequence counting as zero.
template <typename T, bool SEQ>
__device__ float wide_pre(const ConvParams& p, const ConvRow& c, int64_t t) {
  const int64_t W = p.width;
  const float* w = p.w + c.d * W;
  const int64_t sid = SEQ ? conv_seq(p, c.b, t) : 0;
  float acc = p.bias ? p.bias[c.d] : 0.f;
  for (int64_t k = 0; k < W; ++k) {
    const int64_t s = t - (W - 1) + k;
    if (SEQ && conv_seq(p, c.b, s) != sid) continue;
    acc = fmaf(w[k], conv_x<T>(p, c, s), acc);
  }
  return acc;
}

template <typename T, bool SEQ>
__global__ void __launch_bounds__(256) conv_fwd_wide_kernel(const ConvParams p) {
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim * p.seqlen) return;
  int64_t t;
  const ConvRow c = wide_index(p, tid, p.seqlen, t);
  float acc = wide_pre<T, SEQ>(p, c, t);
  if (p.silu) acc = acc * sigmoid(acc);
  st<T>(p.out, c.b * p.sout[0] + c.d * p.sout[1] + t * p.sout[2], acc);
}

template <typename T, bool SEQ>
__global__ void __launch_bounds__(256) conv_dpre_wide_kernel(const ConvParams p) {
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim * p.seqlen) return;
  int64_t t;
  const ConvRow c = wide_index(p, tid, p.seqlen, t);
  const float go = ld<T>(p.dout, c.b * p.sdo[0] + c.d * p.sdo[1] + t * p.sdo[2]);
  float v = go;
  if (p.silu) {
    const float pre = wide_pre<T, SEQ>(p, c, t);
    const float sg = sigmoid(pre);
    v = go * sg * (1.f + pre * (1.f - sg));
  }
  p.dpre[(c.b * p.dim + c.d) * p.seqlen + t] = v;
}

// dX[s] for s in [-(W-1), L): to dx (s >= 0) or dinitial_states (s < 0).
template <typename T, bool SEQ>
__global__ void __launch_bounds__(256) conv_dx_wide_kernel(const ConvParams p) {
  const int64_t W = p.width, W1 = W - 1, L = p.seqlen, span = L + W1;
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim * span) return;
  int64_t i;
  const ConvRow c = wide_index(p, tid, span, i);
  const int64_t s = i - W1;
  if (s < 0 && p.dinit == nullptr) return;
  const float* w = p.w + c.d * W;
  const float* dp = p.dpre + (c.b * p.dim + c.d) * L;
  const int64_t sid = SEQ ? conv_seq(p, c.b, s) : 0;
  float acc = 0.f;
  for (int64_t k = 0; k < W; ++k) {
    const int64_t t = s + W1 - k;  // the output that reads X[s] through tap k
    if (t < 0 || t >= L) continue;
    if (SEQ && conv_seq(p, c.b, t) != sid) continue;
    acc = fmaf(w[k], dp[t], acc);
  }
  if (p.dfinal != nullptr && s >= L - W1) acc += ld<T>(p.dfinal, (c.b * p.dim + c.d) * W1 + (s - (L - W1)));
  if (s >= 0) st<T>(p.dx, c.b * p.sdx[0] + c.d * p.sdx[1] + s * p.sdx[2], acc);
  else st<T>(p.dinit, (c.b * p.dim + c.d) * W1 + (s + W1), acc);
}

// part[((b * nseg + g) * dim + d) * (W+1) + k]: over the steps t of segment g,
// sum dpre[t] X[t-(W-1)+k] (k < W) or dpre[t] (k = W).
template <typename T, bool SEQ>
__global__ void __launch_bounds__(256) conv_dw_wide_kernel(const ConvParams p, int64_t nseg) {
  const int64_t W = p.width, W1 = W - 1, L = p.seqlen, per = p.dim * (W + 1);
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * nseg * per) return;
  const int64_t e = tid % per, bg = tid / per;
  ConvRow c;
  c.r = 0;
  c.d = e / (W + 1);
  c.b = bg / nseg;
  const int64_t k = e % (W + 1), g = bg % nseg;
  const int64_t t0 = g * kConvWideSeg, t1 = t0 + kConvWideSeg < L ? t0 + kConvWideSeg : L;
  const float* dp = p.dpre + (c.b * p.dim + c.d) * L;
  float acc = 0.f;
  for (int64_t t = t0; t < t1; ++t) {
    if (k == W) {
      acc += dp[t];
      continue;
    }
    const int64_t s = t - W1 + k;
    if (SEQ && conv_seq(p, c.b, s) != conv_seq(p, c.b, t)) continue;
    acc = fmaf(dp[t], conv_x<T>(p, c, s), acc);
  }
  p.dw_part[tid] = acc;
}

// dweight[d, k] / dbias[d] = sum over the (batch, R or segment) partials.
// A workgroup covers 64 consecutive (d, k) entries; its four waves each sum
// every fourth partial (four loads in flight per lane), then combine in LDS.
__global__ void __launch_bounds__(256) conv_reduce_dw_kernel(const float* __restrict__ part,
                                                             float* __restrict__ dw,
                                                             float* __restrict__ dbias,
                                                             int64_t nparts, int64_t dim,
                                                             int64_t width) {
  __shared__ float s_acc[4][64];
  const int lane = threadIdx.x & 63, q0 = threadIdx.x >> 6;
  const int64_t per = dim * (width + 1);
  const int64_t i = blockIdx.x * 64ll + lane;
  float acc = 0.f;
  if (i < per) {
    int64_t q = q0;
    for (; q + 12 < nparts; q += 16) {
      const float a0 = part[q * per + i], a1 = part[(q + 4) * per + i];
      const float a2 = part[(q + 8) * per + i], a3 = part[(q + 12) * per + i];
      acc += (a0 + a1) + (a2 + a3);
    }
    for (; q < nparts; q += 4) acc += part[q * per + i];
  }
  s_acc[q0][lane] = acc;
  __syncthreads();
  if (q0 == 0 && i < per) {
    const float total = (s_acc[0][lane] + s_acc[1][lane]) + (s_acc[2][lane] + s_acc[3][lane]);
    const int64_t d = i / (width + 1), k = i % (width + 1);
    if (k < width) dw[d * width + k] = total;
    else if (dbias != nullptr) dbias[d] = total;
  }
}

// Decode update (reference src/mamba_cpu/ops/causal_conv1d.py:56-85): one
// thread per (batch, channel). x_full = [state, x]; out[s] = act(bias +
// sum_k w[k] x_full[state_len-(W-1)+s+k]); state <- last state_len columns.
// With conv_state_indices, batch row b works on state row state_idx[b] (rows
// out of range are skipped: out = 0, state untouched). With cache_seqlens the
// state is a ring buffer (the upstream causal_conv1d package's semantics): the
// W-1 inputs before x sit at (cs - (W-1) + k) mod state_len, and x[s] is
// written at (cs + s) mod state_len after every output has been computed.
template <typename T, bool WIDE>
__global__ void __launch_bounds__(256) conv_update_kernel(const ConvUpdateParams p) {
  const int64_t tid = blockIdx.x * 256ll + threadIdx.x;
  if (tid >= p.batch * p.dim) return;
  const int64_t d = tid % p.dim, b = tid / p.dim;
  const int W = static_cast<int>(p.width);
  const int64_t S = p.state_len, L = p.seqlen;
  const int64_t xb = b * p.sx[0] + d * p.sx[1];
  const int64_t ob = b * p.sout[0] + d * p.sout[1];
  int64_t srow = b;
  if (p.state_idx != nullptr) {
    srow = p.state_idx[b];
    if (srow < 0 || srow >= p.state_batch) {
      for (int64_t s = 0; s < L; ++s) st<T>(p.out, ob + s * p.sout[2], 0.f);
      return;
    }
  }
  const int64_t sb = srow * p.sst[0] + d * p.sst[1];
  const bool ring = p.cache_seqlens != nullptr;
  const int64_t cs = ring ? p.cache_seqlens[b] : 0;
  auto wrap = [&](int64_t i) { const int64_t r = i % S; return r < 0 ? r + S : r; };
  // x_full[i] for i in [S - (W-1), S + L): the W-1 inputs before x, then x.
  auto full = [&](int64_t i) -> float {
    if (i >= S) return ld<T>(p.x, xb + (i - S) * p.sx[2]);
    const int64_t pos = ring ? wrap(cs - S + i) : i;
    return ld<T>(p.state, sb + pos * p.sst[2]);
  };
  // WIDE (widths above kConvMaxW): the taps read the weights from memory.
  float w[WIDE ? 1 : kConvMaxW];
  if constexpr (!WIDE) {
#pragma unroll
    for (int k = 0; k < kConvMaxW; ++k) w[k] = k < W ? p.w[d * W + k] : 0.f;
  }
  const float bias = p.bias ? p.bias[d] : 0.f;
  for (int64_t s = 0; s < L; ++s) {
    float acc = bias;
    if constexpr (WIDE) {
      for (int k = 0; k < W; ++k) acc = fmaf(p.w[d * W + k], full(S - (W - 1) + s + k), acc);
    } else {
#pragma unroll
      for (int k = 0; k < kConvMaxW; ++k)
        if (k < W) acc = fmaf(w[k], full(S - (W - 1) + s + k), acc);
    }
    if (p.silu) acc = acc * sigmoid(acc);
    st<T>(p.out, ob + s * p.sout[2], acc);
  }
  if (ring) {
    for (int64_t s = 0; s < L; ++s) st<T>(p.state, sb + wrap(cs + s) * p.sst[2], full(S + s));
    return;
  }
  // Shift: new_state[i] = x_full[L + i]; ascending i never reads a slot it
  // has already overwritten (reads are at index L + i >= i).
  for (int64_t i = 0; i < S; ++i) {
    const float v = full(L + i);
    st<T>(p.state, sb + i * p.sst[2], v);
  }
}

// Single-step update (the decode step): a 2-D grid of channel tiles x batch
// rows, so no per-thread 64-bit division. Without a ring buffer the whole old
// state row (state_len <= kUpd1MaxS entries) and x are loaded together, the
// output is computed, and the shifted state is stored from registers, so no
// store waits on a reload of a slot it depends on. With a ring buffer (RING,
// any state_len) the W-1 taps are read at (cs - (W-1) + k) mod state_len and x
// is written at cs mod state_len; cs is the batch row's, so the wrap runs once
// per wave in 32-bit scalar arithmetic.
constexpr int kUpd1MaxS = 8;

template <typename T, int W, bool RING>
__global__ void __launch_bounds__(256) conv_update1_kernel(const ConvUpdateParams p) {
  const int64_t d = blockIdx.x * 256ll + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (d >= p.dim) return;
  const int S = static_cast<int>(p.state_len);
  const int64_t ob = b * p.sout[0] + d * p.sout[1];
  int64_t srow = b;
  if (p.state_idx != nullptr) {
    srow = p.state_idx[b];
    if (srow < 0 || srow >= p.state_batch) {
      st<T>(p.out, ob, 0.f);
      return;
    }
  }
  const int64_t sb = srow * p.sst[0] + d * p.sst[1];
  const float xv = ld<T>(p.x, b * p.sx[0] + d * p.sx[1]);
  float w[W];
#pragma unroll
  for (int k = 0; k < W; ++k) w[k] = p.w[d * W + k];
  float acc = p.bias ? p.bias[d] : 0.f;
  if constexpr (RING) {
    const int cs = __builtin_amdgcn_readfirstlane(p.cache_seqlens[b]);
    auto wrap = [&](int i) { const int r = i % S; return r < 0 ? r + S : r; };
#pragma unroll
    for (int k = 0; k < W - 1; ++k)
      acc = fmaf(w[k], ld<T>(p.state, sb + wrap(cs - (W - 1) + k) * p.sst[2]), acc);
    acc = fmaf(w[W - 1], xv, acc);
    if (p.silu) acc = acc * sigmoid(acc);
    st<T>(p.out, ob, acc);
    st<T>(p.state, sb + wrap(cs) * p.sst[2], xv);
    return;
  }
  float old[kUpd1MaxS];
#pragma unroll
  for (int i = 0; i < kUpd1MaxS; ++i) old[i] = i < S ? ld<T>(p.state, sb + i * p.sst[2]) : 0.f;
  // Taps 0 .. W-2 read the newest W-1 state entries, tap W-1 reads x.
#pragma unroll
  for (int k = 0; k < W - 1; ++k) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < kUpd1MaxS; ++i)
      if (i == S - (W - 1) + k) v = old[i];
    acc = fmaf(w[k], v, acc);
  }
  acc = fmaf(w[W - 1], xv, acc);
  if (p.silu) acc = acc * sigmoid(acc);
  st<T>(p.out, ob, acc);
#pragma unroll
  for (int i = 0; i < kUpd1MaxS; ++i)
    if (i < S) st<T>(p.state, sb + i * p.sst[2], i + 1 < S ? old[i + 1 < kUpd1MaxS ? i + 1 : 0] : xv);
}

// ---- Time-contiguous fast path ------------------------------------------------
// For x, out, dout and dx with unit time stride, rows aligned to 4 elements and
// seqlen a multiple of VT: each thread owns VT consecutive steps of one
// (batch, channel) row (VT = 16 where seqlen allows, else 8) with 16-byte
// (fp32) or 8-byte (16-bit) vector loads and stores; the W-1 inputs before its first step (and,
// in the backward, the W-1 steps after its last) are re-read from the
// neighbouring thread's vector, which the cache serves. A workgroup covers
// `rpw` rows of `tpr` threads each (short rows) or one 256 * VT-step segment of
// a row (long rows), so a row segment never straddles a wave.

template <typename T>
__device__ __forceinline__ void ld4(const void* base, int64_t idx, float* v) {
  if constexpr (sizeof(T) == 4) {
    const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  } else {
    const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const T*>(base) + idx);
    const uint32_t h[4] = {q.x & 0xffffu, q.x >> 16, q.y & 0xffffu, q.y >> 16};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (std::is_same_v<T, bf16>) v[i] = to_f32(bf16{static_cast<uint16_t>(h[i])});
      else v[i] = to_f32(__builtin_bit_cast(f16, static_cast<uint16_t>(h[i])));
    }
  }
}

template <typename T>
__device__ __forceinline__ void st4(void* base, int64_t idx, const float* v) {
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4*>(static_cast<float*>(base) + idx) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (std::is_same_v<T, bf16>) {
    *reinterpret_cast<uint2*>(static_cast<T*>(base) + idx) =
        make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  } else {
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = __builtin_bit_cast(uint16_t, from_f32<T>(v[i]));
    *reinterpret_cast<uint2*>(static_cast<T*>(base) + idx) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
  }
}

struct ConvClTile {
  int64_t b, d0, t0, S;  // batch row, first of the lane's 4 channels, segment start and length
  bool wave_on;          // the wave's segment starts inside the sequence
  bool active;           // ... and the lane's channels exist
};

struct ConvTile {
  ConvRow c;      // (batch, channel) of the row
  int64_t t0;     // first step of this thread
  int64_t seg;    // row segment of the workgroup
  bool active;    // the thread has steps to do
};

template <int VT>
__device__ __forceinline__ ConvTile conv_tile(const ConvParams& p, int tid) {
  ConvTile g;
  // A row segment is whole waves (tpr >= 64), so the row is wave-uniform and
  // its (batch, channel) split stays in the scalar unit.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lt = tid & (p.tpr - 1), sub = (wave * 64) / p.tpr;
  int64_t row;
  if (p.nseg > 1) {
    row = blockIdx.x / p.nseg;
    g.seg = blockIdx.x % p.nseg;
  } else {
    row = static_cast<int64_t>(blockIdx.x) * p.rpw + sub;
    g.seg = 0;
  }
  g.t0 = (g.seg * p.tpr + lt) * VT;
  const int64_t rows = p.batch * p.dim;
  g.active = row < rows && g.t0 < p.seqlen;
  if (row >= rows) row = rows - 1;
  g.c.b = row / p.dim;
  g.c.d = row % p.dim;
  g.c.r = 0;
  return g;
}

template <typename T, int W, int VT>
__global__ void __launch_bounds__(256) conv_fwd_vt_kernel(const ConvParams p) {
  const ConvTile g = conv_tile<VT>(p, threadIdx.x);
  if (!g.active) return;
  const ConvRow& c = g.c;
  float w[W];
#pragma unroll
  for (int k = 0; k < W; ++k) w[k] = p.w[c.d * W + k];
  const float bias = p.bias ? p.bias[c.d] : 0.f;
  const int64_t xrow = c.b * p.sx[0] + c.d * p.sx[1];
  float xv[4 + VT];  // X[t0 - 4 .. t0 + VT)
  if (g.t0 > 0) {
    ld4<T>(p.x, xrow + g.t0 - 4, xv);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) xv[i] = conv_x<T>(p, c, i - 4);
  }
#pragma unroll
  for (int q = 0; q < VT; q += 4) ld4<T>(p.x, xrow + g.t0 + q, xv + 4 + q);
  float o[VT];
#pragma unroll
  for (int i = 0; i < VT; ++i) {
    float acc = bias;
#pragma unroll
    for (int k = 0; k < W; ++k) acc = fmaf(w[k], xv[4 + i - (W - 1) + k], acc);
    o[i] = p.silu ? acc * sigmoid(acc) : acc;
  }
  const int64_t orow = c.b * p.sout[0] + c.d * p.sout[1];
#pragma unroll
  for (int q = 0; q < VT; q += 4) st4<T>(p.out, orow + g.t0 + q, o + q);
}

// Sum over the 64 lanes of a wave, in a fixed order, result in every lane.
__device__ __forceinline__ float wave_sum(float x) {
  x = row_allreduce16(x);
  x = swap_sum<32>(x, x);
  return swap_sum<16>(x, x);
}

template <typename T, int W, int VT>
__global__ void __launch_bounds__(256) conv_bwd_vt_kernel(const ConvParams p) {
  __shared__ float s_part[4][W + 1];
  const ConvTile g = conv_tile<VT>(p, threadIdx.x);
  const ConvRow& c = g.c;
  const int64_t L = p.seqlen;
  float dwk[W + 1];  // dweight[0..W), dbias
#pragma unroll
  for (int k = 0; k <= W; ++k) dwk[k] = 0.f;
  const int64_t xrow = c.b * p.sx[0] + c.d * p.sx[1];
  const int64_t orow = c.b * p.sdo[0] + c.d * p.sdo[1];
  float xv[4 + VT + 4];  // X[t0 - 4 .. t0 + VT + 4)
  float go[VT + 4];      // dout[t0 .. t0 + VT + 4)
#pragma unroll
  for (int i = 0; i < 4 + VT + 4; ++i) xv[i] = 0.f;
#pragma unroll
  for (int i = 0; i < VT + 4; ++i) go[i] = 0.f;
  if (g.active) {
#pragma unroll
    for (int q = 0; q < VT; q += 4) {
      ld4<T>(p.x, xrow + g.t0 + q, xv + 4 + q);
      ld4<T>(p.dout, orow + g.t0 + q, go + q);
    }
  }
  // The halos are the neighbouring lanes' own steps: a wave's lanes hold
  // consecutive VT-step pieces of one row, so lane l's four steps before t0
  // are lane l - 1's last four and its four after are lane l + 1's first
  // four (every lane runs the shifts; inactive lanes hold zeros). Only the
  // wave's end lanes read them from memory.
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xv[i] = dpp<kWaveShr1>(xv[VT + i]);
    xv[4 + VT + i] = dpp<kWaveShl1>(xv[4 + i]);
    go[VT + i] = dpp<kWaveShl1>(go[i]);
  }
  if (g.active) {
    float w[W];
#pragma unroll
    for (int k = 0; k < W; ++k) w[k] = p.w[c.d * W + k];
    const float bias = p.bias ? p.bias[c.d] : 0.f;
    const bool tail = g.t0 + VT < L;  // the next VT steps exist
    if (g.t0 == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[i] = conv_x<T>(p, c, i - 4);
    } else if (lane == 0) {
      ld4<T>(p.x, xrow + g.t0 - 4, xv);
    }
    if (tail && lane == 63) {
      ld4<T>(p.x, xrow + g.t0 + VT, xv + 4 + VT);
      ld4<T>(p.dout, orow + g.t0 + VT, go + VT);
    }
    // dpre[t0 + i] for i < VT + W - 1 (zero past the sequence end).
    float dp[VT + W - 1];
#pragma unroll
    for (int i = 0; i < VT + W - 1; ++i) {
      float pre = bias;
#pragma unroll
      for (int k = 0; k < W; ++k) pre = fmaf(w[k], xv[4 + i - (W - 1) + k], pre);
      float v = go[i];
      if (p.silu) {
        const float sg = sigmoid(pre);
        v *= sg * (1.f + pre * (1.f - sg));
      }
      dp[i] = (i < VT || tail) ? v : 0.f;
    }
    float dx[VT];
    const int64_t fin0 = L - (W - 1);
#pragma unroll
    for (int i = 0; i < VT; ++i) {
      dwk[W] += dp[i];
#pragma unroll
      for (int k = 0; k < W; ++k) dwk[k] = fmaf(dp[i], xv[4 + i - (W - 1) + k], dwk[k]);
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < W; ++k) acc = fmaf(w[k], dp[i + (W - 1) - k], acc);
      if (p.dfinal != nullptr && g.t0 + i >= fin0)
        acc += ld<T>(p.dfinal, (c.b * p.dim + c.d) * (W - 1) + (g.t0 + i - fin0));
      dx[i] = acc;
    }
    const int64_t xr = c.b * p.sdx[0] + c.d * p.sdx[1];
#pragma unroll
    for (int q = 0; q < VT; q += 4) st4<T>(p.dx, xr + g.t0 + q, dx + q);
    if (g.t0 == 0 && p.dinit != nullptr) {
      // dX[s] for s in [-(W-1), 0): the initial-state columns.
#pragma unroll
      for (int s = -(W - 1); s < 0; ++s) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < W; ++k)
          if (s + (W - 1) - k >= 0) acc = fmaf(w[k], dp[s + (W - 1) - k], acc);
        st<T>(p.dinit, (c.b * p.dim + c.d) * (W - 1) + (s + W - 1), acc);
      }
    }
  }
  // Per-segment sums of dweight/dbias: wave sums, then the segment's waves in order.
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k <= W; ++k) {
    const float v = wave_sum(dwk[k]);
    if ((threadIdx.x & 63) == 0) s_part[wave][k] = v;
  }
  __syncthreads();
  const int wps = p.tpr / 64;  // waves per segment
  if (threadIdx.x < p.rpw * (W + 1)) {
    const int sg = threadIdx.x / (W + 1), k = threadIdx.x % (W + 1);
    float acc = 0.f;
    for (int q = 0; q < wps; ++q) acc += s_part[sg * wps + q][k];
    const int64_t row = p.nseg > 1 ? static_cast<int64_t>(blockIdx.x) / p.nseg
                                   : static_cast<int64_t>(blockIdx.x) * p.rpw + sg;
    if (row < p.batch * p.dim) {
      const int64_t b = row / p.dim, d = row % p.dim;
      const int64_t seg = p.nseg > 1 ? blockIdx.x % p.nseg : 0;
      p.dw_part[((b * p.nseg + seg) * p.dim + d) * (W + 1) + k] = acc;
    }
  }
}

// ---------------------------------------------------------------------------
// Channel-contiguous fast path: x (and out, or dout and dx) with unit channel
// stride, as Hugging Face's transposed (batch, seqlen, dim) views and the
// fused mixer's halves of xz are. A lane owns four neighbouring channels and
// moves them as one 16-byte (fp32) or 8-byte (16-bit) vector per step; a wave
// covers 256 channels of one batch row over one time segment of
// kConvClG * cl_ng steps, so the step index and the packed-sequence ids are
// wave-uniform. Each lane walks its segment with a rolling window of the last
// W inputs (and, backward, the last W output gradients) in registers; the W-1
// inputs before the segment, and backward the W-1 steps after it, are re-read
// from the neighbouring segments. A workgroup is four waves: four consecutive
// segments of the same 256 channels (grid: channel tiles, segment groups,
// batch). Packed sequences cost only where a segment holds a boundary: a wave
// vote over its ids picks the masked body for those segments alone.

__device__ __forceinline__ ConvClTile conv_cl_tile(const ConvParams& p) {
  ConvClTile g;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  g.S = static_cast<int64_t>(p.cl_ng) * kConvClG;
  g.b = blockIdx.z;
  g.t0 = (static_cast<int64_t>(blockIdx.y) * 4 + wave) * g.S;
  g.d0 = (static_cast<int64_t>(blockIdx.x) * 64 + (threadIdx.x & 63)) * 4;
  g.wave_on = g.t0 < p.seqlen;
  g.active = g.wave_on && g.d0 < p.dim;
  return g;
}

// Sequence id of step s of row b, s clamped to the sequence: positions
// outside it read zeros (seq_idx excludes initial states), so any id serves.
__device__ __forceinline__ int32_t conv_cl_id(const ConvParams& p, int64_t b, int64_t s) {
  s = s < 0 ? 0 : (s >= p.seqlen ? p.seqlen - 1 : s);
  return __builtin_amdgcn_readfirstlane(p.seq_idx[b * p.seqlen + s]);
}

// Whether the ids over steps [lo, hi] (hi - lo < 128) are not all equal.
// Wave-uniform; every lane of the wave must be active.
__device__ __forceinline__ bool conv_cl_breaks(const ConvParams& p, int64_t b, int64_t lo, int64_t hi) {
  const int lane = threadIdx.x & 63;
  const int32_t first = conv_cl_id(p, b, lo);
  const int32_t* ids = p.seq_idx + b * p.seqlen;
  auto at = [&](int64_t s) { return ids[s < 0 ? 0 : (s >= p.seqlen ? p.seqlen - 1 : s)]; };
  const bool d1 = lo + lane <= hi && at(lo + lane) != first;
  const bool d2 = lo + 64 + lane <= hi && at(lo + 64 + lane) != first;
  return __ballot(d1 || d2) != 0;
}

// M: mask the taps by sequence id. TAIL: the segment runs past the sequence
// end (steps there load nothing and store nothing).
template <typename T, int W, bool M, bool TAIL>
__device__ __forceinline__ void conv_fwd_cl_body(const ConvParams& p, const ConvClTile& g,
                                                 const float (&w)[4][W], const float (&bias)[4]) {
  const int64_t L = p.seqlen;
  const int64_t xb = g.b * p.sx[0] + g.d0, ob = g.b * p.sout[0] + g.d0;
  float xw[W][4];  // X[t-(W-1) .. t], four channels each
  int32_t iw[W];   // their sequence ids (M)
#pragma unroll
  for (int j = 0; j < W - 1; ++j) {
    const int64_t s = g.t0 - (W - 1) + j;
    if (s >= 0) {
      ld4<T>(p.x, xb + s * p.sx[2], xw[j]);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) xw[j][c] = 0.f;
    }
    if constexpr (M) iw[j] = conv_cl_id(p, g.b, s);
  }
  // Unrolled groups of G steps; the masked body (segments with a sequence
  // boundary) unrolls less, so the register budget it sets for the kernel
  // stays near the unmasked body's.
  constexpr int G = M ? 2 : kConvClG;
  for (int64_t tg = g.t0; tg < g.t0 + g.S; tg += G) {
    if (TAIL && tg >= L) break;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int64_t t = tg + i;
      const bool in = !TAIL || t < L;
      if (in) {
        ld4<T>(p.x, xb + t * p.sx[2], xw[W - 1]);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) xw[W - 1][c] = 0.f;
      }
      if constexpr (M) iw[W - 1] = conv_cl_id(p, g.b, t);
      float o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float acc = bias[c];
#pragma unroll
        for (int k = 0; k < W; ++k) {
          float xk = xw[k][c];
          if constexpr (M) xk = iw[k] == iw[W - 1] ? xk : 0.f;
          acc = fmaf(w[c][k], xk, acc);
        }
        o[c] = p.silu ? acc * sigmoid(acc) : acc;
      }
      if (in) st4<T>(p.out, ob + t * p.sout[2], o);
#pragma unroll
      for (int k = 0; k < W - 1; ++k) {
#pragma unroll
        for (int c = 0; c < 4; ++c) xw[k][c] = xw[k + 1][c];
        if constexpr (M) iw[k] = iw[k + 1];
      }
    }
  }
}

template <typename T, int W, bool SEQ>
__global__ void __launch_bounds__(256) conv_fwd_cl_kernel(const ConvParams p) {
  const ConvClTile g = conv_cl_tile(p);
  if (!g.wave_on) return;
  bool masked = false;
  if constexpr (SEQ) masked = conv_cl_breaks(p, g.b, g.t0 - (W - 1), g.t0 + g.S - 1);
  if (!g.active) return;
  float w[4][W], bias[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int k = 0; k < W; ++k) w[c][k] = p.w[(g.d0 + c) * W + k];
    bias[c] = p.bias ? p.bias[g.d0 + c] : 0.f;
  }
  const bool tail = g.t0 + g.S > p.seqlen;
  if (SEQ && masked) {
    if (tail) conv_fwd_cl_body<T, W, SEQ, true>(p, g, w, bias);
    else conv_fwd_cl_body<T, W, SEQ, false>(p, g, w, bias);
  } else {
    if (tail) conv_fwd_cl_body<T, W, false, true>(p, g, w, bias);
    else conv_fwd_cl_body<T, W, false, false>(p, g, w, bias);
  }
}

// One step t of the backward walk. OWN: t is one of the segment's steps (its
// dweight/dbias terms are this segment's); otherwise it is one of the W-1
// look-ahead steps past the segment. dx is emitted for s = t - (W-1) once s
// is inside the segment.
template <typename T, int W, bool M, bool TAIL, bool OWN>
__device__ __forceinline__ void conv_bwd_cl_step(const ConvParams& p, const ConvClTile& g, int64_t t,
                                                 const float (&w)[4][W], const float (&bias)[4],
                                                 float (&xw)[W][4], float (&dpw)[W][4], int32_t (&iw)[W],
                                                 float (&dw)[4][W], float (&db)[4]) {
  const int64_t L = p.seqlen;
  const bool in = !TAIL || t < L;
  float go[4];
  if (in) {
    ld4<T>(p.x, g.b * p.sx[0] + g.d0 + t * p.sx[2], xw[W - 1]);
    ld4<T>(p.dout, g.b * p.sdo[0] + g.d0 + t * p.sdo[2], go);
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) xw[W - 1][c] = go[c] = 0.f;
  }
  if constexpr (M) iw[W - 1] = conv_cl_id(p, g.b, t);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float xm[W];
    float pre = bias[c];
#pragma unroll
    for (int k = 0; k < W; ++k) {
      xm[k] = xw[k][c];
      if constexpr (M) xm[k] = iw[k] == iw[W - 1] ? xm[k] : 0.f;
      pre = fmaf(w[c][k], xm[k], pre);
    }
    float v = go[c];
    if (p.silu) {
      const float sg = sigmoid(pre);
      v *= sg * (1.f + pre * (1.f - sg));
    }
    dpw[W - 1][c] = v;
    if constexpr (OWN) {
      db[c] += v;
#pragma unroll
      for (int k = 0; k < W; ++k) dw[c][k] = fmaf(v, xm[k], dw[c][k]);
    }
  }
  // dx[s] = sum_k w[k] dpre[s + (W-1) - k], the tap of output s + (W-1) - k
  // that reads input s; dpre[s + (W-1) - k] sits in dpw[W-1-k].
  const int64_t s = t - (W - 1);
  if (s >= g.t0 && (!TAIL || s < L)) {
    float dx[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        float d = dpw[W - 1 - k][c];
        if constexpr (M) d = iw[0] == iw[W - 1 - k] ? d : 0.f;
        acc = fmaf(w[c][k], d, acc);
      }
      dx[c] = acc;
    }
    st4<T>(p.dx, g.b * p.sdx[0] + g.d0 + s * p.sdx[2], dx);
  }
#pragma unroll
  for (int k = 0; k < W - 1; ++k) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      xw[k][c] = xw[k + 1][c];
      dpw[k][c] = dpw[k + 1][c];
    }
    if constexpr (M) iw[k] = iw[k + 1];
  }
}

template <typename T, int W, bool M, bool TAIL>
__device__ __forceinline__ void conv_bwd_cl_body(const ConvParams& p, const ConvClTile& g,
                                                 const float (&w)[4][W], const float (&bias)[4],
                                                 float (&dw)[4][W], float (&db)[4]) {
  float xw[W][4], dpw[W][4];
  int32_t iw[W];
#pragma unroll
  for (int j = 0; j < W; ++j) {
#pragma unroll
    for (int c = 0; c < 4; ++c) xw[j][c] = dpw[j][c] = 0.f;
    iw[j] = 0;
  }
#pragma unroll
  for (int j = 0; j < W - 1; ++j) {
    const int64_t s = g.t0 - (W - 1) + j;
    if (s >= 0) ld4<T>(p.x, g.b * p.sx[0] + g.d0 + s * p.sx[2], xw[j]);
    if constexpr (M) iw[j] = conv_cl_id(p, g.b, s);
  }
  // The segment's own steps, in unrolled groups of G; a tail segment stops
  // after the group holding the sequence's last step. Groups of 4 (2 when
  // masked) keep the kernel at 104 VGPRs, 4 waves per SIMD: measured 3 %
  // faster than 8 (137 VGPRs) and no slower than 2.
  constexpr int G = M ? 2 : 4;
  const int64_t own_end = TAIL && p.seqlen < g.t0 + g.S ? p.seqlen : g.t0 + g.S;
  int64_t tg = g.t0;
  for (; tg < own_end; tg += G) {
#pragma unroll
    for (int i = 0; i < G; ++i)
      conv_bwd_cl_step<T, W, M, TAIL, true>(p, g, tg + i, w, bias, xw, dpw, iw, dw, db);
  }
  // W-1 more steps right after the last one walked (the windows roll one
  // step per call), for the dx of the segment's last W-1 steps.
#pragma unroll
  for (int i = 0; i < W - 1; ++i)
    conv_bwd_cl_step<T, W, M, TAIL, false>(p, g, tg + i, w, bias, xw, dpw, iw, dw, db);
}

template <typename T, int W, bool SEQ>
__global__ void __launch_bounds__(256) conv_bwd_cl_kernel(const ConvParams p) {
  __shared__ float s_part[4][W + 1][256];
  const ConvClTile g = conv_cl_tile(p);
  float dw[4][W], db[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    db[c] = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) dw[c][k] = 0.f;
  }
  if (g.wave_on) {
    bool masked = false;
    if constexpr (SEQ) masked = conv_cl_breaks(p, g.b, g.t0 - (W - 1), g.t0 + g.S + W - 2);
    if (g.active) {
      float w[4][W], bias[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int k = 0; k < W; ++k) w[c][k] = p.w[(g.d0 + c) * W + k];
        bias[c] = p.bias ? p.bias[g.d0 + c] : 0.f;
      }
      const bool tail = g.t0 + g.S + (W - 1) > p.seqlen;
      if (SEQ && masked) {
        if (tail) conv_bwd_cl_body<T, W, SEQ, true>(p, g, w, bias, dw, db);
        else conv_bwd_cl_body<T, W, SEQ, false>(p, g, w, bias, dw, db);
      } else {
        if (tail) conv_bwd_cl_body<T, W, false, true>(p, g, w, bias, dw, db);
        else conv_bwd_cl_body<T, W, false, false>(p, g, w, bias, dw, db);
      }
    }
  }
  // The workgroup's four segments summed in order: one partial per
  // (batch, segment group, channel).
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int k = 0; k < W; ++k) s_part[wave][k][lane * 4 + c] = dw[c][k];
    s_part[wave][W][lane * 4 + c] = db[c];
  }
  __syncthreads();
  const int64_t d = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (d < p.dim) {
    float* part = p.dw_part + ((g.b * p.cl_gy + blockIdx.y) * p.dim + d) * (W + 1);
#pragma unroll
    for (int k = 0; k <= W; ++k)
      part[k] = (s_part[0][k][threadIdx.x] + s_part[1][k][threadIdx.x]) +
                (s_part[2][k][threadIdx.x] + s_part[3][k][threadIdx.x]);
  }
}

template <typename T, bool SEQ>
static hipError_t launch_cl_seq(const ConvParams& p, bool bwd, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((p.dim + 255) / 256), static_cast<unsigned>(p.cl_gy),
                  static_cast<unsigned>(p.batch));
  switch (p.width) {
#define MCPU_CONV_CL(WW)                                                                         \
  case WW:                                                                                       \
    if (bwd) hipLaunchKernelGGL((conv_bwd_cl_kernel<T, WW, SEQ>), grid, dim3(256), 0, st, p);   \
    else hipLaunchKernelGGL((conv_fwd_cl_kernel<T, WW, SEQ>), grid, dim3(256), 0, st, p);       \
    break;
    MCPU_CONV_CL(2)
    MCPU_CONV_CL(3)
    MCPU_CONV_CL(4)
    MCPU_CONV_CL(5)
#undef MCPU_CONV_CL
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_cl(const ConvParams& p, bool bwd, hipStream_t st) {
  return p.seq_idx != nullptr ? launch_cl_seq<T, true>(p, bwd, st) : launch_cl_seq<T, false>(p, bwd, st);
}

static hipError_t launch_cl_dtype(const ConvParams& p, int dtype, bool bwd, hipStream_t st) {
  switch (dtype) {
    case MCPU_F32: return launch_cl<float>(p, bwd, st);
    case MCPU_BF16: return launch_cl<bf16>(p, bwd, st);
    default: return launch_cl<f16>(p, bwd, st);
  }
}

template <typename T>
static hipError_t launch_vt(const ConvParams& p, bool bwd, hipStream_t st) {
  const unsigned grid = static_cast<unsigned>(
      p.nseg > 1 ? p.batch * p.dim * p.nseg : (p.batch * p.dim + p.rpw - 1) / p.rpw);
  switch (p.width) {
#define MCPU_CONV_VT(WW)                                                                             \
  case WW:                                                                                           \
    if (p.vt == 16) {                                                                                \
      if (bwd) hipLaunchKernelGGL((conv_bwd_vt_kernel<T, WW, 16>), dim3(grid), dim3(256), 0, st, p);  \
      else hipLaunchKernelGGL((conv_fwd_vt_kernel<T, WW, 16>), dim3(grid), dim3(256), 0, st, p);      \
    } else {                                                                                         \
      if (bwd) hipLaunchKernelGGL((conv_bwd_vt_kernel<T, WW, 8>), dim3(grid), dim3(256), 0, st, p);   \
      else hipLaunchKernelGGL((conv_fwd_vt_kernel<T, WW, 8>), dim3(grid), dim3(256), 0, st, p);       \
    }                                                                                                \
    break;
    MCPU_CONV_VT(2)
    MCPU_CONV_VT(3)
    MCPU_CONV_VT(4)
    MCPU_CONV_VT(5)
#undef MCPU_CONV_VT
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

static hipError_t launch_vt_dtype(const ConvParams& p, int dtype, bool bwd, hipStream_t st) {
  switch (dtype) {
    case MCPU_F32: return launch_vt<float>(p, bwd, st);
    case MCPU_BF16: return launch_vt<bf16>(p, bwd, st);
    default: return launch_vt<f16>(p, bwd, st);
  }
}

static unsigned blocks_for(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

// Segments of the per-element backward's dweight partials.
int64_t conv_wide_nseg(int64_t seqlen) { return seqlen > 0 ? (seqlen + kConvWideSeg - 1) / kConvWideSeg : 1; }

template <typename T, bool SEQ>
static hipError_t launch_wide_seq(const ConvParams& p, bool bwd, float* dweight, float* dbias, hipStream_t st) {
  const int64_t n = p.batch * p.dim * p.seqlen;
  if (!bwd) {
    if (n > 0) hipLaunchKernelGGL((conv_fwd_wide_kernel<T, SEQ>), dim3(blocks_for(n)), dim3(256), 0, st, p);
    return hipGetLastError();
  }
  if (n > 0) hipLaunchKernelGGL((conv_dpre_wide_kernel<T, SEQ>), dim3(blocks_for(n)), dim3(256), 0, st, p);
  const int64_t nx = p.batch * p.dim * (p.seqlen + p.width - 1);
  if (nx > 0) hipLaunchKernelGGL((conv_dx_wide_kernel<T, SEQ>), dim3(blocks_for(nx)), dim3(256), 0, st, p);
  const int64_t nseg = conv_wide_nseg(p.seqlen), per = p.dim * (p.width + 1);
  if (p.batch * nseg * per > 0)
    hipLaunchKernelGGL((conv_dw_wide_kernel<T, SEQ>), dim3(blocks_for(p.batch * nseg * per)), dim3(256), 0, st,
                       p, nseg);
  hipLaunchKernelGGL(conv_reduce_dw_kernel, dim3(static_cast<unsigned>((per + 63) / 64)), dim3(256), 0, st,
                     p.dw_part, dweight, dbias, p.batch * nseg, p.dim, p.width);
  return hipGetLastError();
}

static hipError_t launch_wide(const ConvParams& p, int dtype, bool bwd, float* dweight, float* dbias,
                              hipStream_t st) {
  const bool seq = p.seq_idx != nullptr;
  switch (dtype) {
    case MCPU_F32:
      return seq ? launch_wide_seq<float, true>(p, bwd, dweight, dbias, st)
                 : launch_wide_seq<float, false>(p, bwd, dweight, dbias, st);
    case MCPU_BF16:
      return seq ? launch_wide_seq<bf16, true>(p, bwd, dweight, dbias, st)
                 : launch_wide_seq<bf16, false>(p, bwd, dweight, dbias, st);
    default:
      return seq ? launch_wide_seq<f16, true>(p, bwd, dweight, dbias, st)
                 : launch_wide_seq<f16, false>(p, bwd, dweight, dbias, st);
  }
}

// The chunked kernels, specialised for widths 2..5 (Mamba's is 4).
template <typename T, bool SEQ>
static hipError_t launch_generic_seq(const ConvParams& p, bool bwd, unsigned grid, hipStream_t st) {
  switch (p.width) {
#define MCPU_CONV_GEN(WW)                                                                          \
  case WW:                                                                                         \
    if (bwd) hipLaunchKernelGGL((conv_bwd_kernel<T, WW, SEQ>), dim3(grid), dim3(256), 0, st, p);  \
    else hipLaunchKernelGGL((conv_fwd_kernel<T, WW, SEQ>), dim3(grid), dim3(256), 0, st, p);      \
    break;
    MCPU_CONV_GEN(2)
    MCPU_CONV_GEN(3)
    MCPU_CONV_GEN(4)
    MCPU_CONV_GEN(5)
#undef MCPU_CONV_GEN
    default:
      if (bwd) hipLaunchKernelGGL((conv_bwd_kernel<T, 0, SEQ>), dim3(grid), dim3(256), 0, st, p);
      else hipLaunchKernelGGL((conv_fwd_kernel<T, 0, SEQ>), dim3(grid), dim3(256), 0, st, p);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_generic(const ConvParams& p, bool bwd, unsigned grid, hipStream_t st) {
  return p.seq_idx != nullptr ? launch_generic_seq<T, true>(p, bwd, grid, st)
                              : launch_generic_seq<T, false>(p, bwd, grid, st);
}

static hipError_t launch_generic_dtype(const ConvParams& p, int dtype, bool bwd, unsigned grid,
                                       hipStream_t st) {
  switch (dtype) {
    case MCPU_F32: return launch_generic<float>(p, bwd, grid, st);
    case MCPU_BF16: return launch_generic<bf16>(p, bwd, grid, st);
    default: return launch_generic<f16>(p, bwd, grid, st);
  }
}

hipError_t conv_fwd_launch(const ConvParams& p, int dtype, hipStream_t st) {
  const int64_t n = p.batch * p.dim * p.R;
  if (p.width > kConvMaxW) {
    if (hipError_t e = launch_wide(p, dtype, false, nullptr, nullptr, st)) return e;
  } else if (n > 0 && p.vt) {
    if (hipError_t e = launch_vt_dtype(p, dtype, false, st)) return e;
  } else if (n > 0 && p.cl) {
    if (hipError_t e = launch_cl_dtype(p, dtype, false, st)) return e;
  } else if (n > 0) {
    if (hipError_t e = launch_generic_dtype(p, dtype, false, blocks_for(n), st)) return e;
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
  if (p.width > kConvMaxW) return launch_wide(p, dtype, true, dweight, dbias, st);
  if (n > 0 && p.vt) {
    if (hipError_t e = launch_vt_dtype(p, dtype, true, st)) return e;
    const int64_t per = p.dim * (p.width + 1);
    hipLaunchKernelGGL(conv_reduce_dw_kernel, dim3(static_cast<unsigned>((per + 63) / 64)), dim3(256),
                       0, st, p.dw_part, dweight, dbias, p.batch * p.nseg, p.dim, p.width);
    return hipGetLastError();
  }
  if (n > 0 && p.cl) {
    if (hipError_t e = launch_cl_dtype(p, dtype, true, st)) return e;
    const int64_t per = p.dim * (p.width + 1);
    hipLaunchKernelGGL(conv_reduce_dw_kernel, dim3(static_cast<unsigned>((per + 63) / 64)), dim3(256),
                       0, st, p.dw_part, dweight, dbias, p.batch * p.cl_gy, p.dim, p.width);
    return hipGetLastError();
  }
  if (n > 0) {
    if (hipError_t e = launch_generic_dtype(p, dtype, true, blocks_for(n), st)) return e;
  }
  const int64_t per = p.dim * (p.width + 1);
  hipLaunchKernelGGL(conv_reduce_dw_kernel, dim3(static_cast<unsigned>((per + 63) / 64)), dim3(256), 0,
                     st, p.dw_part, dweight, dbias, p.batch * p.R, p.dim, p.width);
  return hipGetLastError();
}

template <typename T, bool RING>
static bool launch_update1_ring(const ConvUpdateParams& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((p.dim + 255) / 256), static_cast<unsigned>(p.batch));
  switch (p.width) {
    case 2: hipLaunchKernelGGL((conv_update1_kernel<T, 2, RING>), grid, dim3(256), 0, st, p); return true;
    case 3: hipLaunchKernelGGL((conv_update1_kernel<T, 3, RING>), grid, dim3(256), 0, st, p); return true;
    case 4: hipLaunchKernelGGL((conv_update1_kernel<T, 4, RING>), grid, dim3(256), 0, st, p); return true;
    default: return false;
  }
}

template <typename T>
static bool launch_update1(const ConvUpdateParams& p, hipStream_t st) {
  return p.cache_seqlens != nullptr ? launch_update1_ring<T, true>(p, st) : launch_update1_ring<T, false>(p, st);
}

hipError_t conv_update_launch(const ConvUpdateParams& p, int dtype, hipStream_t st) {
  const int64_t n = p.batch * p.dim;
  if (n == 0) return hipSuccess;
  const bool fits = p.cache_seqlens != nullptr ? p.state_len <= INT32_MAX : p.state_len <= kUpd1MaxS;
  if (p.seqlen == 1 && fits && p.batch <= 65535) {
    bool done = false;
    switch (dtype) {
      case MCPU_F32: done = launch_update1<float>(p, st); break;
      case MCPU_BF16: done = launch_update1<bf16>(p, st); break;
      default: done = launch_update1<f16>(p, st); break;
    }
    if (done) return hipGetLastError();
  }
  const bool wide = p.width > kConvMaxW;
  switch (dtype) {
    case MCPU_F32:
      if (wide) hipLaunchKernelGGL((conv_update_kernel<float, true>), dim3(blocks_for(n)), dim3(256), 0, st, p);
      else hipLaunchKernelGGL((conv_update_kernel<float, false>), dim3(blocks_for(n)), dim3(256), 0, st, p);
      break;
    case MCPU_BF16:
      if (wide) hipLaunchKernelGGL((conv_update_kernel<bf16, true>), dim3(blocks_for(n)), dim3(256), 0, st, p);
      else hipLaunchKernelGGL((conv_update_kernel<bf16, false>), dim3(blocks_for(n)), dim3(256), 0, st, p);
      break;
    default:
      if (wide) hipLaunchKernelGGL((conv_update_kernel<f16, true>), dim3(blocks_for(n)), dim3(256), 0, st, p);
      else hipLaunchKernelGGL((conv_update_kernel<f16, false>), dim3(blocks_for(n)), dim3(256), 0, st, p);
      break;
  }
  return hipGetLastError();
}

}  // namespace mcpu
