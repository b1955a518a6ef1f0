// Selective state update (one decode step) on gfx950.
//
// Per row (batch, head, p) and state n (reference
// src/mamba_cpu/ops/selective_state_update.py:5-57):
//   dt    = softplus?(dt + dt_bias)
//   state = state * exp(dt * A) + dt * x * B[group]
//   out   = (<state, C[group]> + D * x) * silu(z)
// Same lane layout as the scan: 16 state lanes per row, 4 rows per wave, so a
// 256-thread workgroup updates 16 rows of one batch entry (grid: row tiles of
// the (nheads, headdim) rows x batch, so the row decode is one 32-bit
// division); the <state, C> sum is a DPP row all-reduce. The state is read
// and written in place.
#include "mcpu_common.h"
#include "op_params.h"

namespace mcpu {

template <typename Tx, typename Ts, int SPL>
__global__ void __launch_bounds__(256) state_update_kernel(const StateUpdateParams p) {
  const int j = threadIdx.x & 15;
  const uint32_t hp = blockIdx.x * 16u + (threadIdx.x >> 4);  // row within (nheads, headdim)
  // Whole rows of 16 lanes share every branch, so the DPP reduction below
  // never mixes live and retired lanes of one row.
  if (hp >= static_cast<uint32_t>(p.nheads * p.headdim)) return;
  const uint32_t hd = static_cast<uint32_t>(p.headdim);
  const uint32_t h = hp / hd, pp = hp - h * hd;
  const int64_t g = h / static_cast<uint32_t>(p.nheads / p.ngroups);
  const int64_t N = p.dstate;
  for (int64_t b = blockIdx.y; b < p.batch; b += gridDim.y) {
    const int64_t rowid = b * p.nheads * p.headdim + hp;
    const float x = ld<Tx>(p.x, b * p.sx[0] + h * p.sx[1] + pp * p.sx[2]);
    float dt = ld<Tx>(p.dt, b * p.sdt[0] + h * p.sdt[1] + pp * p.sdt[2]);
    if (p.dt_bias != nullptr) dt += p.dt_bias[h * p.sbias[0] + pp * p.sbias[1]];
    if (p.softplus) dt = softplus(dt);
    const float dtx = dt * x;
    int64_t srow = b;
    if (p.state_idx != nullptr) {
      srow = p.state_idx[b];
      if (srow < 0 || srow >= p.state_batch) {
        if (j == 0) st<Tx>(p.out, rowid, 0.f);
        continue;
      }
    }
    const int64_t sbase = srow * p.sst[0] + h * p.sst[1] + pp * p.sst[2];
    const float* Arow = p.A + h * p.sA[0] + pp * p.sA[1];
    const float* Brow = p.B + b * p.sB[0] + g * p.sB[1];
    const float* Crow = p.C + b * p.sC[0] + g * p.sC[1];
    // Every load of the lane's states first: a load after a store to the
    // state could not be moved above it, which would make each state a
    // memory round trip of its own.
    float sv[SPL], av[SPL], bv[SPL], cv[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      const int n = j + 16 * s;
      const bool ok = n < N;
      sv[s] = ok ? ld<Ts>(p.state, sbase + n) : 0.f;
      av[s] = ok ? Arow[n * p.sA[2]] : 0.f;
      bv[s] = ok ? Brow[n] : 0.f;
      cv[s] = ok ? Crow[n] : 0.f;
    }
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      const int n = j + 16 * s;
      if (n < N) {
        const float v = fmaf(sv[s], fast_exp(dt * av[s]), dtx * bv[s]);
        st<Ts>(p.state, sbase + n, v);
        acc = fmaf(v, cv[s], acc);
      }
    }
    float y = row_allreduce16(acc);
    if (j == 0) {
      if (p.D != nullptr) y = fmaf(x, p.D[h * p.sD[0] + pp * p.sD[1]], y);
      if (p.z != nullptr) {
        const float zz = ld<Tx>(p.z, b * p.sz[0] + h * p.sz[1] + pp * p.sz[2]);
        y *= zz * sigmoid(zz);
      }
      st<Tx>(p.out, rowid, y);
    }
  }
}

template <typename Tx, typename Ts>
static hipError_t launch_su(const StateUpdateParams& p, hipStream_t st) {
  const dim3 blocks(static_cast<unsigned>((p.nheads * p.headdim + 15) / 16),
                    static_cast<unsigned>(p.batch < 65535 ? p.batch : 65535));
  if (p.dstate <= 16)
    hipLaunchKernelGGL((state_update_kernel<Tx, Ts, 1>), dim3(blocks), dim3(256), 0, st, p);
  else if (p.dstate <= 32)
    hipLaunchKernelGGL((state_update_kernel<Tx, Ts, 2>), dim3(blocks), dim3(256), 0, st, p);
  else if (p.dstate <= 64)
    hipLaunchKernelGGL((state_update_kernel<Tx, Ts, 4>), dim3(blocks), dim3(256), 0, st, p);
  else if (p.dstate <= 128)
    hipLaunchKernelGGL((state_update_kernel<Tx, Ts, 8>), dim3(blocks), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((state_update_kernel<Tx, Ts, 16>), dim3(blocks), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename Tx>
static hipError_t launch_su_state(const StateUpdateParams& p, int state_dtype, hipStream_t st) {
  switch (state_dtype) {
    case MCPU_F32: return launch_su<Tx, float>(p, st);
    case MCPU_BF16: return launch_su<Tx, bf16>(p, st);
    default: return launch_su<Tx, f16>(p, st);
  }
}

hipError_t state_update_launch(const StateUpdateParams& p, int dtype, int state_dtype, hipStream_t st) {
  if (p.batch * p.nheads * p.headdim == 0) return hipSuccess;
  switch (dtype) {
    case MCPU_F32: return launch_su_state<float>(p, state_dtype, st);
    case MCPU_BF16: return launch_su_state<bf16>(p, state_dtype, st);
    default: return launch_su_state<f16>(p, state_dtype, st);
  }
}

}  // namespace mcpu
