// C-ABI entry points of the Mamba-2 SSD scan: argument checks, the layout of
// the saved buffer and of the backward's workspace, and kernel sequencing.
// Nothing is allocated here.
#include <cmath>
#include <cstring>

#include "abi_util.h"
#include "scan_common.h"
#include "ssd_params.h"

namespace mcpu {
namespace {

int check_ssd(const mcpu_ssd_args* a) {
  if (a == nullptr) return fail(MCPU_ERR_INVALID, "ssd: null argument block");
  if (a->batch < 0 || a->seqlen < 0 || a->nheads < 1 || a->ngroups < 1)
    return fail(MCPU_ERR_INVALID, "ssd: bad sizes");
  // Per-step tensors may be NULL (empty) when there are no steps.
  const bool steps = a->batch > 0 && a->seqlen > 0;
  if (a->A == nullptr || (steps && (a->x == nullptr || a->dt == nullptr || a->B == nullptr || a->C == nullptr)))
    return fail(MCPU_ERR_INVALID, "ssd: x, dt, A, B and C are required");
  if (a->nheads % a->ngroups != 0)
    return fail(MCPU_ERR_INVALID, "ssd: nheads (%lld) must be divisible by ngroups (%lld)",
                (long long)a->nheads, (long long)a->ngroups);
  if (a->headdim < 16 || a->headdim > kSsdMaxP || a->headdim % 16 != 0)
    return fail(MCPU_ERR_UNSUPPORTED, "ssd: headdim must be a multiple of 16 up to %d, got %lld", kSsdMaxP,
                (long long)a->headdim);
  if (a->dstate < 16 || a->dstate > kSsdMaxN || a->dstate % 16 != 0)
    return fail(MCPU_ERR_UNSUPPORTED, "ssd: dstate must be a multiple of 16 up to %d, got %lld", kSsdMaxN,
                (long long)a->dstate);
  if (!valid_dtype(a->dtype)) return fail(MCPU_ERR_INVALID, "ssd: bad dtype %d", a->dtype);
  if (!(a->dt_limit_lo <= a->dt_limit_hi))
    return fail(MCPU_ERR_INVALID, "ssd: dt_limit must be an interval (lo <= hi)");
  if (a->head_block != 0 &&
      (a->head_block < 1 || a->head_block > kSsdMaxHeadBlock || (a->nheads / a->ngroups) % a->head_block != 0))
    return fail(MCPU_ERR_INVALID, "ssd: head_block %d must be 0 or a divisor of nheads / ngroups up to %d",
                a->head_block, kSsdMaxHeadBlock);
  if (a->chunk_pass < 0 || a->chunk_pass > 2)
    return fail(MCPU_ERR_INVALID, "ssd: chunk_pass %d must be 0, 1 or 2", a->chunk_pass);
  const int64_t nchunks = (a->seqlen + kSsdQ - 1) / kSsdQ;
  if (nchunks > 0x7fffffffll || a->nheads > 65535 || a->batch > 65535)
    return fail(MCPU_ERR_UNSUPPORTED, "ssd: grid too large");
  // Tiles move four elements at a time.
  for (const void* t : {a->x, a->B, a->C, a->z, static_cast<const void*>(a->out), static_cast<const void*>(a->ysave),
                        a->dout, static_cast<const void*>(a->dx), static_cast<const void*>(a->dz)})
    if (reinterpret_cast<uintptr_t>(t) % 16 != 0)
      return fail(MCPU_ERR_INVALID, "ssd: x, z, B, C, out, ysave, dout, dx and dz must be 16-byte aligned");
  return MCPU_OK;
}

// Heads per workgroup of the chunk kernels. Their LDS holds one workgroup
// per CU, so a launch takes ceil(workgroups / CUs) rounds, each as long as one
// workgroup: a part shared by its heads (staging B and C, forming C B^T) plus
// a part per head, the shared part about 0.4 of a head's in both directions.
// The divisor of the heads per group, up to kSsdMaxHeadBlock, with the least
// rounds x (0.4 + heads) is chosen; against timings of both directions at
// batch 1-8, 24-80 heads, seqlen 256-4096 this picks the fastest block or one
// within 3 % of it.
int head_block(const mcpu_ssd_args* a) {
  const int64_t hpg = a->nheads / a->ngroups;
  const int64_t chunks = a->batch * ((a->seqlen + kSsdQ - 1) / kSsdQ);
  int hb = 1;
  int64_t best = -1;
  for (int d = 1; d <= kSsdMaxHeadBlock; ++d) {
    if (hpg % d != 0) continue;
    const int64_t rounds = (chunks * (a->nheads / d) + kSsdCUs - 1) / kSsdCUs;
    const int64_t cost = rounds * (4 + 10 * d);
    if (best < 0 || cost < best) {
      best = cost;
      hb = d;
    }
  }
  return hb;
}

// Whether the chunk states are carried by the in-order kernels, one
// workgroup per (batch, head, 64-state column block) walking every chunk, or
// by the two-launch form, parallel over chunks. The in-order forward is the
// faster from about 256 such workgroups, the in-order backward from about
// 160 (measured at 48-640 of them); the two directions choose on their own
// (the saved buffer is the same for both forms).
bool in_order(const mcpu_ssd_args* a, bool bwd) {
  if (a->chunk_pass != 0) return a->chunk_pass == 2;
  const int64_t cols = (a->dstate + kSsdPassCols - 1) / kSsdPassCols;
  return a->batch * a->nheads * cols >= (bwd ? 160 : 256);
}

SsdParams make_ssd(const mcpu_ssd_args* a, bool bwd = false) {
  SsdParams p;
  std::memset(&p, 0, sizeof(p));
  p.x = a->x;
  p.dt = a->dt;
  p.A = a->A;
  p.B = a->B;
  p.C = a->C;
  p.D = a->D;
  p.z = a->z;
  p.dt_bias = a->dt_bias;
  p.init = a->initial_states;
  p.seq_idx = a->seq_idx;
  p.batch = a->batch;
  p.seqlen = a->seqlen;
  p.nheads = a->nheads;
  p.headdim = a->headdim;
  p.ngroups = a->ngroups;
  p.dstate = a->dstate;
  p.nchunks = (a->seqlen + kSsdQ - 1) / kSsdQ;
  p.in_order = in_order(a, bwd) ? 1 : 0;
  p.nslices = p.in_order ? (a->dstate + kSsdPassCols - 1) / kSsdPassCols
                         : (a->headdim * a->dstate + kSsdSlice - 1) / kSsdSlice;
  p.hb = a->head_block != 0 ? a->head_block : head_block(a);
  p.nhb = static_cast<int>(a->nheads / p.hb);
  p.softplus = a->dt_softplus != 0;
  p.dt_lo = a->dt_limit_lo;
  p.dt_hi = a->dt_limit_hi;
  return p;
}

// The saved buffer: cs, cs_lo and step (batch, nheads, nchunks, 64), then
// states (batch, nchunks, nheads, headdim, dstate), all float32.
struct SavedLayout {
  size_t cs = 0, cs_lo = 0, step = 0, states = 0, total = 0;
};
SavedLayout saved_layout(const SsdParams& p) {
  SavedLayout w;
  const size_t chunk = sizeof(float) * p.batch * p.nheads * p.nchunks * kSsdQ;
  w.cs = 0;
  w.cs_lo = align_up(chunk);
  w.step = w.cs_lo + align_up(chunk);
  w.states = w.step + align_up(chunk);
  w.total = w.states + align_up(sizeof(float) * p.batch * p.nchunks * p.nheads * p.headdim * p.dstate);
  return w;
}

// The backward's workspace.
struct BwdLayout {
  size_t dstates = 0, dB = 0, dC = 0, dcsL = 0, dA = 0, dbias = 0, dD = 0, total = 0;
};
BwdLayout bwd_layout(const SsdParams& p) {
  BwdLayout w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  const size_t f = sizeof(float);
  w.dstates = take(f * p.batch * p.nchunks * p.nheads * p.headdim * p.dstate);
  w.dB = take(f * p.batch * p.seqlen * p.nhb * p.dstate);
  w.dC = take(f * p.batch * p.seqlen * p.nhb * p.dstate);
  w.dcsL = take(f * p.batch * p.nheads * p.nchunks * p.nslices);
  w.dA = take(f * p.batch * p.nchunks * p.nheads);
  w.dbias = take(f * p.batch * p.nchunks * p.nheads);
  w.dD = take(f * p.batch * p.nchunks * p.nheads * p.headdim);
  w.total = off;
  return w;
}

void bind_saved(SsdParams& p, const void* saved) {
  const SavedLayout w = saved_layout(p);
  char* s = static_cast<char*>(const_cast<void*>(saved));
  p.cs = reinterpret_cast<float*>(s + w.cs);
  p.cs_lo = reinterpret_cast<float*>(s + w.cs_lo);
  p.step = reinterpret_cast<float*>(s + w.step);
  p.states = reinterpret_cast<float*>(s + w.states);
}

}  // namespace
}  // namespace mcpu

using namespace mcpu;

extern "C" size_t mcpu_ssd_saved_size(const mcpu_ssd_args* a) {
  if (check_ssd(a) != MCPU_OK) {
    clear_error();
    return 0;
  }
  return saved_layout(make_ssd(a)).total;
}

extern "C" int mcpu_ssd_fwd(const mcpu_ssd_args* a, void* saved, size_t saved_bytes, void* stream) {
  clear_error();
  if (int rc = check_ssd(a)) return rc;
  if (a->out == nullptr && a->batch > 0 && a->seqlen > 0) return fail(MCPU_ERR_INVALID, "ssd_fwd: out is required");
  SsdParams p = make_ssd(a);
  const size_t need = saved_layout(p).total;
  if (need > 0 && (saved == nullptr || saved_bytes < need))
    return fail(MCPU_ERR_INVALID, "ssd_fwd: saved buffer of %zu bytes needed, got %zu", need, saved_bytes);
  if (int rc = mcpu_check_device()) return rc;
  if (a->batch == 0 || a->seqlen == 0) {
    // Nothing to scan: the final state is the initial state (or 0).
    if (a->final_states != nullptr && a->batch > 0) {
      const int64_t n = a->batch * a->nheads * a->headdim * a->dstate;
      if (a->initial_states != nullptr)
        return hip_status(hipMemcpyAsync(a->final_states, a->initial_states, sizeof(float) * n,
                                         hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)),
                          "ssd_fwd copy");
      return zero_f32(a->final_states, n, static_cast<hipStream_t>(stream));
    }
    return MCPU_OK;
  }
  bind_saved(p, saved);
  p.out = a->out;
  p.final_states = a->final_states;
  p.ysave = a->ysave;
  return hip_status(ssd_fwd_launch(p, a->dtype, static_cast<hipStream_t>(stream)), "ssd_fwd launch");
}

extern "C" int mcpu_ssd_varlen_states(const mcpu_ssd_args* a, const void* saved, size_t saved_bytes,
                                      const int32_t* cu_seqlens, int64_t nseqs, float* varlen_states, void* stream) {
  clear_error();
  if (int rc = check_ssd(a)) return rc;
  if (a->batch != 1)
    return fail(MCPU_ERR_INVALID, "ssd_varlen_states: packed sequences need batch 1, got %lld", (long long)a->batch);
  if (nseqs < 0 || nseqs > 0x7fffffffll)
    return fail(MCPU_ERR_INVALID, "ssd_varlen_states: bad sequence count %lld", (long long)nseqs);
  if (nseqs == 0) return MCPU_OK;
  if (cu_seqlens == nullptr || varlen_states == nullptr)
    return fail(MCPU_ERR_INVALID, "ssd_varlen_states: cu_seqlens and varlen_states are required");
  SsdParams p = make_ssd(a);
  const size_t need = saved_layout(p).total;
  if (need > 0 && (saved == nullptr || saved_bytes < need))
    return fail(MCPU_ERR_INVALID, "ssd_varlen_states: the forward's saved buffer of %zu bytes is needed, got %zu",
                need, saved_bytes);
  if (int rc = mcpu_check_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->seqlen == 0)  // every sequence is empty
    return zero_f32(varlen_states, nseqs * a->nheads * a->headdim * a->dstate, st);
  bind_saved(p, saved);
  return hip_status(ssd_varlen_launch(p, cu_seqlens, nseqs, varlen_states, a->dtype, st), "ssd_varlen_states launch");
}

extern "C" size_t mcpu_ssd_bwd_workspace_size(const mcpu_ssd_args* a) {
  if (check_ssd(a) != MCPU_OK) {
    clear_error();
    return 0;
  }
  return bwd_layout(make_ssd(a, true)).total;
}

extern "C" int mcpu_ssd_bwd(const mcpu_ssd_args* a, const void* saved, size_t saved_bytes, void* workspace,
                            size_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_ssd(a)) return rc;
  if (a->dA == nullptr || (a->batch > 0 && a->seqlen > 0 &&
                           (a->dout == nullptr || a->dx == nullptr || a->ddt == nullptr || a->dB == nullptr ||
                            a->dC == nullptr)))
    return fail(MCPU_ERR_INVALID, "ssd_bwd: dout, dx, ddt, dA, dB and dC are required");
  if (a->z != nullptr && (a->dz == nullptr || a->ysave == nullptr))
    return fail(MCPU_ERR_INVALID, "ssd_bwd: dz and the forward's ysave are required when z is given");
  if (a->D != nullptr && a->dD == nullptr)
    return fail(MCPU_ERR_INVALID, "ssd_bwd: dD is required when D is given");
  if (a->dt_bias != nullptr && a->ddt_bias == nullptr)
    return fail(MCPU_ERR_INVALID, "ssd_bwd: ddt_bias is required when dt_bias is given");
  if (a->initial_states != nullptr && a->dinitial_states == nullptr)
    return fail(MCPU_ERR_INVALID, "ssd_bwd: dinitial_states is required when initial_states is given");
  SsdParams p = make_ssd(a, true);
  const size_t need_saved = saved_layout(p).total;
  if (need_saved > 0 && (saved == nullptr || saved_bytes < need_saved))
    return fail(MCPU_ERR_INVALID, "ssd_bwd: the forward's saved buffer of %zu bytes is needed, got %zu",
                need_saved, saved_bytes);
  const BwdLayout w = bwd_layout(p);
  if (w.total > 0 && (workspace == nullptr || workspace_bytes < w.total))
    return fail(MCPU_ERR_INVALID, "ssd_bwd: workspace of %zu bytes needed, got %zu", w.total, workspace_bytes);
  if (int rc = mcpu_check_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->batch == 0 || a->seqlen == 0) {
    // Parameter gradients are zero; the initial state's is the final state's.
    if (int rc = zero_f32(a->dA, a->nheads, st)) return rc;
    if (a->dD) if (int rc = zero_f32(a->dD, a->nheads * a->headdim, st)) return rc;
    if (a->ddt_bias) if (int rc = zero_f32(a->ddt_bias, a->nheads, st)) return rc;
    if (a->dinitial_states && a->batch > 0) {
      const int64_t n = a->batch * a->nheads * a->headdim * a->dstate;
      if (a->dfinal_states)
        return hip_status(hipMemcpyAsync(a->dinitial_states, a->dfinal_states, sizeof(float) * n,
                                         hipMemcpyDeviceToDevice, st),
                          "ssd_bwd copy");
      return zero_f32(a->dinitial_states, n, st);
    }
    return MCPU_OK;
  }
  bind_saved(p, saved);
  char* ws = static_cast<char*>(workspace);
  p.ysave = a->ysave;
  p.dout = a->dout;
  p.dfinal = a->dfinal_states;
  p.dx = a->dx;
  p.ddt = a->ddt;
  p.dz = a->dz;
  p.dinit = a->dinitial_states;
  p.dstates = reinterpret_cast<float*>(ws + w.dstates);
  p.dB_part = reinterpret_cast<float*>(ws + w.dB);
  p.dC_part = reinterpret_cast<float*>(ws + w.dC);
  p.dcsL = reinterpret_cast<float*>(ws + w.dcsL);
  p.dA_part = reinterpret_cast<float*>(ws + w.dA);
  p.dbias_part = reinterpret_cast<float*>(ws + w.dbias);
  p.dD_part = reinterpret_cast<float*>(ws + w.dD);
  if (int rc = hip_status(ssd_bwd_launch(p, a->dtype, st), "ssd_bwd launch")) return rc;
  // dB/dC summed over each group's head blocks; dA / dD / ddt_bias over (batch, chunk).
  const int64_t blocks_per_group = p.nhb / p.ngroups;
  const PartialSum sums[5] = {
      {p.dB_part, a->dB, p.batch * p.seqlen * p.ngroups, blocks_per_group, p.dstate},
      {p.dC_part, a->dC, p.batch * p.seqlen * p.ngroups, blocks_per_group, p.dstate},
      {p.dA_part, a->dA, 1, p.batch * p.nchunks, p.nheads},
      {a->ddt_bias ? p.dbias_part : nullptr, a->ddt_bias, 1, p.batch * p.nchunks, p.nheads},
      {a->dD ? p.dD_part : nullptr, a->dD, 1, p.batch * p.nchunks, p.nheads * p.headdim},
  };
  return hip_status(partial_sums_launch(sums, 5, st), "ssd_bwd reduce");
}
