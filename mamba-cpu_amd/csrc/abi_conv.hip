// C-ABI entry points for causal conv1d (forward, backward, decode update) and
// the selective state update: argument checks, workspace layout, launches.
#include <cstring>

#include "abi_util.h"
#include "mcpu_common.h"
#include "op_params.h"

namespace mcpu {

int64_t conv_wide_nseg(int64_t seqlen);

namespace {

int check_conv(const mcpu_conv_args* a) {
  if (a == nullptr) return fail(MCPU_ERR_INVALID, "causal_conv1d: null argument block");
  if (a->batch < 0 || a->dim < 0 || a->seqlen < 0)
    return fail(MCPU_ERR_INVALID, "causal_conv1d: negative size");
  // A tensor with no elements may come as NULL (torch's empty tensors do).
  if ((a->x == nullptr && a->batch * a->dim * a->seqlen > 0) || (a->weight == nullptr && a->dim > 0))
    return fail(MCPU_ERR_INVALID, "causal_conv1d: x and weight are required");
  if (a->width < 1 || a->width > kConvWideMaxW)
    return fail(MCPU_ERR_UNSUPPORTED, "causal_conv1d: width must be in [1, %lld], got %lld",
                (long long)kConvWideMaxW, (long long)a->width);
  if (!valid_dtype(a->dtype)) return fail(MCPU_ERR_INVALID, "causal_conv1d: bad dtype %d", a->dtype);
  if (a->seq_idx != nullptr &&
      (a->initial_states != nullptr || a->final_states != nullptr || a->dfinal_states != nullptr ||
       a->dinitial_states != nullptr))
    return fail(MCPU_ERR_INVALID, "causal_conv1d: seq_idx excludes initial and final states");
  return MCPU_OK;
}

ConvParams make_conv(const mcpu_conv_args* a) {
  ConvParams p;
  std::memset(&p, 0, sizeof(p));
  p.x = a->x;
  p.w = a->weight;
  p.bias = a->bias;
  p.init = a->initial_states;
  p.batch = a->batch;
  p.dim = a->dim;
  p.seqlen = a->seqlen;
  p.width = a->width;
  p.nchunks = (a->seqlen + kConvT - 1) / kConvT;
  p.R = p.nchunks < kConvRMax ? (p.nchunks < 1 ? 1 : p.nchunks) : kConvRMax;
  for (int i = 0; i < 3; ++i) {
    p.sx[i] = a->x_stride[i];
    p.sinit[i] = a->init_stride[i];
    p.sout[i] = a->out_stride[i];
    p.sdo[i] = a->dout_stride[i];
    p.sdx[i] = a->dx_stride[i];
  }
  p.silu = a->silu != 0;
  p.seq_idx = a->seq_idx;
  p.channels_last = (a->x_stride[1] == 1 && a->x_stride[2] != 1) ? 1 : 0;
  return p;
}

// Steps per thread of the time-contiguous fast path: 8 for fp32 (32 bytes of
// each tensor per thread); 16 for 16-bit types where the sequence length
// allows it (measured: fp32 is slower at 16, 16-bit faster).
int conv_vt_steps(int dtype, int64_t seqlen) {
  return (dtype != MCPU_F32 && seqlen % (2 * kConvVTSteps) == 0) ? 2 * kConvVTSteps : kConvVTSteps;
}

// Launch shape of the time-contiguous fast path: `steps` steps per thread; a
// row segment is 64, 128 or 256 threads (one to four whole waves).
void conv_vt_shape(ConvParams& p, int steps) {
  const int64_t threads = p.seqlen / steps;
  if (threads >= 256) {
    p.tpr = 256;
    p.nseg = (threads + 255) / 256;
  } else {
    p.tpr = threads <= 64 ? 64 : (threads <= 128 ? 128 : 256);
    p.nseg = 1;
  }
  p.rpw = 256 / p.tpr;
}

// A (batch, dim, seqlen) operand the fast path can move in vectors: unit time
// stride, rows starting on 4-element boundaries, an aligned base.
bool vt_operand(const void* ptr, const int64_t (&s)[3], int dtype) {
  const uintptr_t align = dtype == MCPU_F32 ? 16 : 8;
  return ptr != nullptr && s[2] == 1 && s[0] % 4 == 0 && s[1] % 4 == 0 &&
         reinterpret_cast<uintptr_t>(ptr) % align == 0;
}

// The fast path's steps per thread (8 or 16), or 0 where it does not apply.
int vt_ok(const ConvParams& p, int dtype, bool bwd) {
  if (p.seq_idx != nullptr) return 0;  // the chunked kernels mask the taps
  const int steps = conv_vt_steps(dtype, p.seqlen);
  if (p.width < 2 || p.width > 5 || p.seqlen < steps || p.seqlen % steps != 0) return 0;
  if (!vt_operand(p.x, p.sx, dtype)) return 0;
  const bool ok = bwd ? vt_operand(p.dout, p.sdo, dtype) && vt_operand(p.dx, p.sdx, dtype)
                      : vt_operand(p.out, p.sout, dtype);
  return ok ? steps : 0;
}

// Launch shape of the channel-contiguous fast path: time segments of 64, 32,
// 16 or 8 steps per wave, the longest that still gives 8192 waves (or 8).
void conv_cl_shape(ConvParams& p) {
  const int64_t tiles = p.batch * ((p.dim + 255) / 256);
  int ng = 8;
  while (ng > 1 && tiles * ((p.seqlen + kConvClG * ng - 1) / (kConvClG * ng)) < 8192) ng /= 2;
  p.cl_ng = ng;
  const int64_t nseg = (p.seqlen + kConvClG * ng - 1) / (kConvClG * ng);
  p.cl_gy = (nseg + 3) / 4;
}

// A (batch, dim, seqlen) operand the channel-contiguous path can move in
// four-channel vectors: unit channel stride, batch and time strides on
// 4-element boundaries, an aligned base.
bool cl_operand(const void* ptr, const int64_t (&s)[3], int dtype) {
  const uintptr_t align = dtype == MCPU_F32 ? 16 : 8;
  return ptr != nullptr && s[1] == 1 && s[0] % 4 == 0 && s[2] % 4 == 0 &&
         reinterpret_cast<uintptr_t>(ptr) % align == 0;
}

// Whether the channel-contiguous path applies (after conv_cl_shape): widths
// 2..5, whole four-channel vectors, no initial states (its kernels read zeros
// before step 0) and, in the backward, no initial- or final-state gradients;
// seq_idx is allowed.
bool cl_ok(const ConvParams& p, int dtype, bool bwd) {
  if (p.width < 2 || p.width > 5 || p.dim % 4 != 0 || p.seqlen < 1) return false;
  if (!p.channels_last || p.batch > 65535 || p.cl_gy > 65535) return false;
  if (p.init != nullptr || !cl_operand(p.x, p.sx, dtype)) return false;
  if (bwd)
    return p.dinit == nullptr && p.dfinal == nullptr && cl_operand(p.dout, p.sdo, dtype) &&
           cl_operand(p.dx, p.sdx, dtype);
  return cl_operand(p.out, p.sout, dtype);
}

// Bytes of the backward's workspace: the dweight/dbias partials, and for
// widths above kConvMaxW the per-element dout * act'(pre) after them.
size_t conv_ws(const ConvParams& p) {
  if (p.width > kConvMaxW)
    return align_up(sizeof(float) * p.batch * conv_wide_nseg(p.seqlen) * p.dim * (p.width + 1)) +
           align_up(sizeof(float) * p.batch * p.dim * p.seqlen);
  ConvParams q = p;
  conv_vt_shape(q, kConvVTSteps);  // the fewest steps per thread: the most segments
  conv_cl_shape(q);
  int64_t parts = q.nseg > p.R ? q.nseg : p.R;
  if (q.cl_gy > parts) parts = q.cl_gy;
  return align_up(sizeof(float) * p.batch * parts * p.dim * (p.width + 1));
}

}  // namespace
}  // namespace mcpu

using namespace mcpu;

extern "C" int mcpu_causal_conv1d_fwd(const mcpu_conv_args* a, void* stream) {
  clear_error();
  if (int rc = check_conv(a)) return rc;
  if (a->out == nullptr && a->batch * a->dim * a->seqlen > 0)
    return fail(MCPU_ERR_INVALID, "causal_conv1d_fwd: out is required");
  if (int rc = mcpu_check_device()) return rc;
  ConvParams p = make_conv(a);
  p.out = a->out;
  p.final_states = a->final_states;
  p.vt = vt_ok(p, a->dtype, false);
  if (p.vt) conv_vt_shape(p, p.vt);
  conv_cl_shape(p);
  p.cl = !p.vt && cl_ok(p, a->dtype, false);
  return hip_status(conv_fwd_launch(p, a->dtype, static_cast<hipStream_t>(stream)),
                    "causal_conv1d_fwd launch");
}

extern "C" size_t mcpu_causal_conv1d_bwd_workspace_size(const mcpu_conv_args* a) {
  if (check_conv(a) != MCPU_OK) {
    clear_error();
    return 0;
  }
  return conv_ws(make_conv(a));
}

extern "C" int mcpu_causal_conv1d_bwd(const mcpu_conv_args* a, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_conv(a)) return rc;
  if (((a->dout == nullptr || a->dx == nullptr) && a->batch * a->dim * a->seqlen > 0) ||
      (a->dweight == nullptr && a->dim > 0))
    return fail(MCPU_ERR_INVALID, "causal_conv1d_bwd: dout, dx and dweight are required");
  if (a->bias != nullptr && a->dbias == nullptr)
    return fail(MCPU_ERR_INVALID, "causal_conv1d_bwd: dbias is required when bias is given");
  ConvParams p = make_conv(a);
  const size_t need = conv_ws(p);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(MCPU_ERR_INVALID, "causal_conv1d_bwd: workspace of %zu bytes needed, got %zu", need,
                workspace_bytes);
  if (int rc = mcpu_check_device()) return rc;
  p.dout = a->dout;
  p.dfinal = a->dfinal_states;
  p.dx = a->dx;
  p.dinit = a->dinitial_states;
  p.dw_part = static_cast<float*>(workspace);
  if (p.width > kConvMaxW)
    p.dpre = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                      align_up(sizeof(float) * p.batch * conv_wide_nseg(p.seqlen) * p.dim *
                                               (p.width + 1)));
  p.vt = vt_ok(p, a->dtype, true);
  if (p.vt) conv_vt_shape(p, p.vt);
  conv_cl_shape(p);
  p.cl = !p.vt && cl_ok(p, a->dtype, true);
  if (a->batch == 0 || a->dim == 0) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (int rc = zero_f32(a->dweight, a->dim * a->width, st)) return rc;
    if (a->dbias) return zero_f32(a->dbias, a->dim, st);
    return MCPU_OK;
  }
  return hip_status(conv_bwd_launch(p, a->dtype, a->dweight, a->dbias, static_cast<hipStream_t>(stream)),
                    "causal_conv1d_bwd launch");
}

extern "C" int mcpu_causal_conv1d_update(const mcpu_conv_update_args* a, void* stream) {
  clear_error();
  if (a == nullptr) return fail(MCPU_ERR_INVALID, "causal_conv1d_update: null argument block");
  if (a->batch < 0 || a->dim < 0 || a->seqlen < 0)
    return fail(MCPU_ERR_INVALID, "causal_conv1d_update: negative size");
  // With no rows (or channels) the tensors may come as NULL.
  if (a->batch * a->dim > 0 &&
      (a->x == nullptr || a->conv_state == nullptr || a->weight == nullptr || a->out == nullptr))
    return fail(MCPU_ERR_INVALID, "causal_conv1d_update: x, conv_state, weight and out are required");
  if (a->width < 1 || a->width > kConvWideMaxW)
    return fail(MCPU_ERR_UNSUPPORTED, "causal_conv1d_update: width must be in [1, %lld]",
                (long long)kConvWideMaxW);
  if (a->state_len < a->width - 1)
    return fail(MCPU_ERR_INVALID, "conv_state length (%lld) must be at least width - 1 (%lld)",
                (long long)a->state_len, (long long)(a->width - 1));
  if (a->cache_seqlens != nullptr && a->state_len < 1)
    return fail(MCPU_ERR_INVALID, "causal_conv1d_update: cache_seqlens needs a conv_state of at least one slot");
  if (!valid_dtype(a->dtype)) return fail(MCPU_ERR_INVALID, "causal_conv1d_update: bad dtype");
  if (int rc = mcpu_check_device()) return rc;
  ConvUpdateParams p;
  std::memset(&p, 0, sizeof(p));
  p.x = a->x;
  p.state = a->conv_state;
  p.w = a->weight;
  p.bias = a->bias;
  p.out = a->out;
  p.batch = a->batch;
  p.dim = a->dim;
  p.seqlen = a->seqlen;
  p.width = a->width;
  p.state_len = a->state_len;
  for (int i = 0; i < 3; ++i) {
    p.sx[i] = a->x_stride[i];
    p.sst[i] = a->state_stride[i];
    p.sout[i] = a->out_stride[i];
  }
  p.silu = a->silu != 0;
  p.cache_seqlens = a->cache_seqlens;
  p.state_idx = a->conv_state_indices;
  p.state_batch = a->state_batch > 0 ? a->state_batch : a->batch;
  if (a->state_batch < 0) return fail(MCPU_ERR_INVALID, "causal_conv1d_update: negative state_batch");
  if (a->conv_state_indices == nullptr && p.state_batch < a->batch)
    return fail(MCPU_ERR_INVALID, "causal_conv1d_update: conv_state has fewer rows than the batch");
  return hip_status(conv_update_launch(p, a->dtype, static_cast<hipStream_t>(stream)),
                    "causal_conv1d_update launch");
}

extern "C" int mcpu_selective_state_update(const mcpu_state_update_args* a, void* stream) {
  clear_error();
  if (a == nullptr) return fail(MCPU_ERR_INVALID, "selective_state_update: null argument block");
  if (a->batch < 0 || a->nheads < 0 || a->headdim < 0)
    return fail(MCPU_ERR_INVALID, "selective_state_update: negative size");
  // With no rows (or channels) the tensors may come as NULL.
  if (a->batch * a->nheads * a->headdim > 0 &&
      (a->state == nullptr || a->x == nullptr || a->dt == nullptr || a->A == nullptr || a->B == nullptr ||
       a->C == nullptr || a->out == nullptr))
    return fail(MCPU_ERR_INVALID, "selective_state_update: state, x, dt, A, B, C and out are required");
  if (a->dstate < 1 || a->dstate > 256)
    return fail(MCPU_ERR_UNSUPPORTED, "selective_state_update: dstate must be in [1, 256]");
  if (a->ngroups < 1 || (a->nheads > 0 && a->nheads % a->ngroups != 0))
    return fail(MCPU_ERR_INVALID, "selective_state_update: nheads must be divisible by ngroups");
  if (!valid_dtype(a->dtype) || !valid_dtype(a->state_dtype))
    return fail(MCPU_ERR_INVALID, "selective_state_update: bad dtype");
  if (a->nheads * a->headdim > 0xffff0000ll)
    return fail(MCPU_ERR_UNSUPPORTED, "selective_state_update: nheads * headdim too large");
  if (a->param_strides != 0 && a->param_strides != 1)
    return fail(MCPU_ERR_INVALID, "selective_state_update: param_strides must be 0 or 1");
  if (int rc = mcpu_check_device()) return rc;
  StateUpdateParams p;
  std::memset(&p, 0, sizeof(p));
  p.state = a->state;
  p.x = a->x;
  p.dt = a->dt;
  p.A = a->A;
  p.B = a->B;
  p.C = a->C;
  p.D = a->D;
  p.z = a->z;
  p.dt_bias = a->dt_bias;
  p.out = a->out;
  p.batch = a->batch;
  p.nheads = a->nheads;
  p.headdim = a->headdim;
  p.dstate = a->dstate;
  p.ngroups = a->ngroups;
  for (int i = 0; i < 3; ++i) {
    p.sst[i] = a->state_stride[i];
    p.sx[i] = a->x_stride[i];
    p.sdt[i] = a->dt_stride[i];
    p.sz[i] = a->z_stride[i];
  }
  for (int i = 0; i < 2; ++i) {
    p.sB[i] = a->B_stride[i];
    p.sC[i] = a->C_stride[i];
  }
  if (a->param_strides) {
    for (int i = 0; i < 3; ++i) p.sA[i] = a->A_stride[i];
    for (int i = 0; i < 2; ++i) {
      p.sD[i] = a->D_stride[i];
      p.sbias[i] = a->dt_bias_stride[i];
    }
  } else {
    p.sA[0] = a->headdim * a->dstate;
    p.sA[1] = a->dstate;
    p.sA[2] = 1;
    p.sD[0] = p.sbias[0] = a->headdim;
    p.sD[1] = p.sbias[1] = 1;
  }
  if (a->state_batch < 0) return fail(MCPU_ERR_INVALID, "selective_state_update: negative state_batch");
  p.state_idx = a->state_batch_indices;
  p.state_batch = a->state_batch > 0 ? a->state_batch : a->batch;
  if (a->state_batch_indices == nullptr && p.state_batch < a->batch)
    return fail(MCPU_ERR_INVALID, "selective_state_update: state has fewer rows than the batch");
  p.softplus = a->dt_softplus != 0;
  return hip_status(state_update_launch(p, a->dtype, a->state_dtype, static_cast<hipStream_t>(stream)),
                    "selective_state_update launch");
}
