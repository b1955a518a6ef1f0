// C-ABI entry points for the selective scan: argument checks, workspace
// layout and kernel sequencing. No allocation happens here; every buffer comes
// from the caller.
#include <cstdio>
#include <cstring>
#include <mutex>

#include "abi_util.h"
#include "scan_common.h"

namespace mcpu {
int scan_fwd_waves();
void scan_fwd_chunks(ScanParams& p);
int scan_bwd_waves(int64_t batch, int64_t ngroups, int64_t dpg, int64_t dstate);
hipError_t scan_fwd_launch(const ScanParams& p, int dtype, bool write_out, hipStream_t stream);
hipError_t scan_bwd_launch(const ScanParams& p, int dtype, int waves, hipStream_t stream);
hipError_t scan_bwd_summary_launch(const ScanParams& p, int dtype, hipStream_t stream);
hipError_t scan_bwd_finish_launch(const ScanParams& p, int dtype, hipStream_t stream);
hipError_t scan_fwd_finish_launch(const ScanParams& p, int dtype, hipStream_t stream);
int scan_complex_waves();
hipError_t scan_cfwd_launch(const ScanParams& p, int dtype, bool write_out, hipStream_t stream);
hipError_t scan_cbwd_launch(const ScanParams& p, int dtype, hipStream_t stream);
hipError_t scan_reduce_launch(const float* dB_part, float* dB, const float* dC_part, float* dC,
                              int64_t slices, int64_t nblk_c, int64_t per_slice,
                              const float* dA_part, float* dA, int64_t nA, const float* dD_part,
                              float* dD, const float* dbias_part, float* dbias, int64_t dim,
                              int64_t batch, hipStream_t stream);

namespace {

// State slices: above kSliceAbove states (what one lane group of the kernels
// holds in registers) the states are cut into slices that the grid scans side
// by side: 64 states per forward slice (four per lane), 16 per backward slice
// (the backward's fastest form). With complex A, whose (re, im) states take
// twice the registers, above kCSlice states in slices of kCSlice, forward and
// backward. Up to kMaxSlicedDstate states.
constexpr int64_t kSliceAbove = 64;
constexpr int64_t kFwdSlice = 64;
constexpr int64_t kBwdSlice = 16;
constexpr int64_t kCSlice = 32;
constexpr int64_t kMaxSlicedDstate = 4096;

int64_t slices_of(int64_t dstate, int64_t slice, int64_t above = kSliceAbove) {
  return dstate > above ? (dstate + slice - 1) / slice : 1;
}

// Cuts p (made for all states) into slices of `slice` states when sliced.
void slice_params(ScanParams& p, int64_t slice, int64_t above = kSliceAbove) {
  const int64_t ns = slices_of(p.ntotal, slice, above);
  if (ns > 1) {
    p.dstate = slice;
    p.nslices = ns;
  }
}

// An output's strides as given, or contiguous (batch, dim, seqlen) when all zero.
void out_strides(const int64_t (&given)[3], int64_t dim, int64_t seqlen, int64_t (&s)[3]) {
  const bool none = given[0] == 0 && given[1] == 0 && given[2] == 0;
  s[0] = none ? dim * seqlen : given[0];
  s[1] = none ? seqlen : given[1];
  s[2] = none ? 1 : given[2];
}

int check_scan(const mcpu_scan_args* a) {
  if (a == nullptr) return fail(MCPU_ERR_INVALID, "selective_scan: null argument block");
  if (a->batch < 0 || a->dim < 0 || a->seqlen < 0)
    return fail(MCPU_ERR_INVALID, "selective_scan: negative size");
  // A tensor with no elements may come as NULL (torch's empty tensors do).
  const bool has_steps = a->batch > 0 && a->dim > 0 && a->seqlen > 0;
  if ((has_steps && (a->u == nullptr || a->delta == nullptr || a->B == nullptr || a->C == nullptr)) ||
      (a->dim > 0 && a->A == nullptr))
    return fail(MCPU_ERR_INVALID, "selective_scan: u, delta, A, B and C are required");
  if (a->ngroups < 1 || (a->dim > 0 && a->dim % a->ngroups != 0))
    return fail(MCPU_ERR_INVALID, "selective_scan: dim (%lld) must be divisible by ngroups (%lld)",
                (long long)a->dim, (long long)a->ngroups);
  if (a->dstate < 1 || a->dstate > kMaxSlicedDstate)
    return fail(MCPU_ERR_UNSUPPORTED, "selective_scan: dstate must be in [1, %lld], got %lld",
                (long long)kMaxSlicedDstate, (long long)a->dstate);
  if (!valid_dtype(a->dtype)) return fail(MCPU_ERR_INVALID, "selective_scan: bad dtype %d", a->dtype);
  if (a->bwd_waves != 0 &&
      (a->complex_a || a->dstate > 16 || (a->bwd_waves != 4 && a->bwd_waves != 8 && a->bwd_waves != 12)))
    return fail(MCPU_ERR_INVALID, "selective_scan: bwd_waves must be 0, or 4, 8 or 12 with real A "
                "and dstate <= 16, got %d", a->bwd_waves);
  const int64_t dpg = a->dim / a->ngroups;
  const int64_t blocks = a->batch * a->ngroups * ((dpg + 15) / 16) *
                        (a->complex_a ? slices_of(a->dstate, kCSlice, kCSlice) : slices_of(a->dstate, kBwdSlice));
  if (blocks > 0x7fffffffll) return fail(MCPU_ERR_UNSUPPORTED, "selective_scan: grid too large");
  for (int i = 0; i < 3; ++i)
    if (a->u_stride[i] < 0 || a->delta_stride[i] < 0 || a->z_stride[i] < 0 || a->dout_stride[i] < 0 ||
        a->out_stride[i] < 0 || a->du_stride[i] < 0 || a->ddelta_stride[i] < 0 || a->dz_stride[i] < 0)
      return fail(MCPU_ERR_INVALID, "selective_scan: negative stride");
  int64_t so[3], sdu[3], sdd[3], sdz[3];
  out_strides(a->out_stride, a->dim, a->seqlen, so);
  out_strides(a->du_stride, a->dim, a->seqlen, sdu);
  out_strides(a->ddelta_stride, a->dim, a->seqlen, sdd);
  out_strides(a->dz_stride, a->dim, a->seqlen, sdz);
  for (int i = 0; i < 4; ++i)
    if (a->B_stride[i] < 0 || a->C_stride[i] < 0)
      return fail(MCPU_ERR_INVALID, "selective_scan: negative stride");
  // The kernels address a thread's element within one (channels x 16 steps)
  // tile with a 32-bit byte offset from the tile's base.
  const int64_t esz = dtype_size(a->dtype), ch = 4 * kScanMaxWaves - 1, T = kScanBlockT - 1;
  const int64_t nblk = (a->seqlen + kScanBlockT - 1) / kScanBlockT;
  auto x_span = [&](const int64_t (&s)[3]) { return esz * (ch * s[1] + T * s[2]); };
  const int64_t cw = a->complex_a ? 2 : 1;  // floats per state element
  auto bc_span = [&](const int64_t (&s)[4]) { return 4 * (T * s[2] + 63 * s[3] + cw - 1); };
  const int64_t spans[] = {x_span(a->u_stride), x_span(a->delta_stride), x_span(a->z_stride),
                           x_span(a->dout_stride), bc_span(a->B_stride), bc_span(a->C_stride),
                           4 * cw * (ch * nblk * a->dstate + 63), esz * (ch * a->seqlen + T),
                           x_span(so), x_span(sdu), x_span(sdd), x_span(sdz)};
  for (int64_t sp : spans)
    if (sp >= 0xffffffffll)
      return fail(MCPU_ERR_UNSUPPORTED, "selective_scan: strides or sizes too large for 32-bit tile offsets");
  // The staging cursors move by one 16-step block as a signed 32-bit byte step.
  const int64_t steps[] = {esz * kScanBlockT * a->u_stride[2], esz * kScanBlockT * a->delta_stride[2],
                           esz * kScanBlockT * a->z_stride[2], esz * kScanBlockT * a->dout_stride[2],
                           4 * kScanBlockT * a->B_stride[2], 4 * kScanBlockT * a->C_stride[2],
                           esz * kScanBlockT * so[2], esz * kScanBlockT * sdu[2],
                           esz * kScanBlockT * sdd[2], esz * kScanBlockT * sdz[2]};
  for (int64_t st : steps)
    if (st > 0x7fffffffll)
      return fail(MCPU_ERR_UNSUPPORTED, "selective_scan: time stride too large for 32-bit block steps");
  return MCPU_OK;
}

// Kernel parameters for a launch with `waves` waves per workgroup.
ScanParams make_params(const mcpu_scan_args* a, int waves) {
  ScanParams p;
  std::memset(&p, 0, sizeof(p));
  p.u = a->u;
  p.delta = a->delta;
  p.A = a->A;
  p.B = a->B;
  p.C = a->C;
  p.D = a->D;
  p.z = a->z;
  p.delta_bias = a->delta_bias;
  p.batch = a->batch;
  p.dim = a->dim;
  p.seqlen = a->seqlen;
  p.dstate = a->dstate;
  p.ngroups = a->ngroups;
  p.dpg = a->dim / a->ngroups;
  p.nblk = (a->seqlen + kScanBlockT - 1) / kScanBlockT;
  p.nblk_c = (p.dpg + 4 * waves - 1) / (4 * waves);
  for (int i = 0; i < 3; ++i) {
    p.su[i] = a->u_stride[i];
    p.sdl[i] = a->delta_stride[i];
    p.sz[i] = a->z_stride[i];
    p.sdo[i] = a->dout_stride[i];
  }
  out_strides(a->out_stride, a->dim, a->seqlen, p.sout);
  out_strides(a->du_stride, a->dim, a->seqlen, p.sdu);
  out_strides(a->ddelta_stride, a->dim, a->seqlen, p.sdd);
  out_strides(a->dz_stride, a->dim, a->seqlen, p.sdz);
  for (int i = 0; i < 4; ++i) {
    p.sB[i] = a->B_stride[i];
    p.sC[i] = a->C_stride[i];
  }
  p.softplus = a->delta_softplus != 0;
  p.nchunk = 1;
  p.chunk_blocks = p.nblk > 0 ? p.nblk : 1;
  p.nslices = 1;
  p.nstride = p.ntotal = a->dstate;
  return p;
}

// Forward parameters: sliced when dstate needs it, chunked by the shape.
ScanParams fwd_params(const mcpu_scan_args* a) {
  ScanParams p = make_params(a, scan_fwd_waves());
  slice_params(p, kFwdSlice);
  scan_fwd_chunks(p);
  return p;
}

// Workspace of a forward: chunk-end states and chunk sums of dt when
// chunked; each slice's share of y when sliced and writing outputs.
struct FwdLayout {
  size_t sum_h = 0, sum_dt = 0, ypart = 0, total = 0;
};

FwdLayout fwd_layout(const ScanParams& p, bool write_out) {
  FwdLayout w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  if (p.nchunk > 1) {
    w.sum_h = take(sizeof(float) * p.batch * p.dim * p.nchunk * p.ntotal);
    w.sum_dt = take(sizeof(float) * p.batch * p.dim * p.nchunk);
  }
  if (p.nslices > 1 && write_out) w.ypart = take(sizeof(float) * p.nslices * p.batch * p.dim * p.seqlen);
  w.total = off;
  return w;
}

// The backward's workgroup width: pinned by the caller (bwd_waves, checked by
// check_scan) or chosen from the shape (a sliced backward's slices count as
// more batch rows of kBwdSlice states).
int bwd_waves(const mcpu_scan_args* a) {
  if (a->bwd_waves != 0) return a->bwd_waves;
  const int64_t ns = slices_of(a->dstate, kBwdSlice);
  return scan_bwd_waves(a->batch * ns, a->ngroups, a->dim / a->ngroups, ns > 1 ? kBwdSlice : a->dstate);
}

// Time chunks of a backward with these parameters: when the rows give fewer
// than two waves per SIMD of the GPU's 1024, the sequence is cut into chunks
// (at least four 16-step blocks each) so that about four waves per SIMD run,
// the most that fit at the backward's register use, and chunks hold at most
// 64 blocks (measured: batch 1, dim 5120, seqlen 16384 bf16 takes 1.33 ms at
// 16 chunks against 1.40 ms at 3). Two chunks of a sequence of at most 16
// blocks are not worth their summary pass (batch 4, dim 1536, 256 steps fp32
// with z: 49.8 us in one chunk against 53.0 us in two). Sets p.nchunk /
// p.chunk_blocks.
void bwd_chunks(ScanParams& p, int waves) {
  int64_t n = 1;
  const int64_t wv = p.batch * p.ngroups * p.nblk_c * waves * p.nslices;
  if (wv > 0 && wv < 2048 && p.nblk >= 8) {
    n = 4096 / wv;  // about four waves per SIMD, the register limit of the kernel
    if (n < p.nblk / 64) n = p.nblk / 64;  // chunks of at most 64 blocks
    if (n > p.nblk / 4) n = p.nblk / 4;
    if (n < 1) n = 1;
    if (n == 2 && p.nblk <= 16) n = 1;
  }
  p.chunk_blocks = n > 1 ? (p.nblk + n - 1) / n : (p.nblk > 0 ? p.nblk : 1);
  p.nchunk = n > 1 ? (p.nblk + p.chunk_blocks - 1) / p.chunk_blocks : 1;
  p.nsum = p.nchunk;
  p.sum_blocks = p.chunk_blocks;
  p.sum_per_chunk = 1;
  if (p.nchunk > 1) {
    // Summary units: enough of them after the first chunk for about four
    // waves per SIMD in the summary pass; chunks are whole units.
    int64_t m = (4096 + wv * (p.nchunk - 1) - 1) / (wv * (p.nchunk - 1));
    if (m > p.chunk_blocks) m = p.chunk_blocks;
    if (m < 1) m = 1;
    p.sum_blocks = (p.chunk_blocks + m - 1) / m;
    p.chunk_blocks = p.sum_blocks * m;
    p.nchunk = (p.nblk + p.chunk_blocks - 1) / p.chunk_blocks;
    p.nsum = (p.nblk + p.sum_blocks - 1) / p.sum_blocks;
    p.sum_per_chunk = m;
  }
}

// A sliced backward also needs: each slice's <ga, A> and <g, B> shares
// (rpart), y before the gate when z is given and the caller saved none
// (ysave, the input dtype), and for the forward that makes it (or the
// checkpoints), that forward's own workspace (fwd).
struct BwdLayout {
  size_t ckpt = 0, dB = 0, dC = 0, dA = 0, dD = 0, dbias = 0, sum_h = 0, sum_dt = 0;
  size_t rpart = 0, ysave = 0, fwd = 0, fwd_bytes = 0, total = 0;
  bool own_ckpt = false, part_bc = false, part_dA = false, own_ysave = false, sliced = false;
  int64_t nchunk = 1, chunk_blocks = 1, nsum = 1, sum_blocks = 1, sum_per_chunk = 1;
};

BwdLayout bwd_layout(const mcpu_scan_args* a) {
  ScanParams p = make_params(a, bwd_waves(a));
  slice_params(p, kBwdSlice);
  bwd_chunks(p, bwd_waves(a));
  BwdLayout w;
  w.nchunk = p.nchunk;
  w.chunk_blocks = p.chunk_blocks;
  w.nsum = p.nsum;
  w.sum_blocks = p.sum_blocks;
  w.sum_per_chunk = p.sum_per_chunk;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  w.own_ckpt = a->ckpt == nullptr;
  if (w.own_ckpt) w.ckpt = take(sizeof(float) * p.batch * p.dim * p.nblk * p.ntotal);
  w.part_bc = p.nblk_c > 1;
  if (w.part_bc) {
    const size_t bc = sizeof(float) * p.batch * p.ngroups * p.nblk_c * p.seqlen * p.ntotal;
    w.dB = take(bc);
    w.dC = take(bc);
  }
  // dA, dD and ddelta_bias partials per (chunk, batch).
  const int64_t parts = p.batch * p.nchunk;
  w.part_dA = parts > 1;
  if (w.part_dA) w.dA = take(sizeof(float) * parts * p.dim * p.ntotal);
  w.dD = take(sizeof(float) * parts * p.dim);
  w.dbias = take(sizeof(float) * parts * p.dim);
  if (p.nchunk > 1) {
    w.sum_h = take(sizeof(float) * p.batch * p.dim * p.nsum * p.ntotal);
    w.sum_dt = take(sizeof(float) * p.batch * p.dim * p.nsum);
  }
  w.sliced = p.nslices > 1;
  if (w.sliced) {
    const int64_t n = p.batch * p.dim * p.seqlen;
    w.rpart = take(sizeof(float) * 2 * p.nslices * n);
    w.own_ysave = a->z != nullptr && (a->ckpt == nullptr || a->ysave == nullptr);
    if (w.own_ysave) w.ysave = take(dtype_size(a->dtype) * n);
    if (w.own_ckpt || w.own_ysave) {
      w.fwd_bytes = fwd_layout(fwd_params(a), w.own_ysave).total;
      w.fwd = take(w.fwd_bytes);
    }
  } else if (w.own_ckpt) {
    // The states-only forward that makes the checkpoints runs with the
    // forward's own time chunks (its chunk summaries go here), so that its
    // checkpoints are bit-identical to those a forward call saves.
    w.fwd_bytes = fwd_layout(fwd_params(a), false).total;
    if (w.fwd_bytes > 0) w.fwd = take(w.fwd_bytes);
  }
  w.total = off;
  return w;
}

// Complex A: one time chunk, 4-wave workgroups, states as (re, im) pairs;
// above kCSlice states, kCSlice-state slices (the forward's shares of y and
// the backward's shares of its two state sums go through the workspace and
// the real scan's finish kernels).
ScanParams cparams(const mcpu_scan_args* a) {
  ScanParams p = make_params(a, scan_complex_waves());
  slice_params(p, kCSlice, kCSlice);
  return p;
}

// A sliced complex forward's workspace: the slices' shares of y.
size_t cfwd_bytes(const ScanParams& p, bool write_out) {
  return p.nslices > 1 && write_out ? align_up(sizeof(float) * p.nslices * p.batch * p.dim * p.seqlen) : 0;
}

struct CBwdLayout {
  size_t ckpt = 0, dB = 0, dC = 0, dA = 0, dD = 0, dbias = 0, rpart = 0, ysave = 0, fwd = 0, total = 0;
  bool own_ckpt = false, part_bc = false, part_dA = false, sliced = false, own_ysave = false;
};

CBwdLayout cbwd_layout(const mcpu_scan_args* a) {
  const ScanParams p = cparams(a);
  CBwdLayout w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  w.own_ckpt = a->ckpt == nullptr;
  if (w.own_ckpt) w.ckpt = take(sizeof(float) * 2 * p.batch * p.dim * p.nblk * p.ntotal);
  w.part_bc = p.nblk_c > 1;
  if (w.part_bc) {
    const size_t bc = sizeof(float) * 2 * p.batch * p.ngroups * p.nblk_c * p.seqlen * p.ntotal;
    w.dB = take(bc);
    w.dC = take(bc);
  }
  w.part_dA = p.batch > 1;
  if (w.part_dA) w.dA = take(sizeof(float) * 2 * p.batch * p.dim * p.ntotal);
  w.dD = take(sizeof(float) * p.batch * p.dim);
  w.dbias = take(sizeof(float) * p.batch * p.dim);
  w.sliced = p.nslices > 1;
  if (w.sliced) {
    w.rpart = take(sizeof(float) * 2 * p.nslices * p.batch * p.dim * p.seqlen);
    // y before the gate for dz: the caller's (with its checkpoints) or made here
    w.own_ysave = a->z != nullptr && (a->ckpt == nullptr || a->ysave == nullptr);
    if (w.own_ysave) {
      w.ysave = take(dtype_size(a->dtype) * p.batch * p.dim * p.seqlen);
      w.fwd = take(cfwd_bytes(p, true));
    }
  }
  w.total = off;
  return w;
}

// The forward: scan_cfwd_kernel, and for a sliced one writing outputs its
// slices' shares of y (workspace) and then scan_fwd_finish_kernel.
int complex_fwd_run(ScanParams p, bool write_out, float* ypart, int dtype, hipStream_t st, const char* what) {
  if (p.nslices > 1 && write_out) {
    ScanParams ps = p;
    ps.ypart = ypart;
    ps.D = nullptr;
    ps.z = nullptr;
    ps.ysave = nullptr;
    if (int rc = hip_status(scan_cfwd_launch(ps, dtype, true, st), what)) return rc;
    p.ypart = ypart;
    return hip_status(scan_fwd_finish_launch(p, dtype, st), what);
  }
  return hip_status(scan_cfwd_launch(p, dtype, write_out, st), what);
}

int complex_fwd(const mcpu_scan_args* a, void* workspace, size_t workspace_bytes, hipStream_t st) {
  ScanParams p = cparams(a);
  p.out = a->out;
  p.last_state = a->last_state;
  p.ckpt = a->ckpt;
  p.ysave = a->out != nullptr ? a->ysave : nullptr;
  if (p.out == nullptr && p.last_state == nullptr && p.ckpt == nullptr) return MCPU_OK;
  const size_t need = cfwd_bytes(p, a->out != nullptr);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(MCPU_ERR_INVALID, "selective_scan_fwd: complex dstate %lld needs a workspace of %zu bytes, got %zu",
                (long long)a->dstate, need, workspace_bytes);
  return complex_fwd_run(p, a->out != nullptr, static_cast<float*>(workspace), a->dtype, st,
                         "selective_scan_fwd launch");
}

int complex_bwd(const mcpu_scan_args* a, void* workspace, size_t workspace_bytes, hipStream_t st) {
  const CBwdLayout w = cbwd_layout(a);
  if (w.total > 0 && (workspace == nullptr || workspace_bytes < w.total))
    return fail(MCPU_ERR_INVALID, "selective_scan_bwd: workspace of %zu bytes needed, got %zu",
                w.total, workspace_bytes);
  if (int rc = mcpu_check_device()) return rc;
  if (a->batch == 0 || a->dim == 0 || a->seqlen == 0) {
    // Nothing to scan: parameter grads are zero (dB/dC, du, ... are empty
    // unless seqlen is 0 with a nonempty batch, where they have no elements).
    if (int rc = zero_f32(a->dA, 2 * a->dim * a->dstate, st)) return rc;
    if (a->dD) if (int rc = zero_f32(a->dD, a->dim, st)) return rc;
    if (a->ddelta_bias) if (int rc = zero_f32(a->ddelta_bias, a->dim, st)) return rc;
    return MCPU_OK;
  }
  char* ws = static_cast<char*>(workspace);
  ScanParams p = cparams(a);
  p.ckpt = w.own_ckpt ? reinterpret_cast<float*>(ws + w.ckpt) : a->ckpt;
  p.ysave = w.sliced && a->z != nullptr ? (w.own_ysave ? ws + w.ysave : a->ysave) : nullptr;
  if (w.own_ckpt || w.own_ysave) {
    // The forward for the block checkpoints and/or (sliced, with z) y before
    // the gate.
    ScanParams pf = p;
    pf.ckpt = w.own_ckpt ? p.ckpt : nullptr;
    if (int rc = complex_fwd_run(pf, w.own_ysave, reinterpret_cast<float*>(ws + w.fwd), a->dtype, st,
                                 "selective_scan_bwd fwd launch"))
      return rc;
  }
  p.dout = a->dout;
  p.dlast_state = a->dlast_state;
  p.du = a->du;
  p.ddelta = a->ddelta;
  p.dz = a->dz;
  p.dB_part = w.part_bc ? reinterpret_cast<float*>(ws + w.dB) : a->dB;
  p.dC_part = w.part_bc ? reinterpret_cast<float*>(ws + w.dC) : a->dC;
  p.dA_part = w.part_dA ? reinterpret_cast<float*>(ws + w.dA) : a->dA;
  p.dD_part = reinterpret_cast<float*>(ws + w.dD);
  p.dbias_part = reinterpret_cast<float*>(ws + w.dbias);
  if (w.sliced) p.rpart = reinterpret_cast<float*>(ws + w.rpart);
  if (int rc = hip_status(scan_cbwd_launch(p, a->dtype, st), "selective_scan_bwd launch")) return rc;
  if (w.sliced) {
    // du, ddelta, dz and the dD / ddelta_bias batch partials from the slices'
    // shares, then the partials as for one slice.
    if (int rc = hip_status(scan_bwd_finish_launch(p, a->dtype, st), "selective_scan_bwd finish launch"))
      return rc;
  }
  return hip_status(
      scan_reduce_launch(w.part_bc ? p.dB_part : nullptr, a->dB, w.part_bc ? p.dC_part : nullptr,
                         a->dC, p.batch * p.ngroups, p.nblk_c, 2 * p.seqlen * p.ntotal,
                         w.part_dA ? p.dA_part : nullptr, a->dA, 2 * p.dim * p.ntotal,
                         a->dD ? p.dD_part : nullptr, a->dD,
                         a->ddelta_bias ? p.dbias_part : nullptr, a->ddelta_bias, p.dim, p.batch, st),
      "selective_scan_bwd reduce");
}

}  // namespace
}  // namespace mcpu

using namespace mcpu;

extern "C" size_t mcpu_selective_scan_ckpt_size(const mcpu_scan_args* a) {
  if (a == nullptr || a->batch < 0 || a->dim < 0 || a->seqlen < 0 || a->dstate < 0) return 0;
  const int64_t nblk = (a->seqlen + kScanBlockT - 1) / kScanBlockT;
  return sizeof(float) * a->batch * a->dim * nblk * a->dstate * (a->complex_a ? 2 : 1);
}

extern "C" size_t mcpu_selective_scan_fwd_workspace_size(const mcpu_scan_args* a) {
  if (check_scan(a) != MCPU_OK) {
    clear_error();
    return 0;
  }
  if (a->complex_a) return cfwd_bytes(cparams(a), a->out != nullptr);
  return fwd_layout(fwd_params(a), a->out != nullptr).total;
}

extern "C" int mcpu_selective_scan_fwd(const mcpu_scan_args* a, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_scan(a)) return rc;
  if (int rc = mcpu_check_device()) return rc;
  if (a->batch == 0 || a->dim == 0) return MCPU_OK;
  if (a->seqlen == 0) {  // no steps: the state stays at its zero start
    if (a->last_state == nullptr) return MCPU_OK;
    return zero_f32(a->last_state, (a->complex_a ? 2 : 1) * a->batch * a->dim * a->dstate,
                    static_cast<hipStream_t>(stream));
  }
  if (a->complex_a) return complex_fwd(a, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  ScanParams p = fwd_params(a);
  const bool write_out = a->out != nullptr;
  FwdLayout w = fwd_layout(p, write_out);
  char* ws = static_cast<char*>(workspace);
  if (p.nslices > 1 && write_out) {
    // A sliced forward cannot do without the slices' shares of y.
    if (workspace == nullptr || workspace_bytes < w.total)
      return fail(MCPU_ERR_INVALID, "selective_scan_fwd: dstate %lld needs a workspace of %zu bytes, got %zu",
                  (long long)a->dstate, w.total, workspace_bytes);
    p.ypart = reinterpret_cast<float*>(ws + w.ypart);
  }
  if (p.nchunk > 1 && workspace != nullptr && workspace_bytes >= w.total) {
    p.sum_h = reinterpret_cast<float*>(ws + w.sum_h);
    p.sum_dt = reinterpret_cast<float*>(ws + w.sum_dt);
  } else {
    // Without the workspace the sequence is scanned in one chunk.
    p.nchunk = 1;
    p.chunk_blocks = p.nblk > 0 ? p.nblk : 1;
  }
  p.out = a->out;
  p.last_state = a->last_state;
  p.ckpt = a->ckpt;
  p.ysave = a->out != nullptr ? a->ysave : nullptr;
  if (p.out == nullptr && p.last_state == nullptr && p.ckpt == nullptr) return MCPU_OK;
  return hip_status(scan_fwd_launch(p, a->dtype, a->out != nullptr, static_cast<hipStream_t>(stream)),
                    "selective_scan_fwd launch");
}

extern "C" size_t mcpu_selective_scan_bwd_workspace_size(const mcpu_scan_args* a) {
  if (check_scan(a) != MCPU_OK) {
    clear_error();
    return 0;
  }
  return a->complex_a ? cbwd_layout(a).total : bwd_layout(a).total;
}

extern "C" int mcpu_selective_scan_bwd(const mcpu_scan_args* a, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = check_scan(a)) return rc;
  const bool has_steps = a->batch > 0 && a->dim > 0 && a->seqlen > 0;
  if ((has_steps && (a->du == nullptr || a->ddelta == nullptr || a->dB == nullptr || a->dC == nullptr)) ||
      (a->dim > 0 && a->dA == nullptr))
    return fail(MCPU_ERR_INVALID, "selective_scan_bwd: du, ddelta, dA, dB and dC are required");
  if (a->z != nullptr && a->dz == nullptr)
    return fail(MCPU_ERR_INVALID, "selective_scan_bwd: dz is required when z is given");
  if (a->D != nullptr && a->dD == nullptr)
    return fail(MCPU_ERR_INVALID, "selective_scan_bwd: dD is required when D is given");
  if (a->delta_bias != nullptr && a->ddelta_bias == nullptr)
    return fail(MCPU_ERR_INVALID, "selective_scan_bwd: ddelta_bias is required when delta_bias is given");
  if (a->complex_a) return complex_bwd(a, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
  const BwdLayout w = bwd_layout(a);
  if (w.total > 0 && (workspace == nullptr || workspace_bytes < w.total))
    return fail(MCPU_ERR_INVALID, "selective_scan_bwd: workspace of %zu bytes needed, got %zu",
                w.total, workspace_bytes);
  if (int rc = mcpu_check_device()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!has_steps) {
    // No steps or rows: every per-step gradient is empty and the parameter
    // gradients are zero.
    if (int rc = zero_f32(a->dA, a->dim * a->dstate, st)) return rc;
    if (a->dD) if (int rc = zero_f32(a->dD, a->dim, st)) return rc;
    if (a->ddelta_bias) if (int rc = zero_f32(a->ddelta_bias, a->dim, st)) return rc;
    return MCPU_OK;
  }
  char* ws = static_cast<char*>(workspace);
  const int waves = bwd_waves(a);
  ScanParams p = make_params(a, waves);
  slice_params(p, kBwdSlice);
  p.ckpt = w.own_ckpt ? reinterpret_cast<float*>(ws + w.ckpt) : a->ckpt;
  p.ysave = (a->z != nullptr && a->ckpt != nullptr) ? a->ysave : nullptr;
  if (w.sliced) {
    if (a->z != nullptr && w.own_ysave) p.ysave = ws + w.ysave;
    p.rpart = reinterpret_cast<float*>(ws + w.rpart);
    if (w.own_ckpt || w.own_ysave) {
      // The sliced forward for the checkpoints and/or y before the gate.
      ScanParams pf = fwd_params(a);
      const FwdLayout fw = fwd_layout(pf, w.own_ysave);
      char* fws = ws + w.fwd;
      if (pf.nchunk > 1) {
        pf.sum_h = reinterpret_cast<float*>(fws + fw.sum_h);
        pf.sum_dt = reinterpret_cast<float*>(fws + fw.sum_dt);
      }
      if (w.own_ysave) {
        pf.ypart = reinterpret_cast<float*>(fws + fw.ypart);
        pf.ysave = p.ysave;
      }
      pf.ckpt = w.own_ckpt ? p.ckpt : nullptr;
      if (int rc = hip_status(scan_fwd_launch(pf, a->dtype, w.own_ysave, st), "selective_scan_bwd fwd launch"))
        return rc;
    }
  } else if (w.own_ckpt) {
    // States-only forward for the block checkpoints, time-chunked as a
    // forward call is.
    ScanParams pf = fwd_params(a);
    pf.ckpt = p.ckpt;
    if (pf.nchunk > 1) {
      const FwdLayout fw = fwd_layout(pf, false);
      pf.sum_h = reinterpret_cast<float*>(ws + w.fwd + fw.sum_h);
      pf.sum_dt = reinterpret_cast<float*>(ws + w.fwd + fw.sum_dt);
    }
    if (int rc = hip_status(scan_fwd_launch(pf, a->dtype, false, st), "selective_scan_bwd ckpt launch"))
      return rc;
  }
  p.dout = a->dout;
  p.dlast_state = a->dlast_state;
  p.du = a->du;
  p.ddelta = a->ddelta;
  p.dz = a->dz;
  p.dB_part = w.part_bc ? reinterpret_cast<float*>(ws + w.dB) : a->dB;
  p.dC_part = w.part_bc ? reinterpret_cast<float*>(ws + w.dC) : a->dC;
  p.dA_part = w.part_dA ? reinterpret_cast<float*>(ws + w.dA) : a->dA;
  p.dD_part = reinterpret_cast<float*>(ws + w.dD);
  p.dbias_part = reinterpret_cast<float*>(ws + w.dbias);
  p.nchunk = w.nchunk;
  p.chunk_blocks = w.chunk_blocks;
  p.nsum = w.nsum;
  p.sum_blocks = w.sum_blocks;
  p.sum_per_chunk = w.sum_per_chunk;
  if (p.nchunk > 1) {
    // Chunked: the adjoint summaries of chunks 1.. first.
    p.sum_h = reinterpret_cast<float*>(ws + w.sum_h);
    p.sum_dt = reinterpret_cast<float*>(ws + w.sum_dt);
    // The summary kernel's workgroups are kScanSumWaves waves (channel blocks
    // of 4 * kScanSumWaves), whatever the main kernel's width.
    ScanParams ps = p;
    ps.nblk_c = (p.dpg + 4 * kScanSumWaves - 1) / (4 * kScanSumWaves);
    if (int rc = hip_status(scan_bwd_summary_launch(ps, a->dtype, st), "selective_scan_bwd summary launch"))
      return rc;
  }
  if (int rc = hip_status(scan_bwd_launch(p, a->dtype, waves, st), "selective_scan_bwd launch"))
    return rc;
  if (w.sliced) {
    // du, ddelta, dz and the dD / ddelta_bias batch partials from the slices'
    // shares; then dB/dC over channel blocks, dA over (chunk, batch) and
    // dD / ddelta_bias over the batch.
    if (int rc = hip_status(scan_bwd_finish_launch(p, a->dtype, st), "selective_scan_bwd finish launch"))
      return rc;
    if (int rc = hip_status(
            scan_reduce_launch(w.part_bc ? p.dB_part : nullptr, a->dB, w.part_bc ? p.dC_part : nullptr, a->dC,
                               p.batch * p.ngroups, p.nblk_c, p.seqlen * p.ntotal,
                               w.part_dA ? p.dA_part : nullptr, a->dA, p.dim * p.ntotal, nullptr, nullptr,
                               nullptr, nullptr, p.dim, p.batch * p.nchunk, st),
            "selective_scan_bwd reduce"))
      return rc;
    return hip_status(scan_reduce_launch(nullptr, nullptr, nullptr, nullptr, 0, 1, 0, nullptr, nullptr, 0,
                                         a->dD ? p.dD_part : nullptr, a->dD,
                                         a->ddelta_bias ? p.dbias_part : nullptr, a->ddelta_bias, p.dim,
                                         p.batch, st),
                      "selective_scan_bwd reduce");
  }
  // One launch sums every partial: dB/dC over channel blocks (when there is
  // more than one), dA/dD/ddelta_bias over the batch.
  return hip_status(
      scan_reduce_launch(w.part_bc ? p.dB_part : nullptr, a->dB, w.part_bc ? p.dC_part : nullptr,
                         a->dC, p.batch * p.ngroups, p.nblk_c, p.seqlen * p.ntotal,
                         w.part_dA ? p.dA_part : nullptr, a->dA, p.dim * p.ntotal,
                         a->dD ? p.dD_part : nullptr, a->dD,
                         a->ddelta_bias ? p.dbias_part : nullptr, a->ddelta_bias, p.dim,
                         p.batch * p.nchunk, st),
      "selective_scan_bwd reduce");
}

// ---- backward without allocation ------------------------------------------

namespace mcpu {

// Scratch of mcpu_selective_scan_bwd_noalloc, in place of a caller workspace.
// Each device holds its own copy; host code must use the address
// hipGetSymbolAddress returns for the current device, never this name.
static __device__ __align__(256) unsigned char scratch[MCPU_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices];  // device address of `scratch` per device, once looked up

// The current device's copy of `scratch`, looked up on the first call on
// that device (with it current) and kept for the process.
int scratch_address(void** out) {
  int dev = 0;
  if (int rc = hip_status(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kScratchDevices)
    return fail(MCPU_ERR_UNSUPPORTED, "selective_scan_bwd_noalloc: device index %d beyond %d", dev,
                kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (int rc = hip_status(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)),
                            "selective_scan_bwd_noalloc: hipGetSymbolAddress"))
      return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MCPU_OK;
}

}  // namespace
}  // namespace mcpu

extern "C" int mcpu_selective_scan_bwd_noalloc(const mcpu_scan_args* a, void* stream) {
  clear_error();
  if (int rc = check_scan(a)) return rc;
  const size_t need = a->complex_a ? cbwd_layout(a).total : bwd_layout(a).total;
  if (need > MCPU_NOALLOC_SCRATCH_BYTES)
    return fail(MCPU_ERR_UNSUPPORTED,
                "selective_scan_bwd_noalloc: needs %zu bytes of scratch, the library's array holds %zu; "
                "use mcpu_selective_scan_bwd with a workspace",
                need, (size_t)MCPU_NOALLOC_SCRATCH_BYTES);
  if (int rc = mcpu_check_device()) return rc;
  void* ws = nullptr;
  if (need > 0)
    if (int rc = scratch_address(&ws)) return rc;
  return mcpu_selective_scan_bwd(a, ws, need > 0 ? (size_t)MCPU_NOALLOC_SCRATCH_BYTES : 0, stream);
}
