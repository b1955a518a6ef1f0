/* mamba_hip.h — C ABI of the MI355X (gfx950) Mamba-1 op library libmamba_hip.so.
 *
 * Plain C: raw device pointers, element strides, sizes and a HIP stream passed
 * as `void*` (a hipStream_t; NULL = the null stream). No torch types. Every
 * entry point is asynchronous on the given stream, allocates no memory and
 * returns MCPU_OK or an error code; mcpu_last_error() then describes it.
 * The caller owns every buffer, including workspaces sized by the matching
 * *_workspace_size query (the reference's caller-owns-memory rule,
 * csrc/selective_scan.h:14-20, 42-50). A tensor with no elements (zero steps,
 * rows or channels) may be passed as NULL, as torch's empty tensors are.
 *
 * Storage types: "x-group" tensors (u, delta, z, out, dout, du, ddelta, dz for
 * the scan; x, out, states for the conv; x, dt, z, out for the state update)
 * share one storage type given by `dtype`; everything else is float32.
 * Arithmetic is float32 throughout.
 */
#ifndef MAMBA_HIP_H_
#define MAMBA_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MCPU_OK = 0,
  MCPU_ERR_INVALID = 1,     /* bad argument: shape, stride, null pointer, size */
  MCPU_ERR_UNSUPPORTED = 2, /* valid but not implemented (e.g. dstate > 4096) */
  MCPU_ERR_DEVICE = 3,      /* current device is not gfx950 */
  MCPU_ERR_HIP = 4          /* a HIP runtime call or launch failed */
};

enum { MCPU_F32 = 0, MCPU_BF16 = 1, MCPU_F16 = 2 };

/* Text of the last error raised on the calling thread ("" if none). */
const char* mcpu_last_error(void);

/* Checks that the current HIP device is gfx950. Called by every entry point
 * (result cached per device); exported so callers can fail early. */
int mcpu_check_device(void);

/* Library version string. 0.3.0: the argument blocks have grown fields since
 * 0.1.0 (mcpu_scan_args.bwd_waves; mcpu_state_update_args.param_strides and
 * the A, D and dt_bias strides), so a binding built against an older header
 * passes a shorter block: check mcpu_args_size() first. */
const char* mcpu_version(void);

/* sizeof() of an argument block ("scan", "conv", "conv_update",
 * "state_update", "ssd", "mixer_step", "norm_linear", "mamba2_step"), 0 for
 * an unknown name. A binding must compare it with its own sizeof of each
 * block it uses before its first call: the library reads a whole block,
 * whatever the caller allocated. */
size_t mcpu_args_size(const char* name);

/* ------------------------------------------------------------------------ */
/* Selective scan.                                                           */
/* ------------------------------------------------------------------------ */

/* One argument block for forward and backward. Field meaning follows the
 * reference's SelectiveScanParams / SelectiveScanBwdParams
 * (csrc/selective_scan.h:21-38, 51-63), with these differences:
 *   - u/delta/z/dout may be any strided (batch, dim, seqlen) view;
 *   - B/C may be any strided (batch, ngroups, seqlen, dstate) view (the
 *     reference's kernel layout is the contiguous special case, its public
 *     (batch, ngroups, dstate, seqlen) layout the transposed one);
 *   - dA, dD and ddelta_bias come back summed over the batch (the reference
 *     returns per-batch partials that its Python side sums,
 *     src/mamba_cpu/ops/selective_scan_interface.py:87);
 *   - dB/dC are written, not accumulated (no zero-fill needed).
 * Optional inputs/outputs are NULL when absent. */
typedef struct mcpu_scan_args {
  /* forward inputs */
  const void* u;            /* (batch, dim, seqlen), dtype */
  const void* delta;        /* (batch, dim, seqlen), dtype */
  const float* A;           /* (dim, dstate) contiguous */
  const float* B;           /* (batch, ngroups, seqlen, dstate), any strides */
  const float* C;           /* same as B */
  const float* D;           /* (dim), optional */
  const void* z;            /* (batch, dim, seqlen), dtype, optional */
  const float* delta_bias;  /* (dim), optional */
  int64_t batch, dim, seqlen, dstate, ngroups;
  int32_t delta_softplus;
  int32_t dtype;            /* MCPU_F32 / MCPU_BF16 / MCPU_F16 for the x-group */
  int64_t u_stride[3];      /* element strides over (batch, dim, seqlen) */
  int64_t delta_stride[3];
  int64_t z_stride[3];
  int64_t B_stride[4];      /* element strides over (batch, group, seqlen, dstate) */
  int64_t C_stride[4];
  /* forward outputs */
  void* out;                /* (batch, dim, seqlen), dtype, strides out_stride; NULL = states only */
  float* last_state;        /* (batch, dim, dstate) contiguous, optional */
  float* ckpt;              /* optional state checkpoints, see mcpu_selective_scan_ckpt_size */
  void* ysave;              /* optional (batch, dim, seqlen) contiguous, dtype: the forward
                               writes y = <h, C> + D u (before the z gate) here; a backward
                               call given the same buffer reads y instead of recomputing it */
  /* backward inputs */
  const void* dout;         /* (batch, dim, seqlen), dtype; NULL = zeros */
  int64_t dout_stride[3];
  const float* dlast_state; /* (batch, dim, dstate) contiguous, optional */
  /* backward outputs */
  void* du;                 /* (batch, dim, seqlen), dtype, strides du_stride */
  void* ddelta;             /* (batch, dim, seqlen), dtype, strides ddelta_stride */
  void* dz;                 /* (batch, dim, seqlen), dtype, strides dz_stride; required iff z != NULL */
  float* dA;                /* (dim, dstate) */
  float* dB;                /* (batch, ngroups, seqlen, dstate) */
  float* dC;                /* (batch, ngroups, seqlen, dstate) */
  float* dD;                /* (dim); required iff D != NULL */
  float* ddelta_bias;       /* (dim); required iff delta_bias != NULL */
  /* Element strides over (batch, dim, seqlen) of out, du, ddelta and dz; all
     three zero = contiguous. A channel-contiguous layout (dim stride 1, the
     transposed views Hugging Face's mixer passes) lets a caller hand the
     result to a (batch, seqlen, dim) consumer without a copy. */
  int64_t out_stride[3];
  int64_t du_stride[3];
  int64_t ddelta_stride[3];
  int64_t dz_stride[3];
  /* Nonzero: complex A (mamba_ssm's complex-A scan, y = 2 Re(<h, C>) + D u;
     the reference rejects complex A, ops/selective_scan_interface.py:160-161).
     Then A, dA are (dim, dstate) complex64 as (re, im) float pairs; B/C
     strides locate the real part of element (batch, group, seqlen, dstate)
     and the imaginary part is the next float (mamba_ssm's real
     (batch, ngroups, dstate, 2 seqlen) layout, or a complex tensor's view);
     last_state, dlast_state and the checkpoints hold complex pairs; dB/dC are
     (batch, ngroups, seqlen, dstate, 2) contiguous. dstate up to 4096:
     above 32 the states run in 32-state slices, and the forward then needs
     mcpu_selective_scan_fwd_workspace_size() bytes of workspace and, with z,
     writes y before the gate to ysave when given (a sliced backward reads
     it; without it the backward runs that forward itself). At 32 states or
     fewer, ysave and the forward workspace are not used. */
  int32_t complex_a;
  /* Backward workgroup width in waves: 0 = chosen by the library from the
     shape (the production setting); 4, 8 or 12 pins it (dstate <= 16, real A
     only), so tests can cover every width on one shape. The workspace size
     query must see the same value as the call. */
  int32_t bwd_waves;
} mcpu_scan_args;

/* Bytes of the optional checkpoint buffer: the float32 scan state at the
 * start of every 16-step block, (batch, dim, ceil(seqlen/16), dstate)
 * (twice that with complex_a: (re, im) pairs).
 * A forward call with ckpt != NULL fills it; a backward call with the same
 * inputs and ckpt != NULL reads it instead of recomputing it. */
size_t mcpu_selective_scan_ckpt_size(const mcpu_scan_args* a);

/* Workspace bytes that let mcpu_selective_scan_fwd cut the sequence into
 * chunks scanned in parallel (0 when the rows alone fill the GPU). */
size_t mcpu_selective_scan_fwd_workspace_size(const mcpu_scan_args* a);

/* Forward. Replaces selective_scan_fwd_f32 (csrc/selective_scan.h:40) as bound
 * by _C.selective_scan_fwd_f32 (csrc/bindings.cpp:23-45). With a workspace of
 * at least mcpu_selective_scan_fwd_workspace_size() bytes, short batches of
 * long sequences are scanned in parallel time chunks; with NULL (or a smaller
 * one) the sequence is scanned in one pass. Results agree within float32
 * rounding either way. */
int mcpu_selective_scan_fwd(const mcpu_scan_args* a, void* workspace, size_t workspace_bytes,
                            void* stream);

/* Workspace bytes needed by mcpu_selective_scan_bwd for these arguments:
 * the dB/dC/dA partial sums, the adjoint's chunk summaries when time-chunked
 * and, when ckpt is NULL, the block checkpoints and the chunk summaries of
 * the forward that makes them (that forward is time-chunked as a forward call
 * given its workspace is, so the checkpoints equal that call's bit for
 * bit). */
size_t mcpu_selective_scan_bwd_workspace_size(const mcpu_scan_args* a);

/* Backward. Replaces selective_scan_bwd_f32 (csrc/selective_scan.h:65) as
 * bound by _C.selective_scan_bwd_f32 (csrc/bindings.cpp:47-84). */
int mcpu_selective_scan_bwd(const mcpu_scan_args* a, void* workspace, size_t workspace_bytes,
                            void* stream);

/* Bytes of the per-device scratch array behind mcpu_selective_scan_bwd_noalloc.
 * The array is a file-scope __device__ object in a code object of its own: a
 * device reserves it (with that code object, about 66 MiB measured) when the first
 * mcpu_selective_scan_bwd_noalloc call on it looks up the array's address, and
 * holds it until the process ends. Other entry points never reserve it. */
#define MCPU_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* Backward that allocates nothing and takes no workspace. No counterpart in
 * the reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops that forbid allocation). It runs
 * the kernels of mcpu_selective_scan_bwd with their scratch (partial sums,
 * chunk summaries, and when ckpt is NULL the block checkpoints) in a fixed
 * library array of MCPU_NOALLOC_SCRATCH_BYTES per device (reserved by the
 * first call on each device, see above). Results equal
 * mcpu_selective_scan_bwd's. Returns MCPU_ERR_UNSUPPORTED, before any device
 * work, when mcpu_selective_scan_bwd_workspace_size(a) exceeds the array
 * (the training-step shape batch 8, dim 1536, seqlen 1024, dstate 16 needs
 * 35 MB with the forward's checkpoints given). Every call on one device
 * shares that device's array: calls that overlap on one device (other
 * streams, other threads) race and must be serialised by the caller. The
 * first call on each device looks up the array's address; make it outside
 * graph capture. */
int mcpu_selective_scan_bwd_noalloc(const mcpu_scan_args* a, void* stream);

/* ------------------------------------------------------------------------ */
/* Causal depthwise conv1d.                                                  */
/* ------------------------------------------------------------------------ */

/* Replaces the F.conv1d paths of causal_conv1d_fn and its autograd
 * (src/mamba_cpu/ops/causal_conv1d.py:16-53). */
typedef struct mcpu_conv_args {
  const void* x;                /* (batch, dim, seqlen), dtype, any strides */
  const float* weight;          /* (dim, width) contiguous */
  const float* bias;            /* (dim), optional */
  const void* initial_states;   /* (batch, dim, width-1), dtype, optional */
  int64_t batch, dim, seqlen, width;
  int32_t silu;                 /* 1: out = silu(conv), 0: identity */
  int32_t dtype;
  int64_t x_stride[3];
  int64_t init_stride[3];
  /* forward outputs */
  void* out;                    /* (batch, dim, seqlen), dtype, strides out_stride */
  int64_t out_stride[3];
  void* final_states;           /* (batch, dim, width-1) contiguous, dtype, optional */
  /* backward */
  const void* dout;             /* (batch, dim, seqlen), dtype, any strides */
  int64_t dout_stride[3];
  const void* dfinal_states;    /* (batch, dim, width-1) contiguous, dtype, optional */
  void* dx;                     /* (batch, dim, seqlen), dtype, strides dx_stride */
  int64_t dx_stride[3];
  float* dweight;               /* (dim, width) */
  float* dbias;                 /* (dim), required iff bias != NULL */
  void* dinitial_states;        /* (batch, dim, width-1) contiguous, dtype; optional */
  /* (batch, seqlen) contiguous int32, optional: packed sequences; a tap
     reading an input of another sequence counts as zero (the upstream
     causal_conv1d package's semantics; the reference rejects seq_idx,
     ops/causal_conv1d.py:34-35). Excludes initial_states, final_states and
     dfinal_states. */
  const int32_t* seq_idx;
} mcpu_conv_args;

int mcpu_causal_conv1d_fwd(const mcpu_conv_args* a, void* stream);
/* Bytes of device workspace the backward needs: the dweight/dbias partials,
   float32 (batch, parts, dim, width+1). It depends only on batch, dim, seqlen
   and width (the largest of the three kernel paths' partial counts), so one
   workspace serves every layout of a shape. 0 for invalid arguments. */
size_t mcpu_causal_conv1d_bwd_workspace_size(const mcpu_conv_args* a);
int mcpu_causal_conv1d_bwd(const mcpu_conv_args* a, void* workspace, size_t workspace_bytes,
                           void* stream);

/* Decode step(s), conv_state updated in place. Replaces causal_conv1d_update
 * (src/mamba_cpu/ops/causal_conv1d.py:56-85). */
typedef struct mcpu_conv_update_args {
  const void* x;          /* (batch, dim, seqlen), dtype, any strides */
  void* conv_state;       /* (batch, dim, state_len), dtype, any strides, state_len >= width-1 */
  const float* weight;    /* (dim, width) contiguous */
  const float* bias;      /* (dim), optional */
  void* out;              /* (batch, dim, seqlen), dtype, strides out_stride */
  int64_t batch, dim, seqlen, width, state_len;
  int32_t silu;
  int32_t dtype;
  int64_t x_stride[3];
  int64_t state_stride[3];
  int64_t out_stride[3];
  /* Continuous batching (no counterpart in the reference, which raises
     NotImplementedError for both, ops/causal_conv1d.py:66-67; the semantics
     of the upstream causal_conv1d package):
     conv_state_indices (batch) int32, optional: batch row b uses
       conv_state[conv_state_indices[b]]; rows outside [0, state_batch) are
       skipped (out = 0, no state written). Indices must be distinct.
     cache_seqlens (batch) int32, optional: conv_state is a ring buffer; the
       W-1 inputs before x are at (cache_seqlens[b] - (W-1) + k) mod state_len
       and x[s] is written at (cache_seqlens[b] + s) mod state_len.
     state_batch: rows of conv_state (0 = batch). */
  const int32_t* cache_seqlens;
  const int32_t* conv_state_indices;
  int64_t state_batch;
} mcpu_conv_update_args;

int mcpu_causal_conv1d_update(const mcpu_conv_update_args* a, void* stream);

/* ------------------------------------------------------------------------ */
/* Selective state update (one decode step).                                 */
/* ------------------------------------------------------------------------ */

/* Replaces selective_state_update (src/mamba_cpu/ops/selective_state_update.py:5-57).
 * Written for the Mamba-2 head layout; the Mamba-1 layout is the special case
 * nheads = 1, headdim = dim, ngroups = 1. Heads are split into ngroups
 * contiguous groups that share B/C. The state is updated in place. */
typedef struct mcpu_state_update_args {
  void* state;             /* (batch, nheads, headdim, dstate), state_dtype, unit dstate stride */
  const void* x;           /* (batch, nheads, headdim), dtype */
  const void* dt;          /* (batch, nheads, headdim), dtype */
  const float* A;          /* (nheads, headdim, dstate) contiguous */
  const float* B;          /* (batch, ngroups, dstate), unit dstate stride */
  const float* C;          /* (batch, ngroups, dstate), unit dstate stride */
  const float* D;          /* (nheads, headdim), optional */
  const void* z;           /* (batch, nheads, headdim), dtype, optional */
  const float* dt_bias;    /* (nheads, headdim), optional */
  void* out;               /* (batch, nheads, headdim) contiguous, dtype */
  int64_t batch, nheads, headdim, dstate, ngroups;
  int32_t dt_softplus;
  int32_t dtype;           /* storage type of x, dt, z, out */
  int32_t state_dtype;     /* storage type of state */
  int32_t _pad;
  int64_t state_stride[3]; /* over (batch, head, headdim) */
  int64_t x_stride[3];
  int64_t dt_stride[3];
  int64_t z_stride[3];
  int64_t B_stride[2];     /* over (batch, group) */
  int64_t C_stride[2];
  /* state_batch_indices (batch) int32, optional: batch row b updates
     state[state_batch_indices[b]]; rows outside [0, state_batch) are skipped
     (out = 0, no state written). Indices must be distinct. No counterpart in
     the reference, which raises NotImplementedError for it
     (ops/selective_state_update.py:24-25); the semantics of mamba_ssm's
     selective_state_update. state_batch: rows of state (0 = batch). */
  const int32_t* state_batch_indices;
  int64_t state_batch;
  /* 0: A is (nheads, headdim, dstate) and D, dt_bias (nheads, headdim),
     contiguous, and the strides below are ignored. 1: they are read through
     the strides below, in elements, 0 for a broadcast dimension (the Mamba-2
     decode step passes A, D and dt_bias expanded from per-head values).
     No counterpart in the reference, whose op materialises them. */
  int32_t param_strides;
  int32_t _pad2;
  int64_t A_stride[3];     /* over (head, headdim, dstate) */
  int64_t D_stride[2];     /* over (head, headdim) */
  int64_t dt_bias_stride[2];
} mcpu_state_update_args;

int mcpu_selective_state_update(const mcpu_state_update_args* a, void* stream);

/* ------------------------------------------------------------------------ */
/* Mamba-2 SSD scan.                                                         */
/* ------------------------------------------------------------------------ */

/* mamba_ssm's mamba_chunk_scan_combined (mamba_ssm/ops/triton/ssd_combined.py),
 * which the reference lists as roadmap (README.md:7, 94) and does not have.
 * Per batch row and head h (heads split into ngroups contiguous groups that
 * share B and C):
 *   step_t = clamp(softplus?(dt_t + dt_bias_h), dt_limit_lo, dt_limit_hi)
 *   h_t = exp(step_t A_h) h_{t-1} + step_t x_t B_t^T      (headdim x dstate,
 *                                                          h_{-1} = initial state or 0)
 *   y_t = h_t C_t + D x_t ;  out_t = y_t silu(z_t) when z is given
 * All tensors contiguous. headdim a multiple of 16 up to 64, dstate a multiple
 * of 16 up to 128. The forward fills a caller-owned "saved" buffer of
 * mcpu_ssd_saved_size() bytes (per-chunk decays and states) that the backward
 * reads; the chunking is internal (64 steps) and does not change the result
 * beyond float32 rounding. */
typedef struct mcpu_ssd_args {
  const void* x;                /* (batch, seqlen, nheads, headdim), dtype */
  const float* dt;              /* (batch, seqlen, nheads), before dt_bias and softplus */
  const float* A;               /* (nheads) */
  const void* B;                /* (batch, seqlen, ngroups, dstate), dtype */
  const void* C;                /* same as B */
  const float* D;               /* (nheads, headdim), optional */
  const void* z;                /* like x, optional */
  const float* dt_bias;         /* (nheads), optional */
  const float* initial_states;  /* (batch, nheads, headdim, dstate), optional */
  int64_t batch, seqlen, nheads, headdim, ngroups, dstate;
  int32_t dtype;                /* storage type of x, z, B, C, out, ysave, dout, dx, dz */
  int32_t dt_softplus;
  float dt_limit_lo, dt_limit_hi; /* clamp of the step, always applied (mamba_ssm's default is 0, +inf,
                                    which makes a negative raw step 0); the raw-dt gradient is 0 outside */
  /* forward outputs */
  void* out;                    /* like x */
  float* final_states;          /* (batch, nheads, headdim, dstate), optional */
  void* ysave;                  /* like x: y before the z gate; the forward writes it when
                                   given (needed by the backward when z is given) */
  /* backward inputs */
  const void* dout;             /* like x */
  const float* dfinal_states;   /* like final_states, optional */
  /* backward outputs */
  void* dx;                     /* like x */
  float* ddt;                   /* (batch, seqlen, nheads): gradient of the raw dt */
  float* dA;                    /* (nheads) */
  float* dB;                    /* (batch, seqlen, ngroups, dstate) float32 */
  float* dC;
  float* dD;                    /* (nheads, headdim); required iff D != NULL */
  void* dz;                     /* like x; required iff z != NULL */
  float* ddt_bias;              /* (nheads); required iff dt_bias != NULL */
  float* dinitial_states;       /* required iff initial_states != NULL */
  /* Heads one workgroup of the chunk kernels walks through: 0 = chosen by
     the library from the shape (the production setting); otherwise a divisor
     of nheads / ngroups, at most 8, which pins it, so tests can cover every
     head-block size on small shapes. The backward's workspace size query
     must see the same value as the call. */
  int32_t head_block;
  /* How the chunk states are carried from chunk to chunk: 0 = chosen by the
     library from the shape (the production setting); 1 = chunk-end states
     computed for every chunk at once, then passed on in a second launch;
     2 = one launch per (batch, head, 64-state column block) that walks the
     chunks in order and never stores the chunk-end states. Both give the
     same result up to float32 rounding; pinning one lets tests cover both.
     The size queries must see the same value as the calls. */
  int32_t chunk_pass;
  /* (batch, seqlen) int32, optional: ids of packed sequences, non-decreasing
     along each row. The state does not carry across a change of id (the
     decay is 0 there), and the initial state belongs to id 0, as mamba_ssm's
     seq_idx. */
  const int32_t* seq_idx;
} mcpu_ssd_args;

/* Bytes of the buffer the forward fills for the backward (0 for an empty
 * batch or sequence, where the buffer may be NULL; 0 too for arguments the
 * entry points reject, which then say why). */
size_t mcpu_ssd_saved_size(const mcpu_ssd_args* a);
/* Forward. Replaces nothing in the reference (see above). */
int mcpu_ssd_fwd(const mcpu_ssd_args* a, void* saved, size_t saved_bytes, void* stream);
/* Workspace bytes of the backward (0, and NULL allowed, when empty). */
size_t mcpu_ssd_bwd_workspace_size(const mcpu_ssd_args* a);
/* Backward, given the forward's saved buffer (and ysave when z is given). */
int mcpu_ssd_bwd(const mcpu_ssd_args* a, const void* saved, size_t saved_bytes, void* workspace,
                 size_t workspace_bytes, void* stream);
/* Per-sequence final states of packed sequences (mamba_ssm's
 * return_varlen_states with cu_seqlens; none in the reference), after
 * mcpu_ssd_fwd with the same arguments, on the same stream, given the saved
 * buffer it filled. batch must be 1. cu_seqlens: nseqs + 1 int32 offsets into
 * the sequence, non-decreasing from 0 to seqlen. varlen_states (nseqs,
 * nheads, headdim, dstate) float32: entry i is the scan's state after step
 * cu_seqlens[i + 1] - 1, with seq_idx as given (pass ids that mark the same
 * sequences so that each state is its own sequence's); zeros for an empty
 * sequence or offsets outside [0, seqlen]. No gradient. */
int mcpu_ssd_varlen_states(const mcpu_ssd_args* a, const void* saved, size_t saved_bytes,
                           const int32_t* cu_seqlens, int64_t nseqs, float* varlen_states, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused single-token Mamba block step (decode).                             */
/* ------------------------------------------------------------------------ */

/* One decode step of a Mamba-1 block for a batch of single tokens: what the
 * reference's patched transformers MambaBlock computes for one token with a
 * cache (src/mamba_cpu/hf.py:26-112 routes its pieces: causal_conv1d_update,
 * selective_state_update), in three launches instead of a dozen (four for
 * blocks of Mamba-790M width and up, whose x_proj runs as its own product):
 *   u    = RMSNorm(hidden) when norm_weight != NULL (else hidden), in dtype
 *   x, z = in_proj(u)                    (2 d_inner)
 *   x    = silu(conv1d_update(conv_state, x))   conv_state shifted in place
 *   dt, B, C = x_proj(x)                 (dt_rank, dstate, dstate)
 *   dt   = dt_proj.weight dt             (no bias here)
 *   y    = selective_state_update(ssm_state, x, dt, A, B, C, D, z, dt_bias, softplus)
 *   out  = out_proj(y) [+ hidden, the residual, when add_residual]
 * Rounding follows transformers: each stage's result is stored in dtype
 * before the next reads it; arithmetic is float32. No counterpart in the
 * reference (it has no fused decode path). All tensors contiguous, 16-byte
 * aligned; batch <= 8; d_model and d_inner multiples of 4; conv width and
 * state length at most 8; with batch rounded up to a power of two, (batch + 1)
 * x d_model and batch x d_inner at most 32768. */
typedef struct mcpu_mixer_step_args {
  const void* hidden;       /* (batch, d_model), hidden_dtype */
  const void* norm_weight;  /* (d_model), dtype, optional */
  const void* in_w;         /* (2 d_inner, d_model), dtype */
  const void* in_b;         /* (2 d_inner), dtype, optional */
  const void* conv_w;       /* (d_inner, width), dtype */
  const void* conv_b;       /* (d_inner), dtype, optional */
  void* conv_state;         /* (batch, d_inner, state_len), dtype, state_len >= width - 1 */
  const void* x_w;          /* (dt_rank + 2 dstate, d_inner), dtype */
  const void* dt_w;         /* (d_inner, dt_rank), dtype */
  const float* dt_b;        /* (d_inner), optional */
  const float* A;           /* (d_inner, dstate): -exp(A_log) */
  const float* D;           /* (d_inner), optional */
  void* ssm_state;          /* (batch, d_inner, dstate), state_dtype */
  const void* out_w;        /* (d_model, d_inner), dtype */
  const void* out_b;        /* (d_model), dtype, optional */
  void* out;                /* (batch, d_model), out_dtype */
  int64_t batch, d_model, d_inner, dt_rank, dstate, width, state_len;
  float norm_eps;
  int32_t add_residual;     /* out = residual + out_proj(y) */
  int32_t residual_in_fp32; /* the residual is hidden in float32 */
  int32_t dtype;            /* weights, activations, conv state */
  int32_t hidden_dtype;     /* dtype or MCPU_F32 */
  int32_t state_dtype;      /* ssm_state */
  int32_t out_dtype;        /* dtype, or MCPU_F32 with a float32 residual */
  int32_t _pad;
} mcpu_mixer_step_args;

/* Workspace bytes of mcpu_mixer_step (the step's intermediate vectors). */
size_t mcpu_mixer_step_workspace_size(const mcpu_mixer_step_args* a);
/* One step. Updates conv_state and ssm_state in place and writes out. */
int mcpu_mixer_step(const mcpu_mixer_step_args* a, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Final norm and output head of a decode step.                              */
/* ------------------------------------------------------------------------ */

/* out = Linear(RMSNorm(hidden)) for a batch of single tokens: a Mamba
 * model's last step after its blocks (transformers' MambaRMSNorm norm_f,
 * then lm_head on the result cast to the weights' dtype, logits .float()):
 *   r   = hidden * rsqrt(mean(hidden^2) + norm_eps)     (float32)
 *   u   = round_dtype(norm_weight * round_hidden(r))    (round_dtype(hidden)
 *                                                        without a norm weight)
 *   out = round_dtype(weight u + bias)                  stored as out_dtype
 * round_hidden rounds to hidden_dtype (nothing for float32 rows); arithmetic
 * is float32. No counterpart in the reference (it has no fused decode path):
 * one launch for callers that replay a whole decode step. All tensors
 * contiguous; hidden, weight and norm_weight 16-byte aligned; batch <= 8;
 * d_in a multiple of 4; with batch rounded up to a power of two,
 * (batch + 1) x d_in at most 32768. */
typedef struct mcpu_norm_linear_args {
  const void* hidden;       /* (batch, d_in), hidden_dtype */
  const void* norm_weight;  /* (d_in), dtype, optional */
  const void* weight;       /* (d_out, d_in), dtype */
  const void* bias;         /* (d_out), dtype, optional */
  void* out;                /* (batch, d_out), out_dtype */
  int64_t batch, d_in, d_out;
  float norm_eps;
  int32_t dtype;            /* weights */
  int32_t hidden_dtype;     /* dtype or MCPU_F32 */
  int32_t out_dtype;        /* dtype or MCPU_F32 */
} mcpu_norm_linear_args;

int mcpu_norm_linear(const mcpu_norm_linear_args* a, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused single-token Mamba-2 block step (decode).                           */
/* ------------------------------------------------------------------------ */

/* One decode step of a Mamba-2 block for a batch of single tokens: what a
 * transformers Mamba2Block computes for one token with a cache (its mixer's
 * recurrent form, which the reference's patched models route through
 * causal_conv1d_update and the Mamba-2 form of selective_state_update,
 * src/mamba_cpu/hf.py), in three launches:
 *   u         = RMSNorm(hidden) when norm_weight != NULL (else hidden), in dtype
 *   gate, xBC, dt = in_proj(u)             (d_inner, conv_dim, nheads)
 *   xBC       = silu(conv1d_update(conv_state, xBC))   conv_state shifted in place
 *   x, B, C   = xBC                        (d_inner, ngroups dstate, ngroups dstate)
 *   y         = selective_state_update(ssm_state, x, dt, A, B, C, D, dt_bias, softplus)
 *               per head h of headdim channels, group h / (nheads / ngroups)
 *   r         = y silu(gate) ;  y = gate_norm_weight round(r rsqrt(mean(r^2) + gate_norm_eps))
 *   out       = out_proj(y) [+ hidden, the residual, when add_residual]
 * conv_dim = d_inner + 2 ngroups dstate. Rounding follows transformers: each
 * stage's result is stored in dtype before the next reads it; arithmetic is
 * float32. No counterpart in the reference (it has no fused decode path). All
 * tensors contiguous, 16-byte aligned; batch <= 8; d_model and d_inner
 * multiples of 4; dstate <= 128; conv width and state length at most 8; with
 * batch rounded up to a power of two, (batch + 1) x d_model and (batch + 1) x
 * d_inner at most 32768. */
typedef struct mcpu_mamba2_step_args {
  const void* hidden;           /* (batch, d_model), hidden_dtype */
  const void* norm_weight;      /* (d_model), dtype, optional */
  const void* in_w;             /* (d_inner + conv_dim + nheads, d_model), dtype */
  const void* in_b;             /* (d_inner + conv_dim + nheads), dtype, optional */
  const void* conv_w;           /* (conv_dim, width), dtype */
  const void* conv_b;           /* (conv_dim), dtype, optional */
  void* conv_state;             /* (batch, conv_dim, state_len), dtype */
  const float* dt_bias;         /* (nheads), optional */
  const float* A;               /* (nheads): -exp(A_log) */
  const float* D;               /* (nheads), optional */
  void* ssm_state;              /* (batch, nheads, headdim, dstate), state_dtype */
  const void* gate_norm_weight; /* (d_inner), dtype */
  const void* out_w;            /* (d_model, d_inner), dtype */
  const void* out_b;            /* (d_model), dtype, optional */
  void* out;                    /* (batch, d_model), out_dtype */
  int64_t batch, d_model, d_inner, nheads, headdim, ngroups, dstate, width, state_len;
  float norm_eps, gate_norm_eps;
  int32_t add_residual;         /* out = residual + out_proj(y) */
  int32_t residual_in_fp32;     /* the residual is hidden in float32 */
  int32_t dtype;                /* weights, activations, conv state */
  int32_t hidden_dtype;         /* dtype or MCPU_F32 */
  int32_t state_dtype;          /* ssm_state */
  int32_t out_dtype;            /* dtype, or MCPU_F32 with a float32 residual */
} mcpu_mamba2_step_args;

/* Workspace bytes of mcpu_mamba2_step (the step's intermediate vectors). */
size_t mcpu_mamba2_step_workspace_size(const mcpu_mamba2_step_args* a);
/* One step. Updates conv_state and ssm_state in place and writes out. */
int mcpu_mamba2_step(const mcpu_mamba2_step_args* a, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MAMBA_HIP_H_ */
