"""Greedy decoding of transformers Mamba models with each token's step
replayed from a HIP graph.

    import mamba_cpu.hf, mamba_cpu.decode
    mamba_cpu.hf.patch_transformers()
    ids = mamba_cpu.decode.greedy_generate(model, prompt, max_new_tokens=128)

`model.generate(prompt, do_sample=False, ...)` spends most of a decode step on
the host: every layer issues a dozen small kernels through Python, each one
dispatched on its own. A Mamba decode step is shape-static once the prompt has
been consumed: the cache holds one conv window and one state per layer, and
both are updated in place (transformers allocates them once, at fixed
addresses). So the whole step, from the token embedding to the last-position
logits, is captured once into a HIP graph (torch.cuda.CUDAGraph) and replayed
per token; only the argmax and the token copies run eagerly between replays.

For Mamba (not FalconMamba, whose mixer normalises dt, B and C) the captured
step runs each block as one fused operator, mamba_cpu::mixer_step: RMSNorm,
in_proj, conv update, x_proj, dt_proj, state update, out_proj and the
residual in three kernels, with the small-batch products as matrix-vector
kernels that read each weight once, and the final norm and lm_head as one
more, mamba_cpu::norm_linear. Mamba-2 blocks run as
mamba_cpu::mamba2_step: RMSNorm, in_proj, the conv update of x, B and C,
the per-head state update, the gated RMSNorm, out_proj and the residual in
three kernels. Both compute what the model computes; the products sum in
another order than the GEMM library's, so logits agree to float32 rounding
and greedy tokens match `model.generate`'s. FalconMamba models replay their
own decode step (on this package's conv update and state update once
mamba_cpu.hf is patched).
"""

import torch

from mamba_cpu import _C  # noqa: F401  (loads the operator library)

_GRAPH_MODELS = ("mamba", "falcon_mamba", "mamba2")
# Limits of mcpu_mixer_step (csrc/mixer_step.hip, check_step): batch rows,
# conv window length, state size, and the float32 LDS budget that holds the
# batch rows (padded to a power of two) of one workgroup.
_MAX_FUSED_BATCH = 8
_MAX_FUSED_CONV_STATE = 8
_MAX_FUSED_DSTATE = 128
_FUSED_LDS_FLOATS = 32768


def _fused_lds_fits(batch_size, d_model, d_inner, gated=False):
    """Whether the fused step's workgroups can hold `batch_size` rows of the
    normed hidden state (plus one row of scratch) and of the conv outputs in
    LDS, as check_step requires (Mamba-2's gated norm also stages its weight
    beside the d_inner rows: check_step2)."""
    rows = 1 if batch_size <= 1 else 2 if batch_size <= 2 else 4 if batch_size <= 4 else 8
    return (rows + 1) * d_model <= _FUSED_LDS_FLOATS and (rows + int(gated)) * d_inner <= _FUSED_LDS_FLOATS


@torch.library.register_fake("mamba_cpu::norm_linear")
def _(hidden, norm_weight, eps, weight, bias, out_float32):
    return hidden.new_empty((hidden.shape[0], weight.shape[0]), dtype=torch.float32 if out_float32 else weight.dtype)


@torch.library.register_fake("mamba_cpu::mamba2_step")
def _(hidden, norm_weight, eps, add_residual, residual_in_fp32, in_w, in_b, conv_w, conv_b, conv_state, dt_bias,
      A, D, ssm_state, gate_norm_w, gate_eps, out_w, out_b):
    f32 = add_residual and (residual_in_fp32 or hidden.dtype == torch.float32)
    return hidden.new_empty(hidden.shape, dtype=torch.float32 if f32 else in_w.dtype)


@torch.library.register_fake("mamba_cpu::mixer_step")
def _(hidden, norm_weight, eps, add_residual, residual_in_fp32, in_w, in_b, conv_w, conv_b, conv_state, x_w,
      dt_w, dt_b, A, D, ssm_state, out_w, out_b):
    f32 = add_residual and (residual_in_fp32 or hidden.dtype == torch.float32)
    return hidden.new_empty(hidden.shape, dtype=torch.float32 if f32 else in_w.dtype)


def _block_constants(mixer):
    """float32 dt bias (Mamba: dt_proj's, Mamba-2: the per-head dt_bias),
    A = -exp(A_log) and D of a mixer, computed once and kept on the module
    until one of the parameters changes."""
    dt_bias = mixer.dt_bias if hasattr(mixer, "dt_bias") else mixer.dt_proj.bias
    params = (mixer.A_log, mixer.D, dt_bias)
    key = tuple((t.data_ptr(), t._version) for t in params if t is not None)
    cached = getattr(mixer, "_mamba_cpu_step_constants", None)
    if cached is None or cached[0] != key:
        with torch.no_grad():
            A = -torch.exp(mixer.A_log.float())
            D = mixer.D.float().contiguous()
            dtb = None if dt_bias is None else dt_bias.float().contiguous()
        cached = (key, A.contiguous(), D, dtb)
        mixer._mamba_cpu_step_constants = cached
    return cached[1:]


def fused_step_supported(model, cache, batch_size):
    """Whether `model`'s decode step can run as fused block steps: a
    transformers Mamba or Mamba-2 model on a ROCm GPU, one weight dtype, silu,
    at most 8 batch rows, widths the fused kernels take, and a cache whose
    conv windows are not recording past inputs. Shapes the kernels would
    refuse keep the unfused step."""
    kind = model.config.model_type
    if kind not in ("mamba", "mamba2") or batch_size > _MAX_FUSED_BATCH:
        return False
    layers = getattr(getattr(model, "backbone", None), "layers", None)
    if not layers:
        return False
    for blk in layers:
        mx = blk.mixer
        w = mx.in_proj.weight
        if w.device.type != "cuda" or mx.activation != "silu":
            return False
        if kind == "mamba":
            own = [mx.x_proj.weight, mx.dt_proj.weight]
        else:
            own = [mx.norm.weight]
        tensors = [blk.norm.weight, w, mx.in_proj.bias, mx.conv1d.weight, mx.conv1d.bias, mx.out_proj.weight,
                   mx.out_proj.bias] + own
        if any(t is not None and (t.dtype != w.dtype or not t.is_contiguous()) for t in tensors):
            return False
        if w.shape[1] % 4 or mx.intermediate_size % 4 or mx.ssm_state_size > _MAX_FUSED_DSTATE \
                or mx.conv_kernel_size > _MAX_FUSED_CONV_STATE \
                or not _fused_lds_fits(batch_size, w.shape[1], mx.intermediate_size, kind == "mamba2"):
            return False
        layer = cache.layers[blk.layer_idx]
        conv, ssm = layer.conv_states[0], layer.recurrent_states[0]
        if layer.record_past or conv is None or ssm is None or not conv.is_contiguous() \
                or not ssm.is_contiguous() or conv.dtype != w.dtype or conv.shape[2] > _MAX_FUSED_CONV_STATE:
            return False
    return True


def fused_block_step(block, hidden, cache):
    """One decode step of a transformers MambaBlock or Mamba2Block: hidden
    (batch, d_model) -> the block's output (batch, d_model), the layer's conv
    window and SSM state in `cache` advanced in place."""
    mx = block.mixer
    layer = cache.layers[block.layer_idx]
    A, D, dtb = _block_constants(mx)
    if hasattr(mx, "dt_bias"):  # Mamba-2
        conv_w = mx.conv1d.weight.view(mx.conv1d.weight.shape[0], -1)
        return torch.ops.mamba_cpu.mamba2_step(
            hidden, block.norm.weight, float(block.norm.variance_epsilon), True, bool(block.residual_in_fp32),
            mx.in_proj.weight, mx.in_proj.bias, conv_w, mx.conv1d.bias, layer.conv_states[0], dtb, A, D,
            layer.recurrent_states[0], mx.norm.weight, float(mx.norm.variance_epsilon), mx.out_proj.weight,
            mx.out_proj.bias)
    conv_w = mx.conv1d.weight.view(mx.intermediate_size, -1)
    return torch.ops.mamba_cpu.mixer_step(
        hidden, block.norm.weight, float(block.norm.variance_epsilon), True, bool(block.residual_in_fp32),
        mx.in_proj.weight, mx.in_proj.bias, conv_w, mx.conv1d.bias, layer.conv_states[0], mx.x_proj.weight,
        mx.dt_proj.weight, dtb, A, D, layer.recurrent_states[0], mx.out_proj.weight, mx.out_proj.bias)


def fused_head_supported(model, batch_size):
    """Whether a Mamba model's final norm and lm_head can run as one
    mamba_cpu::norm_linear launch (mcpu_norm_linear's limits: at most 8 rows,
    a width that is a multiple of 4 and fits the LDS budget, one dtype)."""
    norm, head = model.backbone.norm_f, model.lm_head
    w = head.weight
    rows = 1 if batch_size <= 1 else 2 if batch_size <= 2 else 4 if batch_size <= 4 else 8
    return (batch_size <= _MAX_FUSED_BATCH and w.device.type == "cuda" and w.is_contiguous()
            and w.shape[1] % 4 == 0 and (rows + 1) * w.shape[1] <= _FUSED_LDS_FLOATS
            and norm.weight.dtype == w.dtype and norm.weight.is_contiguous()
            and (head.bias is None or (head.bias.dtype == w.dtype and head.bias.is_contiguous())))


def fused_model_step(model, token, cache):
    """A transformers MambaForCausalLM or Mamba2ForCausalLM decode step with fused blocks: token
    (batch, 1) -> last-position logits (batch, vocab) float32, the cache
    advanced in place."""
    bb = model.backbone
    h = bb.embeddings(token)[:, 0]
    for blk in bb.layers:
        h = fused_block_step(blk, h, cache)
    if fused_head_supported(model, h.shape[0]):
        head = model.lm_head
        return torch.ops.mamba_cpu.norm_linear(h, bb.norm_f.weight, float(bb.norm_f.variance_epsilon),
                                               head.weight, head.bias, True)
    h = bb.norm_f(h)
    return model.lm_head(h.to(model.lm_head.weight.dtype)).float()


def _cache_tensors(cache):
    """Every state tensor of a transformers linear-attention cache."""
    out = []
    for layer in cache.layers:
        for states in (getattr(layer, "conv_states", None), getattr(layer, "recurrent_states", None)):
            if states:
                out.extend(t for t in states.values() if t is not None)
    return out


class GraphedDecodeStep:
    """One decode step of `model` (a transformers MambaForCausalLM,
    FalconMambaForCausalLM or Mamba2ForCausalLM on a ROCm GPU) captured as a
    HIP graph.

    `cache` is the model's cache after the prompt (the `cache_params` a
    `use_cache=True` forward returns). `token` is the (batch, 1) int64 tensor
    the graph reads; `logits` the (batch, vocab) tensor it writes. Each
    `replay()` advances the cache by the token in `token`. With `fused`
    (the default) a Mamba model's blocks run as fused block steps where
    fused_step_supported() allows; `self.fused` says whether they do."""

    def __init__(self, model, cache, batch_size, warmup=2, fused=True):
        if model.config.model_type not in _GRAPH_MODELS:
            raise NotImplementedError(
                f"graph-captured decoding supports {', '.join(_GRAPH_MODELS)} models, "
                f"got {model.config.model_type!r}")
        dev = next(model.parameters()).device
        if dev.type != "cuda":
            raise ValueError(f"graph-captured decoding runs on ROCm GPU models, got device {dev}")
        self.model, self.cache = model, cache
        self.fused = bool(fused) and fused_step_supported(model, cache, batch_size)
        self.token = torch.zeros(batch_size, 1, dtype=torch.long, device=dev)
        states = _cache_tensors(cache)
        saved = [t.clone() for t in states]
        # Warm-up steps on a side stream (first-call work stays out of the
        # graph), then the cache is restored: capturing runs no kernel, so the
        # cache is exactly as the prompt left it.
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(warmup):
                self._step()
        torch.cuda.current_stream(dev).wait_stream(side)
        with torch.no_grad():
            for t, s in zip(states, saved):
                t.copy_(s)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.no_grad():
            self.logits = self._step()

    def _step(self):
        if self.fused:
            return fused_model_step(self.model, self.token, self.cache)
        out = self.model(input_ids=self.token, cache_params=self.cache, use_cache=True)
        return out.logits[:, -1]

    def replay(self):
        self.graph.replay()
        return self.logits


@torch.no_grad()
def greedy_generate(model, input_ids, max_new_tokens, fused=True):
    """Greedy decoding: the prompt in one eager forward, then `max_new_tokens`
    - 1 graph-replayed steps. Returns (batch, prompt + max_new_tokens) int64
    token ids, as `model.generate(input_ids, max_new_tokens=max_new_tokens,
    min_new_tokens=max_new_tokens, do_sample=False)` does for these models."""
    b = input_ids.shape[0]
    out = model(input_ids=input_ids, use_cache=True)
    new = torch.empty(b, max_new_tokens, dtype=torch.long, device=input_ids.device)
    new[:, :1] = out.logits[:, -1].argmax(-1, keepdim=True)
    if max_new_tokens > 1:
        step = GraphedDecodeStep(model, out.cache_params, b, fused=fused)
        for i in range(1, max_new_tokens):
            step.token.copy_(new[:, i - 1:i])
            new[:, i:i + 1] = step.replay().argmax(-1, keepdim=True)
    return torch.cat([input_ids, new], dim=1)
