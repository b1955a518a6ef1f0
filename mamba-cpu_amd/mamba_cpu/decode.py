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
addresses, and the conv update and state update ops write them in place). So
the whole step, from the token embedding to the last-position logits, is
captured once into a HIP graph (torch.cuda.CUDAGraph) and replayed per token;
only the argmax and the token copies run eagerly between replays.

The result is the token sequence `model.generate` returns for greedy decoding
with no logits processors: the replayed kernels are the eager step's kernels
on the same inputs.
"""

import torch

_GRAPH_MODELS = ("mamba", "falcon_mamba")


def _cache_tensors(cache):
    """Every state tensor of a transformers linear-attention cache."""
    out = []
    for layer in cache.layers:
        for states in (getattr(layer, "conv_states", None), getattr(layer, "recurrent_states", None)):
            if states:
                out.extend(t for t in states.values() if t is not None)
    return out


class GraphedDecodeStep:
    """One decode step of `model` (a transformers MambaForCausalLM or
    FalconMambaForCausalLM on a ROCm GPU) captured as a HIP graph.

    `cache` is the model's cache after the prompt (the `cache_params` a
    `use_cache=True` forward returns). `token` is the (batch, 1) int64 tensor
    the graph reads; `logits` the (batch, vocab) tensor it writes. Each
    `replay()` advances the cache by the token in `token`."""

    def __init__(self, model, cache, batch_size, warmup=2):
        if model.config.model_type not in _GRAPH_MODELS:
            raise NotImplementedError(
                f"graph-captured decoding supports {', '.join(_GRAPH_MODELS)} models, "
                f"got {model.config.model_type!r}")
        dev = next(model.parameters()).device
        if dev.type != "cuda":
            raise ValueError(f"graph-captured decoding runs on ROCm GPU models, got device {dev}")
        self.model, self.cache = model, cache
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
        out = self.model(input_ids=self.token, cache_params=self.cache, use_cache=True)
        return out.logits[:, -1]

    def replay(self):
        self.graph.replay()
        return self.logits


@torch.no_grad()
def greedy_generate(model, input_ids, max_new_tokens):
    """Greedy decoding: the prompt in one eager forward, then `max_new_tokens`
    - 1 graph-replayed steps. Returns (batch, prompt + max_new_tokens) int64
    token ids, as `model.generate(input_ids, max_new_tokens=max_new_tokens,
    min_new_tokens=max_new_tokens, do_sample=False)` does for these models."""
    b = input_ids.shape[0]
    out = model(input_ids=input_ids, use_cache=True)
    new = torch.empty(b, max_new_tokens, dtype=torch.long, device=input_ids.device)
    new[:, :1] = out.logits[:, -1].argmax(-1, keepdim=True)
    if max_new_tokens > 1:
        step = GraphedDecodeStep(model, out.cache_params, b)
        for i in range(1, max_new_tokens):
            step.token.copy_(new[:, i - 1:i])
            new[:, i:i + 1] = step.replay().argmax(-1, keepdim=True)
    return torch.cat([input_ids, new], dim=1)
