"""mamba_cpu.hf on small random Mamba, FalconMamba, Jamba and Mamba-2 models.

Each check runs one model twice on the GPU: first on transformers' own
pure-torch kernel functions (the functions the routes replace, reached
through __wrapped__), then with patch_transformers() routing the kernels to
this package's HIP ops, and compares the two. The cases are those of the
reference's tests/test_hf.py: logits, greedy generation, a padded batch,
training gradients, patching twice and undoing it, models on other devices
left alone, a patched model used as installed. Beyond them: the
graph-replayed greedy decoder (mamba_cpu.decode) against model.generate, and
a two-layer model of the Mamba-130M width (d_model 768, vocabulary 50280)
checked with the reference's model-level measures (largest logit
difference, top-1 agreement, greedy identity, per-tensor gradient error:
benchmarks/check_hf_model.py:105-121). Mamba-2 (which the reference does not
route) takes the same cases through mamba_chunk_scan_combined, plus a two-layer
model at the Mamba-2 2.7B layer's head shape (headdim 64, dstate 128).
"""

import contextlib
import importlib

import pytest
import torch

pytest.importorskip("transformers", minversion="5.0")

import transformers

import mamba_cpu.hf

FAMILIES = mamba_cpu.hf.SUPPORTED_MODELS
DEV = "cuda"
TINY = dict(vocab_size=64, hidden_size=32, num_hidden_layers=2, state_size=8, conv_kernel=4, expand=2)


def tiny_model(family, device=DEV):
    torch.manual_seed(0)
    if family == "mamba":
        model = transformers.MambaForCausalLM(transformers.MambaConfig(**TINY))
    elif family == "falcon_mamba":
        model = transformers.FalconMambaForCausalLM(transformers.FalconMambaConfig(**TINY))
    elif family == "mamba2":  # 4 heads of 16 channels, 2 groups
        model = transformers.Mamba2ForCausalLM(transformers.Mamba2Config(
            vocab_size=64, hidden_size=32, num_hidden_layers=2, state_size=16, conv_kernel=4, expand=2,
            num_heads=4, head_dim=16, n_groups=2, chunk_size=16))
    else:  # a Mamba layer then an attention layer, one expert
        model = transformers.JambaForCausalLM(transformers.JambaConfig(
            vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
            num_attention_heads=2, num_key_value_heads=2, num_experts=1, attn_layer_period=2,
            attn_layer_offset=1, expert_layer_period=2, expert_layer_offset=1, mamba_d_state=8,
            mamba_dt_rank=4, use_mamba_kernels=False))
    return model.to(device).eval()


def token_ids(shape, device=DEV, vocab=64, seed=1):
    return torch.randint(0, vocab, shape, generator=torch.Generator().manual_seed(seed)).to(device)


def _modules():
    """(modeling module, its kernel-globals table) of every family."""
    return [(importlib.import_module(f".modeling_{f}", f"transformers.models.{f}"), mamba_cpu.hf.kernel_globals(f))
            for f in FAMILIES]


@contextlib.contextmanager
def torch_kernels():
    """transformers' pure-torch kernel functions in every family's globals
    (the plain functions its hub/fallback decorator wraps), restored after."""
    mamba_cpu.hf.unpatch_transformers()
    saved = []
    for module, table in _modules():
        for name in table:
            fn = getattr(module, name)
            saved.append((module, name, fn))
            setattr(module, name, getattr(fn, "__wrapped__", fn))
    try:
        yield
    finally:
        for module, name, fn in saved:
            setattr(module, name, fn)


@contextlib.contextmanager
def gpu_kernels():
    """Those same globals routed to this package (patched over the pure-torch
    functions, so nothing but this package's ops can run on the GPU)."""
    with torch_kernels():
        mamba_cpu.hf.patch_transformers()
        try:
            yield
        finally:
            mamba_cpu.hf.unpatch_transformers()


def torch_then_gpu(fn):
    """(fn() on this package's ops, fn() on transformers' torch kernels)."""
    with torch_kernels():
        want = fn()
    with gpu_kernels():
        got = fn()
    return got, want


@pytest.fixture
def calls(monkeypatch):
    """Names of the GPU bodies the routes ran, in order."""
    seen = []

    def counted(name, body):
        def run(*args, **kwargs):
            seen.append(name)
            return body(*args, **kwargs)
        return run

    for table in (mamba_cpu.hf.KERNEL_GLOBALS, mamba_cpu.hf.MAMBA2_KERNEL_GLOBALS):
        for name, body in list(table.items()):
            monkeypatch.setitem(table, name, counted(name, body))
    return seen


def used_the_scan(seen):
    # the scan itself, the fused mixer (which runs it) in training, or the
    # Mamba-2 chunked scan
    return any(name in seen for name in ("mamba_selective_scan", "mamba_inner_fn", "mamba2_chunk_scan"))


per_family = pytest.mark.parametrize("family", FAMILIES)


@pytest.mark.gpu
@per_family
def test_logits_match(family, calls):
    model = tiny_model(family)
    ids = token_ids((2, 37))
    got, want = torch_then_gpu(lambda: model(ids).logits.detach())
    assert used_the_scan(calls)
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
@per_family
def test_greedy_generation_matches(family, calls):
    model = tiny_model(family)
    ids = token_ids((2, 11))
    got, want = torch_then_gpu(lambda: model.generate(ids, max_new_tokens=12, do_sample=False))
    assert used_the_scan(calls)
    assert "mamba_selective_state_update" in calls or "mamba2_selective_state_update" in calls
    assert torch.equal(got, want)


@pytest.mark.gpu
@per_family
def test_left_padded_batch_matches(family):
    model = tiny_model(family)
    ids = token_ids((2, 16))
    mask = torch.ones_like(ids)
    mask[1, :5] = 0
    got, want = torch_then_gpu(lambda: model(ids, attention_mask=mask).logits.detach())
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
@per_family
def test_training_gradients_match(family, calls):
    model = tiny_model(family).train()
    ids = token_ids((2, 24))

    def grads():
        model.zero_grad()
        model(ids, labels=ids).loss.backward()
        return {k: p.grad.clone() for k, p in model.named_parameters() if p.grad is not None}

    got, want = torch_then_gpu(grads)
    assert got.keys() == want.keys() and used_the_scan(calls)
    if family == "mamba":
        # float32 Mamba in training takes the fused mixer; FalconMamba keeps
        # its unfused path (its norms differ from the fused mixer's)
        assert "mamba_inner_fn" in calls and "mamba_selective_scan" not in calls
    for k, w in want.items():
        torch.testing.assert_close(got[k], w, rtol=1e-3, atol=1e-4, msg=lambda m: f"{k}: {m}")


def test_patching_twice_changes_nothing_and_unpatch_restores():
    module = importlib.import_module("transformers.models.mamba.modeling_mamba")
    before = {name: getattr(module, name) for name in mamba_cpu.hf.KERNEL_GLOBALS}
    mamba_cpu.hf.patch_transformers()
    try:
        first = {name: getattr(module, name) for name in before}
        assert all(isinstance(r, mamba_cpu.hf.DeviceRoute) for r in first.values())
        mamba_cpu.hf.patch_transformers()
        assert all(getattr(module, name) is first[name] for name in before)
        assert all(first[name].fallback is before[name] for name in before)
    finally:
        mamba_cpu.hf.unpatch_transformers()
    assert all(getattr(module, name) is fn for name, fn in before.items())


def test_patch_refuses_modules_without_the_kernel_globals(monkeypatch):
    module = importlib.import_module("transformers.models.mamba.modeling_mamba")
    monkeypatch.delattr(module, "mamba_inner_fn")
    falcon = importlib.import_module("transformers.models.falcon_mamba.modeling_falcon_mamba")
    before = falcon.mamba_selective_scan
    with pytest.raises(RuntimeError, match="transformers >= 5"):
        mamba_cpu.hf.patch_transformers()
    assert falcon.mamba_selective_scan is before  # nothing was patched


def test_models_on_other_devices_keep_transformers_kernels(calls):
    model = tiny_model("mamba", device="cpu")
    ids = token_ids((1, 9), device="cpu")
    with torch.no_grad():
        want = model(ids).logits
    mamba_cpu.hf.patch_transformers()
    try:
        with torch.no_grad():
            got = model(ids).logits
    finally:
        mamba_cpu.hf.unpatch_transformers()
    assert calls == []
    assert torch.equal(got, want)


@pytest.mark.gpu
@per_family
def test_patched_model_used_as_installed(family, calls):
    """patch_transformers() over whatever transformers installed (no pinning
    of its fallbacks): generation and a training step run through this
    package."""
    model = tiny_model(family)
    ids = token_ids((1, 9))
    mamba_cpu.hf.patch_transformers()
    try:
        model.generate(ids, max_new_tokens=3, do_sample=False)
        model.train()
        model(ids, labels=ids).loss.backward()
    finally:
        mamba_cpu.hf.unpatch_transformers()
    assert used_the_scan(calls)


@pytest.mark.gpu
@pytest.mark.parametrize("family", ["mamba", "falcon_mamba", "mamba2"])
def test_graph_replayed_greedy_equals_generate(family):
    import mamba_cpu.decode

    model = tiny_model(family)
    ids = token_ids((3, 7))
    with gpu_kernels():
        # an explicit mask: generate would otherwise mask prompt tokens equal to the pad id
        want = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=20,
                              min_new_tokens=20, do_sample=False)
        got = mamba_cpu.decode.greedy_generate(model, ids, 20)
    assert torch.equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("family", ["mamba", "mamba2"])
def test_each_graph_replay_equals_the_eager_step(family):
    """Every replay of the captured decode step against the eager step on the
    same token and cache, with eager work and synchronisations between
    replays."""
    import mamba_cpu.decode

    model = tiny_model(family)
    prompt, steps = token_ids((2, 9)), token_ids((2, 12), seed=2)
    with gpu_kernels(), torch.no_grad():
        cache = model(prompt, use_cache=True).cache_params
        eager = [model(input_ids=steps[:, i:i + 1], cache_params=cache, use_cache=True).logits[:, -1].clone()
                 for i in range(steps.shape[1])]
        # the model's own step, captured (the fused block steps have their own test)
        graphed = mamba_cpu.decode.GraphedDecodeStep(model, model(prompt, use_cache=True).cache_params, 2,
                                                     fused=False)
        for i in range(steps.shape[1]):
            graphed.token.copy_(steps[:, i:i + 1])
            got = graphed.replay().clone()
            if i % 3 == 0:
                torch.cuda.synchronize()
            assert torch.equal(got, eager[i]), f"replay {i}"


@pytest.mark.gpu
def test_mamba_130m_width_two_layers_agrees_with_transformers():
    """Two layers of the Mamba-130M architecture (d_model 768, d_inner 1536,
    dstate 16, dt_rank 48, conv width 4, vocabulary 50280), random init,
    float32: prefill logits of 2 x 256 random tokens, 16 greedy steps, and a
    training step of 2 x 128, on this package against transformers' torch
    kernels. Bounds: largest |logit difference| 1e-3 (logits reach a few
    units), top-1 agreement at every position, identical greedy tokens, and a
    worst per-tensor gradient error max|dg| / max|g| of 1e-4."""
    torch.manual_seed(0)
    cfg = transformers.MambaConfig(num_hidden_layers=2, hidden_size=768, state_size=16, expand=2,
                                   conv_kernel=4, vocab_size=50280)
    model = transformers.MambaForCausalLM(cfg).to(DEV).eval()
    ids = token_ids((2, 256), vocab=50280)
    got, want = torch_then_gpu(lambda: model(ids).logits.detach())
    dlogit = (got - want).abs().max().item()
    top1 = (got.argmax(-1) == want.argmax(-1)).float().mean().item()
    print(f"  max|dlogit| {dlogit:.3g} (max|logit| {want.abs().max().item():.3g}), top-1 agreement {top1}")
    assert dlogit < 1e-3 and top1 == 1.0
    gen, gen_want = torch_then_gpu(lambda: model.generate(ids[:, :32], max_new_tokens=16,
                                                          min_new_tokens=16, do_sample=False))
    assert torch.equal(gen, gen_want)
    model.train()
    train_ids = ids[:, :128]

    def step():
        model.zero_grad()
        loss = model(train_ids, labels=train_ids).loss
        loss.backward()
        return loss.item(), {k: p.grad.clone() for k, p in model.named_parameters() if p.grad is not None}

    (loss, grads), (loss_want, grads_want) = torch_then_gpu(step)
    worst = max(((grads[k] - g).abs().max() / g.abs().max().clamp_min(1e-12)).item()
                for k, g in grads_want.items())
    print(f"  train loss {loss:.6f} vs {loss_want:.6f}, worst per-tensor gradient error {worst:.3g}")
    assert abs(loss - loss_want) <= 1e-5 * abs(loss_want)
    assert worst < 1e-4


@pytest.mark.gpu
def test_mamba2_head_shape_two_layers_agrees_with_transformers():
    """Two Mamba-2 layers with the 2.7B model's head shape (headdim 64,
    dstate 128, one group; 16 heads of d_model 512), random init, float32:
    prefill logits of 2 x 300 tokens, 16 greedy steps (the decode path:
    selective_state_update in the head layout and the conv update), and a
    training step of 2 x 200, on this package against transformers' torch
    kernels (which chunk by 256 where the package's kernels chunk by 64);
    the graph-replayed greedy decoder gives the same tokens.
    Bounds: largest |logit difference| 1e-3, top-1 agreement at every
    position, identical greedy tokens, worst per-tensor gradient error
    max|dg| / max|g| of 1e-3."""
    torch.manual_seed(0)
    cfg = transformers.Mamba2Config(num_hidden_layers=2, hidden_size=512, num_heads=16, head_dim=64,
                                    state_size=128, n_groups=1, expand=2, conv_kernel=4, vocab_size=1000,
                                    chunk_size=256)
    model = transformers.Mamba2ForCausalLM(cfg).to(DEV).eval()
    ids = token_ids((2, 300), vocab=1000)
    got, want = torch_then_gpu(lambda: model(ids).logits.detach())
    dlogit = (got - want).abs().max().item()
    top1 = (got.argmax(-1) == want.argmax(-1)).float().mean().item()
    print(f"  max|dlogit| {dlogit:.3g} (max|logit| {want.abs().max().item():.3g}), top-1 agreement {top1}")
    assert dlogit < 1e-3 and top1 == 1.0
    prompt = ids[:, :40]
    gen, gen_want = torch_then_gpu(lambda: model.generate(prompt, attention_mask=torch.ones_like(prompt),
                                                          max_new_tokens=16, min_new_tokens=16,
                                                          do_sample=False))
    assert torch.equal(gen, gen_want)
    import mamba_cpu.decode

    with gpu_kernels():  # the decode step replayed from a HIP graph gives the same tokens
        assert torch.equal(mamba_cpu.decode.greedy_generate(model, prompt, 16), gen)
    model.train()
    train_ids = ids[:, :200]

    def step():
        model.zero_grad()
        loss = model(train_ids, labels=train_ids).loss
        loss.backward()
        return loss.item(), {k: p.grad.clone() for k, p in model.named_parameters() if p.grad is not None}

    (loss, grads), (loss_want, grads_want) = torch_then_gpu(step)
    worst = max(((grads[k] - g).abs().max() / g.abs().max().clamp_min(1e-12)).item()
                for k, g in grads_want.items())
    print(f"  train loss {loss:.6f} vs {loss_want:.6f}, worst per-tensor gradient error {worst:.3g}")
    assert grads.keys() == grads_want.keys()
    assert abs(loss - loss_want) <= 1e-5 * abs(loss_want)
    assert worst < 1e-3


def assert_greedy_agrees(model, prompt, got, want, min_steps, tie):
    """Greedy token sequences of two paths (each (batch, prompt + new)) agree
    for at least `min_steps` new tokens, and where they first part, the two
    chosen tokens are a near-tie: their logits after the common prefix differ
    by at most `tie` on both paths (float32 reordering decides such a pick)."""
    if torch.equal(got, want):
        return
    n0 = prompt.shape[1]
    i = int((got != want).any(0).nonzero()[0])
    assert i - n0 >= min_steps, f"tokens part at new token {i - n0}"
    prefix = got[:, :i]
    with torch.no_grad():
        last, last_want = torch_then_gpu(lambda: model(prefix).logits[:, -1])
    for r in (got[:, i] != want[:, i]).nonzero().flatten().tolist():
        a, b = int(got[r, i]), int(want[r, i])
        for lg in (last, last_want):
            gap = (lg[r, a] - lg[r, b]).abs().item()
            print(f"  row {r} parts at new token {i - n0}: tokens {a} / {b}, logit gap {gap:.3g}")
            assert gap <= tie


@pytest.mark.gpu
def test_mamba_130m_full_architecture_agrees_with_transformers():
    """The Mamba-130M architecture at its full size (24 layers, d_model 768,
    d_inner 1536, dstate 16, dt_rank 48, conv width 4, vocabulary 50280),
    random init, float32, on this package against transformers' torch kernels
    on the same GPU, with the reference's model-level measures
    (benchmarks/check_hf_model.py:105-121): prefill logits of 4 x 1024 random
    tokens (largest |logit difference| 0.02 with logits up to about 17,
    top-1 agreement at least 0.998 of the positions); 128 greedy decode steps
    through model.generate, and through the graph-replayed decoder, with the
    tokens identical for at least the first 16 and the first parting, if
    any, a near-tie (logit gap within 0.02, the prefill bound: random weights
    give flat logits, and a pick decided by float32 rounding sends the two
    sequences apart after it); one training step of 4 x 256 (loss within 1e-5
    relative, worst per-tensor gradient error max|dg| / max|g| of 1e-2).
    These are the float32 reordering floor: the two paths sum the scan, the
    convolution and the GEMMs in different orders, and 24 layers amplify it."""
    import mamba_cpu.decode

    torch.manual_seed(0)
    cfg = transformers.MambaConfig(num_hidden_layers=24, hidden_size=768, state_size=16, expand=2,
                                   conv_kernel=4, vocab_size=50280)
    model = transformers.MambaForCausalLM(cfg).to(DEV).eval()
    ids = token_ids((4, 1024), vocab=50280)
    with torch.no_grad():
        got, want = torch_then_gpu(lambda: model(ids).logits)
    dlogit = (got - want).abs().max().item()
    top1 = (got.argmax(-1) == want.argmax(-1)).float().mean().item()
    print(f"  prefill: max|dlogit| {dlogit:.3g} (max|logit| {want.abs().max().item():.3g}), top-1 agreement {top1}")
    del got, want
    assert dlogit < 2e-2 and top1 >= 0.998
    prompt = ids[:, :16]
    gen, gen_want = torch_then_gpu(lambda: model.generate(prompt, max_new_tokens=128, min_new_tokens=128,
                                                          do_sample=False))
    print(f"  128 greedy steps: token agreement {(gen == gen_want).float().mean().item()}")
    assert_greedy_agrees(model, prompt, gen, gen_want, 16, 2e-2)
    with gpu_kernels():
        graphed = mamba_cpu.decode.greedy_generate(model, prompt, 128)
    print(f"  graph-replayed decoder: token agreement {(graphed == gen).float().mean().item()}")
    assert_greedy_agrees(model, prompt, graphed, gen, 16, 2e-2)
    model.train()
    train_ids = ids[:, :256]

    def step():
        model.zero_grad()
        loss = model(train_ids, labels=train_ids).loss
        loss.backward()
        return loss.item(), {k: p.grad.clone() for k, p in model.named_parameters() if p.grad is not None}

    (loss, grads), (loss_want, grads_want) = torch_then_gpu(step)
    errs = {k: ((grads[k] - g).abs().max() / g.abs().max().clamp_min(1e-12)).item() for k, g in grads_want.items()}
    worst = max(errs, key=errs.get)
    print(f"  train loss {loss:.7f} vs {loss_want:.7f}, worst per-tensor gradient error {errs[worst]:.3g} ({worst})")
    assert grads.keys() == grads_want.keys()
    assert abs(loss - loss_want) <= 1e-5 * abs(loss_want)
    assert errs[worst] < 1e-2
