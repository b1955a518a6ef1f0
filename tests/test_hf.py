"""mamba_cpu.hf against transformers' own pure-torch fallbacks, on small random
models (the cases of the reference's tests/test_hf.py, on the GPU), and the
graph-replayed greedy decoder (mamba_cpu.decode) against model.generate.

The baseline runs the same model on the same GPU through transformers'
fallback functions (pinned through `__wrapped__`, as the reference's tests
pin them); the patched run goes through this package's HIP ops."""

import importlib

import pytest
import torch

pytest.importorskip("transformers", minversion="5.0")

import transformers

import mamba_cpu.hf
from mamba_cpu import selective_scan_fn

SMALL = dict(vocab_size=64, hidden_size=32, num_hidden_layers=2, state_size=8, conv_kernel=4, expand=2)
DEV = "cuda"


def build(name, dev=DEV):
    torch.manual_seed(0)
    if name == "mamba":
        model = transformers.MambaForCausalLM(transformers.MambaConfig(**SMALL))
    elif name == "falcon_mamba":
        model = transformers.FalconMambaForCausalLM(transformers.FalconMambaConfig(**SMALL))
    else:
        config = transformers.JambaConfig(
            vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=2, num_attention_heads=2,
            num_key_value_heads=2, num_experts=1, attn_layer_period=2, attn_layer_offset=1,
            expert_layer_period=2, expert_layer_offset=1, mamba_d_state=8, mamba_dt_rank=4,
            use_mamba_kernels=False,
        )
        model = transformers.JambaForCausalLM(config)
    return model.to(dev).eval()


@pytest.fixture
def patched(monkeypatch):
    """Runs fn on transformers' pure-torch fallbacks, then on mamba_cpu."""
    mamba_cpu.hf.unpatch_transformers()
    for name in mamba_cpu.hf.SUPPORTED_MODELS:
        module = importlib.import_module(f"transformers.models.{name}.modeling_{name}")
        for op in mamba_cpu.hf._OPS:
            monkeypatch.setattr(module, op, getattr(module, op).__wrapped__)

    def run_both(fn):
        want = fn()
        mamba_cpu.hf.patch_transformers()
        try:
            return fn(), want
        finally:
            mamba_cpu.hf.unpatch_transformers()

    return run_both


@pytest.fixture
def scan_calls(monkeypatch):
    """Counts scans through this package: the scan op, or the fused mixer
    (mamba_inner_fn) that transformers' Mamba mixers call in training."""
    calls = []
    monkeypatch.setattr(
        mamba_cpu.hf, "selective_scan_fn", lambda *a: calls.append(1) or selective_scan_fn(*a)
    )
    fused = mamba_cpu.hf.mamba_inner_fn
    monkeypatch.setattr(
        mamba_cpu.hf, "mamba_inner_fn", lambda *a, **k: calls.append(2) or fused(*a, **k)
    )
    return calls


models = pytest.mark.parametrize("name", mamba_cpu.hf.SUPPORTED_MODELS)


def _ids(shape, dev=DEV):
    g = torch.Generator().manual_seed(1)
    return torch.randint(0, 64, shape, generator=g).to(dev)


@pytest.mark.gpu
@models
def test_logits_match(name, patched, scan_calls):
    model = build(name)
    ids = _ids((2, 37))

    def logits():
        with torch.no_grad():
            return model(ids).logits

    got, want = patched(logits)
    assert scan_calls, "patched scan was not used"
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
@models
def test_generate_matches(name, patched, scan_calls):
    model = build(name)
    ids = _ids((2, 11))
    got, want = patched(lambda: model.generate(ids, max_new_tokens=12, do_sample=False))
    assert scan_calls
    assert torch.equal(got, want)


@pytest.mark.gpu
@models
def test_padded_batch_matches(name, patched):
    model = build(name)
    ids = _ids((2, 16))
    mask = torch.ones_like(ids)
    mask[1, :5] = 0

    def logits():
        with torch.no_grad():
            return model(ids, attention_mask=mask).logits

    got, want = patched(logits)
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-4)


@pytest.mark.gpu
@models
def test_training_gradients_match(name, patched, scan_calls):
    model = build(name).train()
    ids = _ids((2, 24))

    def grads():
        model.zero_grad()
        model(ids, labels=ids).loss.backward()
        return {k: p.grad.clone() for k, p in model.named_parameters() if p.grad is not None}

    got, want = patched(grads)
    assert scan_calls and got.keys() == want.keys()
    if name == "mamba":  # FalconMamba keeps its unfused path (its norms differ from the fused ones)
        assert 2 in scan_calls, "the fused mixer was not used"
    for k in want:
        torch.testing.assert_close(got[k], want[k], rtol=1e-3, atol=1e-4, msg=lambda m: f"{k}: {m}")


def test_patch_is_idempotent_and_reversible():
    module = importlib.import_module("transformers.models.mamba.modeling_mamba")
    original = module.mamba_selective_scan
    mamba_cpu.hf.patch_transformers()
    patched_fn = module.mamba_selective_scan
    mamba_cpu.hf.patch_transformers()
    assert module.mamba_selective_scan is patched_fn is not original
    mamba_cpu.hf.unpatch_transformers()
    assert module.mamba_selective_scan is original


def test_cpu_tensors_keep_transformers_path(scan_calls):
    # The routing predicate: tensors on other devices keep transformers' own ops.
    model = build("mamba", dev="cpu")
    ids = _ids((1, 9), dev="cpu")
    with torch.no_grad():
        want = model(ids).logits
    mamba_cpu.hf.patch_transformers()
    try:
        with torch.no_grad():
            got = model(ids).logits
    finally:
        mamba_cpu.hf.unpatch_transformers()
    assert not scan_calls
    torch.testing.assert_close(got, want, rtol=0, atol=0)


@pytest.mark.gpu
@models
def test_patched_model_runs_as_installed(name, scan_calls):
    model = build(name)
    ids = _ids((1, 9))
    mamba_cpu.hf.patch_transformers()
    try:
        model.generate(ids, max_new_tokens=3, do_sample=False)
        model.train()
        model(ids, labels=ids).loss.backward()
    finally:
        mamba_cpu.hf.unpatch_transformers()
    assert scan_calls


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["mamba", "falcon_mamba"])
def test_graphed_greedy_matches_generate(name):
    import mamba_cpu.decode

    model = build(name)
    ids = _ids((3, 7))
    mamba_cpu.hf.patch_transformers()
    try:
        want = model.generate(ids, max_new_tokens=20, min_new_tokens=20, do_sample=False)
        got = mamba_cpu.decode.greedy_generate(model, ids, 20)
    finally:
        mamba_cpu.hf.unpatch_transformers()
    assert torch.equal(got, want)


@pytest.mark.gpu
def test_graph_replays_match_eager_steps():
    # Every replay against the eager step on the same token and cache, with
    # eager work and synchronisations between the replays.
    import mamba_cpu.decode

    model = build("mamba")
    ids = _ids((2, 9))
    toks = _ids((2, 12))
    mamba_cpu.hf.patch_transformers()
    try:
        with torch.no_grad():
            cache = model(ids, use_cache=True).cache_params
            eager = []
            for i in range(toks.shape[1]):
                eager.append(model(input_ids=toks[:, i:i + 1], cache_params=cache, use_cache=True)
                             .logits[:, -1].clone())
            cache = model(ids, use_cache=True).cache_params
            step = mamba_cpu.decode.GraphedDecodeStep(model, cache, 2)
            for i in range(toks.shape[1]):
                step.token.copy_(toks[:, i:i + 1])
                got = step.replay().clone()
                if i % 3 == 0:
                    torch.cuda.synchronize()
                torch.testing.assert_close(got, eager[i], rtol=0, atol=0, msg=lambda m: f"step {i}: {m}")
    finally:
        mamba_cpu.hf.unpatch_transformers()
