"""The fused single-token Mamba block step (mamba_cpu::mixer_step, used by
mamba_cpu.decode) against transformers' own decode step.

- model level, float32, two layers of the Mamba-130M width (d_model 768,
  d_inner 1536, dstate 16, dt_rank 48, width 4, vocabulary 50280), batch 4:
  8 fused decode steps on the GPU against the same model on the CPU through
  transformers' pure-torch path, logits and every cache tensor (logits reach
  about 14: rtol 1e-4, atol 1e-4; SSM states reach about 100 after 24 steps
  and conv windows about 13: rtol 1e-4, atol 1e-3);
- block level, float32 and bfloat16 (residual in float32), batch 1 to 8:
  one fused block step against the block's own forward on the GPU (its
  kernels routed to this package), output and both states (float32: rtol
  1e-4, atol 1e-5 where outputs stay below 4 (the 32-wide model), atol 1e-3
  at the 768 and 1024 widths, whose outputs reach about 100 on
  unit-variance inputs, 5e-6 of the largest output at the 2560 width, where
  outputs reach 5e4 and the products' float32 summation order alone moves
  them by 2e-6 of that; bfloat16: 2e-2 / 2e-2).
  The widths cover both ways the step runs x_proj: as partial sums of the
  in_proj workgroups (32, 768 and 1024, the last with 4 in_proj rows per
  wave) and, at d_inner 4096 and the Mamba-2.8B width (d_inner 5120, dt_rank
  160), as its own product. d_inner 4096 at batch 8 stages 8 x 4096 floats,
  the most a workgroup's LDS takes; the 5120 width at batch 8 is past it and
  keeps the unfused step (tokens equal to transformers' generate);
- the final norm and lm_head as one launch (mamba_cpu::norm_linear) against
  transformers' MambaRMSNorm and nn.Linear on the GPU: float32 (rtol 1e-5,
  atol 1e-5 of the largest logit) and bfloat16 weights with float32 or
  bfloat16 rows (results rounded to bfloat16: rtol 1e-2, atol 1e-2 of the
  largest), widths 32 to 2560 (one and two passes over d_in), batch 1 to 8,
  with and without norm weight and bias, at the 50280-word vocabulary;
- Mamba-2 (mamba_cpu::mamba2_step): one fused block step against the
  block's own recurrent step (its kernels routed to this package) at batch 1
  to 8, float32 and bfloat16, a small model (2 groups, dstate 16) and the
  Mamba-2 130M width (24 heads x 64, dstate 128; same tolerances as Mamba);
  8 fused decode steps of a two-layer 130M-width model against transformers
  on the CPU (logits and every cache tensor, tolerances as Mamba's);
- the captured graph against eager fused steps, bitwise (Mamba and Mamba-2),
  and the torch.library opcheck of every operator.
"""

import copy

import pytest
import torch

pytest.importorskip("transformers", minversion="5.0")

import transformers

import mamba_cpu.decode as dec
import mamba_cpu.hf
from conftest import assert_close_report

pytestmark = pytest.mark.gpu
DEV = "cuda"
W130 = dict(num_hidden_layers=2, hidden_size=768, state_size=16, expand=2, conv_kernel=4, vocab_size=50280)
TINY = dict(vocab_size=64, hidden_size=32, num_hidden_layers=2, state_size=8, conv_kernel=4, expand=2)
W1024 = dict(num_hidden_layers=1, hidden_size=1024, state_size=16, expand=2, conv_kernel=4, vocab_size=64)
W2048 = dict(num_hidden_layers=1, hidden_size=2048, state_size=16, expand=2, conv_kernel=4, vocab_size=64)
W2560 = dict(num_hidden_layers=1, hidden_size=2560, state_size=16, expand=2, conv_kernel=4, vocab_size=64)
CFGS = {"tiny": TINY, "768": W130, "1024": W1024, "2048": W2048, "2560": W2560}
M2_TINY = dict(vocab_size=64, hidden_size=64, num_hidden_layers=2, num_heads=4, head_dim=32, state_size=16,
               n_groups=2, expand=2, conv_kernel=4, chunk_size=16)
M2_130 = dict(vocab_size=50280, hidden_size=768, num_hidden_layers=2, num_heads=24, head_dim=64, state_size=128,
              n_groups=1, expand=2, conv_kernel=4, chunk_size=256)


@pytest.fixture(autouse=True)
def patched():
    mamba_cpu.hf.patch_transformers()
    yield
    mamba_cpu.hf.unpatch_transformers()


def mamba(cfg, dtype=torch.float32, seed=0):
    torch.manual_seed(seed)
    return transformers.MambaForCausalLM(transformers.MambaConfig(**cfg)).to(DEV, dtype).eval()


def ids(shape, vocab, seed=1):
    return torch.randint(0, vocab, shape, generator=torch.Generator().manual_seed(seed))


def states(cache):
    out = []
    for layer in cache.layers:
        out += [layer.conv_states[0], layer.recurrent_states[0]]
    return out


@torch.no_grad()
def test_fused_decode_matches_transformers_on_the_cpu():
    model = mamba(W130)
    cpu_model = copy.deepcopy(model).cpu()
    prompt, toks = ids((4, 16), 50280), ids((4, 8), 50280, seed=2)
    cache = model(prompt.to(DEV), use_cache=True).cache_params
    cpu_cache = cpu_model(prompt, use_cache=True).cache_params
    assert dec.fused_step_supported(model, cache, 4)
    for i in range(toks.shape[1]):
        got = dec.fused_model_step(model, toks[:, i:i + 1].to(DEV), cache)
        want = cpu_model(input_ids=toks[:, i:i + 1], cache_params=cpu_cache, use_cache=True).logits[:, -1]
        assert_close_report(got, want, 1e-4, 1e-4, f"logits step {i}")
    for k, (g, w) in enumerate(zip(states(cache), states(cpu_cache))):
        assert_close_report(g, w, 1e-4, 1e-3, f"cache tensor {k}")


@pytest.mark.parametrize("width,batch", [("tiny", 1), ("tiny", 3), ("768", 4), ("tiny", 8), ("768", 8),
                                         ("1024", 2), ("2048", 8), ("2560", 2)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@torch.no_grad()
def test_fused_block_step_matches_the_block(width, batch, dtype):
    model = mamba(CFGS[width], dtype)
    vocab = model.config.vocab_size
    cache = model(ids((batch, 12), vocab).to(DEV), use_cache=True).cache_params
    ref_cache = copy.deepcopy(cache)
    gen = torch.Generator(device=DEV).manual_seed(3)
    for blk in model.backbone.layers:
        h = torch.randn(batch, model.config.hidden_size, generator=gen, device=DEV).to(dtype)
        got = dec.fused_block_step(blk, h, cache)
        want = blk(h[:, None], cache_params=ref_cache)[:, 0]
        assert got.dtype == want.dtype and got.shape == want.shape
        if dtype == torch.float32:
            hs = model.config.hidden_size
            # at the 2560 width outputs reach 5e4 and sums of 5120 products
            # cancel to a few hundred: float32 summation order alone moves
            # them by up to 2e-6 of the largest output
            big = 5e-6 * want.abs().max().item()
            tol = (1e-4, 1e-5) if hs <= 32 else (1e-4, 1e-3) if hs <= 1024 else (1e-4, big)
        else:
            tol = (2e-2, 2e-2)
        assert_close_report(got, want, *tol, f"layer {blk.layer_idx} out")
        layer, ref = cache.layers[blk.layer_idx], ref_cache.layers[blk.layer_idx]
        assert_close_report(layer.conv_states[0], ref.conv_states[0], *tol, "conv state")
        assert_close_report(layer.recurrent_states[0], ref.recurrent_states[0], *tol, "ssm state")


@torch.no_grad()
def test_graph_replays_equal_eager_fused_steps():
    model = mamba(TINY)
    prompt, toks = ids((2, 9), 64).to(DEV), ids((2, 10), 64, seed=2).to(DEV)
    cache = model(prompt, use_cache=True).cache_params
    eager = [dec.fused_model_step(model, toks[:, i:i + 1], cache).clone() for i in range(toks.shape[1])]
    graphed = dec.GraphedDecodeStep(model, model(prompt, use_cache=True).cache_params, 2)
    assert graphed.fused
    for i in range(toks.shape[1]):
        graphed.token.copy_(toks[:, i:i + 1])
        got = graphed.replay().clone()
        if i % 3 == 0:
            torch.cuda.synchronize()
        assert torch.equal(got, eager[i]), f"replay {i}"


@torch.no_grad()
def test_unsupported_models_keep_the_unfused_step():
    model = mamba(TINY)
    cache = model(ids((9, 4), 64).to(DEV), use_cache=True).cache_params
    assert not dec.fused_step_supported(model, cache, 9)   # more than 8 batch rows
    falcon = transformers.FalconMambaForCausalLM(transformers.FalconMambaConfig(**TINY)).to(DEV).eval()
    fcache = falcon(ids((2, 4), 64).to(DEV), use_cache=True).cache_params
    assert not dec.fused_step_supported(falcon, fcache, 2)


@torch.no_grad()
def test_widths_past_the_lds_limit_keep_the_unfused_step():
    """At the Mamba-2.8B width (d_inner 5120) batch 8 needs more LDS than a
    workgroup holds (8 x 5120 floats), so decoding keeps the unfused step and
    still matches transformers' own; at batch 2 the same model is fused."""
    model = mamba(W2560)
    prompt = ids((8, 5), 64).to(DEV)
    assert dec.fused_step_supported(model, model(prompt[:2], use_cache=True).cache_params, 2)
    cache = model(prompt, use_cache=True).cache_params
    assert not dec.fused_step_supported(model, cache, 8)
    step = dec.GraphedDecodeStep(model, cache, 8)
    assert not step.fused
    toks = dec.greedy_generate(model, prompt, 3)
    want = model.generate(prompt, max_new_tokens=3, min_new_tokens=3, do_sample=False)
    assert torch.equal(toks.cpu(), want.cpu())


def test_opcheck_mixer_step():
    model = mamba(TINY)
    with torch.no_grad():
        cache = model(ids((3, 5), 64).to(DEV), use_cache=True).cache_params
    blk = model.backbone.layers[0]
    mx = blk.mixer
    A, D, dtb = dec._block_constants(mx)
    layer = cache.layers[0]
    h = torch.randn(3, 32, device=DEV)
    args = (h, blk.norm.weight.detach(), 1e-5, True, True, mx.in_proj.weight.detach(), None,
            mx.conv1d.weight.detach().view(mx.intermediate_size, -1), mx.conv1d.bias.detach(),
            layer.conv_states[0], mx.x_proj.weight.detach(), mx.dt_proj.weight.detach(), dtb, A, D,
            layer.recurrent_states[0], mx.out_proj.weight.detach(), None)
    torch.library.opcheck(torch.ops.mamba_cpu.mixer_step.default, args)


@pytest.mark.parametrize("dtype,hdtype,batch,d_in,d_out,norm,bias", [
    (torch.float32, torch.float32, 4, 768, 50280, True, False),
    (torch.float32, torch.float32, 1, 1536, 1000, True, True),
    (torch.float32, torch.float32, 8, 2560, 333, True, False),
    (torch.float32, torch.float32, 3, 32, 64, False, True),
    (torch.bfloat16, torch.float32, 4, 768, 50280, True, False),
    (torch.bfloat16, torch.bfloat16, 2, 1024, 777, True, True),
    (torch.bfloat16, torch.bfloat16, 5, 768, 129, False, False),
], ids=["f32-768-vocab", "f32-1536-bias", "f32-2560-b8", "f32-nonorm", "bf16-f32rows-vocab", "bf16-bf16rows",
        "bf16-nonorm"])
@torch.no_grad()
def test_norm_linear_matches_norm_and_head(dtype, hdtype, batch, d_in, d_out, norm, bias):
    gen = torch.Generator(device=DEV).manual_seed(7)
    h = (torch.randn(batch, d_in, generator=gen, device=DEV) * 3).to(hdtype)
    norm_f = transformers.models.mamba.modeling_mamba.MambaRMSNorm(d_in, eps=1e-5).to(DEV, dtype)
    norm_f.weight.copy_(1 + 0.1 * torch.randn(d_in, generator=gen, device=DEV))
    head = torch.nn.Linear(d_in, d_out, bias=bias).to(DEV, dtype)
    head.weight.copy_(torch.randn(d_out, d_in, generator=gen, device=DEV) * 0.05)
    if bias:
        head.bias.copy_(torch.randn(d_out, generator=gen, device=DEV))
    got = torch.ops.mamba_cpu.norm_linear(h, norm_f.weight if norm else None, 1e-5, head.weight, head.bias, True)
    u = norm_f(h) if norm else h
    want = head(u.to(dtype)).float()
    assert got.dtype == torch.float32 and got.shape == want.shape
    scale = want.abs().max().item()
    tol = (1e-5, 1e-5 * scale) if dtype == torch.float32 else (1e-2, 1e-2 * scale)
    assert_close_report(got, want, *tol, "logits")
    low = torch.ops.mamba_cpu.norm_linear(h, norm_f.weight if norm else None, 1e-5, head.weight, head.bias, False)
    assert low.dtype == dtype and torch.equal(low.float(), got)


def test_opcheck_norm_linear():
    gen = torch.Generator(device=DEV).manual_seed(8)
    args = (torch.randn(3, 32, generator=gen, device=DEV), torch.rand(32, generator=gen, device=DEV) + 0.5, 1e-5,
            torch.randn(70, 32, generator=gen, device=DEV), None, True)
    torch.library.opcheck(torch.ops.mamba_cpu.norm_linear.default, args)


def mamba2(cfg, dtype=torch.float32, seed=0):
    torch.manual_seed(seed)
    return transformers.Mamba2ForCausalLM(transformers.Mamba2Config(**cfg)).to(DEV, dtype).eval()


@pytest.mark.parametrize("width,batch", [("tiny", 1), ("tiny", 3), ("130m", 4), ("tiny", 8), ("130m", 8)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@torch.no_grad()
def test_fused_mamba2_block_step_matches_the_block(width, batch, dtype):
    model = mamba2(M2_TINY if width == "tiny" else M2_130, dtype)
    vocab = model.config.vocab_size
    cache = model(ids((batch, 12), vocab).to(DEV), use_cache=True).cache_params
    assert dec.fused_step_supported(model, cache, batch)
    ref_cache = copy.deepcopy(cache)
    gen = torch.Generator(device=DEV).manual_seed(3)
    for blk in model.backbone.layers:
        h = torch.randn(batch, model.config.hidden_size, generator=gen, device=DEV).to(dtype)
        got = dec.fused_block_step(blk, h, cache)
        want = blk(h[:, None], cache_params=ref_cache)[:, 0]
        assert got.dtype == want.dtype and got.shape == want.shape
        if dtype == torch.float32:
            tol = (1e-4, 1e-5) if model.config.hidden_size <= 64 else (1e-4, 1e-3)
        else:
            tol = (2e-2, 2e-2)
        assert_close_report(got, want, *tol, f"layer {blk.layer_idx} out")
        layer, ref = cache.layers[blk.layer_idx], ref_cache.layers[blk.layer_idx]
        assert_close_report(layer.conv_states[0], ref.conv_states[0], *tol, "conv state")
        assert_close_report(layer.recurrent_states[0], ref.recurrent_states[0], *tol, "ssm state")


@torch.no_grad()
def test_fused_mamba2_decode_matches_transformers_on_the_cpu():
    model = mamba2(M2_130)
    cpu_model = copy.deepcopy(model).cpu()
    prompt, toks = ids((4, 16), 50280), ids((4, 8), 50280, seed=2)
    cache = model(prompt.to(DEV), use_cache=True).cache_params
    cpu_cache = cpu_model(prompt, use_cache=True).cache_params
    assert dec.fused_step_supported(model, cache, 4)
    for i in range(toks.shape[1]):
        got = dec.fused_model_step(model, toks[:, i:i + 1].to(DEV), cache)
        want = cpu_model(input_ids=toks[:, i:i + 1], cache_params=cpu_cache, use_cache=True).logits[:, -1]
        assert_close_report(got, want, 1e-4, 1e-4, f"logits step {i}")
    for k, (g, w) in enumerate(zip(states(cache), states(cpu_cache))):
        assert_close_report(g, w, 1e-4, 1e-3, f"cache tensor {k}")


@torch.no_grad()
def test_mamba2_graph_replays_equal_eager_fused_steps():
    model = mamba2(M2_TINY)
    prompt, toks = ids((2, 9), 64).to(DEV), ids((2, 10), 64, seed=2).to(DEV)
    cache = model(prompt, use_cache=True).cache_params
    eager = [dec.fused_model_step(model, toks[:, i:i + 1], cache).clone() for i in range(toks.shape[1])]
    graphed = dec.GraphedDecodeStep(model, model(prompt, use_cache=True).cache_params, 2)
    assert graphed.fused
    for i in range(toks.shape[1]):
        graphed.token.copy_(toks[:, i:i + 1])
        got = graphed.replay().clone()
        if i % 3 == 0:
            torch.cuda.synchronize()
        assert torch.equal(got, eager[i]), f"replay {i}"


def test_opcheck_mamba2_step():
    model = mamba2(M2_TINY)
    with torch.no_grad():
        cache = model(ids((3, 5), 64).to(DEV), use_cache=True).cache_params
    blk = model.backbone.layers[0]
    mx = blk.mixer
    A, D, dtb = dec._block_constants(mx)
    layer = cache.layers[0]
    h = torch.randn(3, 64, device=DEV)
    args = (h, blk.norm.weight.detach(), 1e-5, True, True, mx.in_proj.weight.detach(), None,
            mx.conv1d.weight.detach().view(mx.conv1d.weight.shape[0], -1), mx.conv1d.bias.detach(),
            layer.conv_states[0], dtb, A, D, layer.recurrent_states[0], mx.norm.weight.detach(), 1e-5,
            mx.out_proj.weight.detach(), None)
    torch.library.opcheck(torch.ops.mamba_cpu.mamba2_step.default, args)
