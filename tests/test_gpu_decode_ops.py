"""Fused decode-step model ops (fl_gemv_bf16, fl_norm_chain, fl_gemv_bf16_chain) against the
torch modules they replace, and the fused engine step against the module step."""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

from flashloop_amd import kernels  # noqa: E402
from flashloop_amd.engine import FlashLoopEngine  # noqa: E402
from flashloop_amd.model import OuroConfig, OuroForCausalLM, RMSNorm, apply_rope  # noqa: E402

DEV = "cuda"


def _w(n, k, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)


def _x(m, k, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(m, k, generator=g, device=DEV).to(dtype)


def _close_bf16(got, want, what, cancel=False):
    """Both sides round an fp32 dot product to bf16; summation order may move a value by
    one bf16 ulp (2^-8 relative), nothing more.  With ``cancel`` (RoPE: a sum of two
    rounded products) the ulp is that of the largest value of the row."""
    got, want = got.float(), want.float()
    tol = want.abs() * 2.0 ** -7 + 1e-6
    if cancel:
        tol = tol + want.abs().amax(dim=-1, keepdim=True) * 2.0 ** -7
    bad = ((got - want).abs() > tol).sum().item()
    assert bad == 0, f"{what}: {bad} values beyond one ulp; max diff {(got - want).abs().max().item()}"
    exact = (got == want).float().mean().item()
    assert exact > 0.9, f"{what}: only {exact:.3f} of the values equal the module's"


@pytest.mark.parametrize("m,n,k", [(1, 2048, 2048), (3, 2048, 5632), (8, 512, 2048), (1, 49152, 2048)])
def test_gemv_plain_and_f32(m, n, k):
    print(f"case: gemv m={m} n={n} k={k}", flush=True)
    x, w = _x(m, k, 1), _w(n, k, 2)
    want = F.linear(x, w)
    _close_bf16(kernels.gemv(x, [w]), want, "plain")
    got32 = kernels.gemv(x, [w], epilogue=kernels.EPI_F32)
    assert got32.dtype == torch.float32
    _close_bf16(got32, want.float(), "f32")
    assert torch.equal(got32, got32.bfloat16().float())  # the widened bf16 value


def test_gemv_f32_input_and_add():
    print("case: gemv f32 input + addend", flush=True)
    x32 = _x(2, 2048, 3, torch.float32)
    w = _w(2048, 2048, 4)
    add = _x(2, 2048, 5)
    want = F.linear(x32.to(torch.bfloat16), w) + add
    _close_bf16(kernels.gemv(x32, [w], epilogue=kernels.EPI_ADD, addend=add), want, "f32-in add")


def test_gemv_swiglu():
    print("case: gemv swiglu", flush=True)
    x = _x(2, 2048, 6)
    wg, wu = _w(5632, 2048, 7), _w(5632, 2048, 8)
    want = F.silu(F.linear(x, wg)) * F.linear(x, wu)
    _close_bf16(kernels.gemv(x, [wg, wu], epilogue=kernels.EPI_SWIGLU), want, "swiglu")


def test_gemv_rope_qkv():
    print("case: gemv rope qkv", flush=True)
    cfg = OuroConfig(num_hidden_layers=1, vocab_size=256)
    model = OuroForCausalLM.random_init(cfg, seed=3, device=DEV)
    a = model.model.layers[0].self_attn
    b, hd, heads = 3, 128, cfg.num_attention_heads
    x = _x(b, cfg.hidden_size, 9)
    pos = torch.tensor([[5], [4000], [123456]], device=DEV)
    cos, sin = model.model.rotary_emb(x[:, None], pos)
    q, k, v = kernels.gemv(x, [a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], epilogue=kernels.EPI_ROPE,
                           rope=(cos.reshape(b, hd), sin.reshape(b, hd)))
    rq = a.q_proj(x[:, None]).view(b, 1, heads, hd).transpose(1, 2)
    rk = a.k_proj(x[:, None]).view(b, 1, heads, hd).transpose(1, 2)
    rv = a.v_proj(x[:, None]).view(b, 1, heads, hd).transpose(1, 2)
    rq, rk = apply_rope(rq, rk, cos, sin)
    _close_bf16(q.view(b, heads, 1, hd), rq, "q", cancel=True)
    _close_bf16(k.view(b, heads, 1, hd), rk, "k", cancel=True)
    _close_bf16(v.view(b, heads, 1, hd), rv, "v")


def test_norm_chain_matches_modules():
    print("case: norm chain", flush=True)
    d, eps = 2048, 1e-6
    mods = [RMSNorm(d, eps).to(DEV, torch.bfloat16) for _ in range(3)]
    with torch.no_grad():
        for i, mod in enumerate(mods):
            mod.weight.copy_(1.0 + 0.1 * _x(1, d, 20 + i, torch.float32)[0])
    r, x = _x(4, d, 10), _x(4, d, 11) * 3.0
    h, z = kernels.norm_chain(r, x=x, w_a=mods[0].weight, w_f=mods[1].weight, w_b=mods[2].weight, eps=eps)
    wh = mods[1](r + mods[0](x))
    wz = mods[2](wh)
    _close_bf16(h, wh, "h")
    _close_bf16(z, wz, "z")
    h2, z2 = kernels.norm_chain(r, w_b=mods[2].weight, eps=eps, want_h=False)
    assert h2 is None
    _close_bf16(z2, mods[2](r), "z only")


def test_fused_step_tracks_module_step():
    """The fused decode step and the torch-module step agree to bf16 rounding noise."""
    tiny = OuroConfig(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=2)
    model = OuroForCausalLM.random_init(tiny, seed=21, device=DEV)
    g = torch.Generator().manual_seed(21)
    ids = torch.randint(0, tiny.vocab_size, (1, 230), generator=g).to(DEV)
    fused = FlashLoopEngine(model, use_graphs=False)
    mods = FlashLoopEngine(model, use_graphs=False)
    mods.fused_decode = False
    fused.prefill(ids[:, :200], decode_capacity=64)
    mods.prefill(ids[:, :200], decode_capacity=64)
    for i in range(200, 230):
        a = fused.decode(ids[:, i:i + 1]).logits
        b = mods.decode(ids[:, i:i + 1]).logits
        cos = F.cosine_similarity(a.double().flatten(), b.double().flatten(), dim=0).item()
        assert cos > 0.9999, f"step {i}: cos {cos}"
        assert (a - b).abs().max().item() < 2e-2 * max(1.0, b.abs().max().item()), f"step {i}"


@pytest.mark.parametrize("k", [2048, 4096])
@pytest.mark.parametrize("m", [1, 3, 8])
def test_gemv_chain_is_norm_chain_then_gemv(m, k):
    """fl_gemv_bf16_chain equals fl_norm_chain + fl_gemv_bf16 bit for bit (h and the
    output), for every epilogue and every optional part of the chain."""
    print(f"case: gemv chain m={m} k={k}", flush=True)
    eps, hd = 1e-6, 128
    wn = [(1.0 + 0.1 * _x(1, k, 40 + i, torch.float32)[0]).to(torch.bfloat16) for i in range(3)]
    r, x = _x(m, k, 30), _x(m, k, 31) * 3.0
    n = 512
    mats = [_w(n, k, 50 + i) for i in range(3)]
    pos = torch.arange(m, device=DEV) + 7
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, device=DEV).float() / hd))
    ang = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], dim=-1)
    rope = (ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16))
    addend = _x(m, n, 32)
    chains = [dict(x=x, w_a=wn[0], w_b=wn[2]), dict(x=x, w_a=wn[0], w_f=wn[1], w_b=wn[2]),
              dict(w_b=wn[2]), dict(x=x, w_a=wn[0], w_f=wn[1])]
    epis = [(kernels.EPI_PLAIN, mats[:1], {}), (kernels.EPI_F32, mats[:1], {}),
            (kernels.EPI_ADD, mats[:1], dict(addend=addend)), (kernels.EPI_SWIGLU, mats[:2], {}),
            (kernels.EPI_ROPE, mats, dict(rope=rope, head_dim=hd))]
    for ci, ch in enumerate(chains):
        h0, z0 = kernels.norm_chain(r, eps=eps, **ch)
        inp = z0 if ch.get("w_b") is not None else h0
        for epi, ws, extra in epis:
            want = kernels.gemv(inp, ws, epilogue=epi, **extra)
            h1, got = kernels.gemv_chain(r, ws, eps=eps, epilogue=epi, **ch, **extra)
            assert torch.equal(h1, h0), f"chain {ci} epilogue {epi}: h differs"
            for g_, w_ in zip(got if isinstance(got, tuple) else (got,), want if isinstance(want, tuple) else (want,)):
                assert torch.equal(g_, w_), f"chain {ci} epilogue {epi}: output differs"
    _, got = kernels.gemv_chain(r, mats[:1], eps=eps, want_h=False, w_b=wn[2])
    _, z0 = kernels.norm_chain(r, eps=eps, w_b=wn[2], want_h=False)
    assert torch.equal(got, kernels.gemv(z0, mats[:1]))


def test_chained_step_equals_unchained_step():
    """The engine's decode step with the chains inside the GEMVs equals the step with
    separate chain launches bit for bit."""
    tiny = OuroConfig(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=2)
    model = OuroForCausalLM.random_init(tiny, seed=22, device=DEV)
    g = torch.Generator().manual_seed(22)
    ids = torch.randint(0, tiny.vocab_size, (1, 150), generator=g).to(DEV)
    a_eng = FlashLoopEngine(model, use_graphs=False)
    b_eng = FlashLoopEngine(model, use_graphs=False)
    b_eng.fused_chain = False
    a_eng.prefill(ids[:, :130], decode_capacity=64)
    b_eng.prefill(ids[:, :130], decode_capacity=64)
    for i in range(130, 150):
        a = a_eng.decode(ids[:, i:i + 1]).logits
        b = b_eng.decode(ids[:, i:i + 1]).logits
        assert torch.equal(a, b), f"step {i}: max diff {(a - b).abs().max().item()}"
