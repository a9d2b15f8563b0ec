"""End-to-end FlashLoopEngine on the HIP kernels (tiny random-init Ouro-shaped model)."""

import math

import numpy as np
import pytest
import torch

from oracle.tokens import select_active_mask

pytestmark = pytest.mark.gpu

from flashloop_amd import kernels  # noqa: E402
from flashloop_amd.config import FlashLoopConfig  # noqa: E402
from flashloop_amd.engine import FlashLoopEngine  # noqa: E402
from flashloop_amd.hooks import flashloop  # noqa: E402
from flashloop_amd.model import OuroConfig, OuroForCausalLM  # noqa: E402

TINY = OuroConfig(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                  num_attention_heads=2, num_key_value_heads=2)


def _ids(t, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, TINY.vocab_size, (1, t), generator=g).cuda()


def _cos(a, b):
    return float(torch.nn.functional.cosine_similarity(a.flatten().double(), b.flatten().double(), dim=0))


def test_prefill_all_rows_matches_dense_forward():
    """With both prefill fractions 1.0 the token-sparse loops recompute every row, so the
    prefill logits are the dense looped model's (gather/scatter + masked SDPA path)."""
    model = OuroForCausalLM.random_init(TINY, seed=2, device="cuda")
    eng = FlashLoopEngine(model, config=FlashLoopConfig(prefill_fraction_loop3=1.0, prefill_fraction_loop4=1.0))
    ids = _ids(150)
    out = eng.prefill(ids)
    ref = model.dense_forward(ids)
    assert torch.isfinite(out.logits).all()
    assert (out.logits - ref).abs().max().item() < 5e-2 * max(1.0, ref.abs().max().item())
    assert [r.active_rows for r in out.state.prefill_receipts] == [150, 150, 150, 150]


def test_prefill_masks_match_oracle():
    model = OuroForCausalLM.random_init(TINY, seed=4, device="cuda")
    eng = FlashLoopEngine(model)
    ids = _ids(200, seed=4)
    seen = {}
    orig = eng._select

    def spy(cur, prev, fraction, eligible=None):
        mask, pos, score = orig(cur, prev, fraction, eligible)
        seen.setdefault("calls", []).append((score.float().cpu().numpy(), fraction,
                                             None if eligible is None else eligible.cpu().numpy(),
                                             mask.cpu().numpy(), pos.cpu().numpy()))
        return mask, pos, score

    eng._select = spy
    st = eng.prefill(ids).state
    assert len(seen["calls"]) == 2
    for score, frac, el, mask, pos in seen["calls"]:
        want = select_active_mask(score, frac, eligible=el)
        np.testing.assert_array_equal(mask, want)
        np.testing.assert_array_equal(pos, np.nonzero(want[0])[0])
    assert [r.active_rows for r in st.prefill_receipts] == [200, 200, 50, 20]
    assert bool(torch.all(~st.mask_loop4 | st.mask_loop3))
    assert bool(st.mask_loop3[0, -1]) and bool(st.mask_loop4[0, -1])


def test_decode_tracks_dense_model():
    """Decode logits through the packed int4 cache stay close to the dense looped model
    on the same tokens (cosine), with all keys selected so only the codec differs."""
    model = OuroForCausalLM.random_init(TINY, seed=5, device="cuda")
    eng = FlashLoopEngine(model, config=FlashLoopConfig(prefill_fraction_loop3=1.0, prefill_fraction_loop4=1.0,
                                                        decode_key_fraction=1.0))
    ids = _ids(130, seed=5)
    eng.prefill(ids[:, :128], decode_capacity=64)
    for i in range(128, 130):
        d = eng.decode(ids[:, i:i + 1])
        ref = model.dense_forward(ids[:, :i + 1])
        assert torch.isfinite(d.logits).all()
        assert _cos(d.logits, ref) > 0.98
    assert d.receipt.sparse_attention_calls == 2 * TINY.num_hidden_layers
    assert d.state.next_position == 130


def test_generate_crosses_rollover_and_hooks():
    model = OuroForCausalLM.random_init(TINY, seed=6, device="cuda")
    eng = FlashLoopEngine(model)
    ids = _ids(190, seed=6)
    out = eng.generate(ids, max_new_tokens=70)  # tail 62 -> rolls over one 64-token group
    assert out.shape == (1, 260) and torch.equal(out[:, :190], ids)
    lay = eng.state.cache.layers[0]
    assert lay.quantized_tokens == 192
    eng.reset()
    with pytest.raises(RuntimeError):
        _ = eng.state
    with flashloop(model) as hooks:
        out2 = model.generate(ids, max_new_tokens=70)
        audit = hooks["kv"].audit()
        joint = hooks["attention_and_prefill"].audit()
    assert torch.equal(out, out2)
    assert audit["status"] == "PASS" and audit["quantized_tokens"] == 192
    assert audit["quantized_groups"] == TINY.num_hidden_layers * 192 // 64
    assert audit["packed_stream_bytes"] + audit["residual_bf16_bytes"] + audit["mask_bytes"] == audit["total_packed_bytes"]
    assert joint["token_sparse_prefill"]["mask_nested"]
    assert joint["attention"]["target_replacements"] == 2 * TINY.num_hidden_layers * 69
    assert model.generate.__func__ is OuroForCausalLM.generate


def test_graph_decode_matches_eager():
    """Decode steps replayed from a captured HIP graph equal the eager launches bit for bit,
    across a rollover (packed eagerly between two replays of the same graph) and a change
    of the selection capacity (which recaptures)."""
    model = OuroForCausalLM.random_init(TINY, seed=7, device="cuda")
    ids = _ids(700, seed=7)
    eager = FlashLoopEngine(model, use_graphs=False)
    graphed = FlashLoopEngine(model, use_graphs=True)
    a = eager.prefill(ids[:, :600], decode_capacity=160).logits
    b = graphed.prefill(ids[:, :600], decode_capacity=160).logits
    assert torch.equal(a, b)
    captures = 0
    for i in range(600, 700):
        tok = ids[:, i:i + 1]
        da = eager.decode(tok)
        before = graphed._runner.graph
        db = graphed.decode(tok)
        captures += graphed._runner.graph is not before
        assert torch.equal(da.logits, db.logits), f"step {i}"
        assert da.receipt == db.receipt
    # the first capture and one at the selection-capacity step (k reaches 64 at 631 keys);
    # the rollover at step 40 replays the same graph over the repacked cache
    assert captures == 2
    la, lb = eager.state.cache.layers[0], graphed.state.cache.layers[0]
    assert la.packed_host == lb.packed_host and la.tail_host == lb.tail_host
    for s in range(4):
        assert torch.equal(la.codes[s], lb.codes[s])
        assert torch.equal(la.tail_key[s], lb.tail_key[s])


def test_saved_cache_decodes_identically(tmp_path):
    """A prefilled cache written to disk and read back decodes to the same logits."""
    from flashloop_amd.cache import CrossLoopKVCache

    model = OuroForCausalLM.random_init(TINY, seed=8, device="cuda")
    ids = _ids(300, seed=8)
    a = FlashLoopEngine(model, use_graphs=False)
    b = FlashLoopEngine(model, use_graphs=False)
    a.prefill(ids[:, :290], decode_capacity=32)
    b.prefill(ids[:, :290], decode_capacity=32)
    path = str(tmp_path / "kv.safetensors")
    a.state.cache.save(path)
    loaded = CrossLoopKVCache.load(path, device="cuda")
    st = b.state
    b._state = type(st)(loaded, st.next_position, st.mask_loop3, st.mask_loop4, st.prefill_receipts)
    for i in range(290, 300):
        da = a.decode(ids[:, i:i + 1])
        db = b.decode(ids[:, i:i + 1])
        assert torch.equal(da.logits, db.logits), f"step {i}"


def test_sparse_decode_disabled_runs_every_loop_dense():
    """enable_sparse_decode=False (flashloop/engine.py:422): loops 3-4 read the cache
    densely like loops 1-2; the step tracks the dense model, graphs equal eager."""
    model = OuroForCausalLM.random_init(TINY, seed=9, device="cuda")
    cfg = FlashLoopConfig(prefill_fraction_loop3=1.0, prefill_fraction_loop4=1.0, enable_sparse_decode=False)
    eager = FlashLoopEngine(model, config=cfg, use_graphs=False)
    graphed = FlashLoopEngine(model, config=cfg, use_graphs=True)
    ids = _ids(200, seed=9)
    eager.prefill(ids[:, :190], decode_capacity=32)
    graphed.prefill(ids[:, :190], decode_capacity=32)
    for i in range(190, 200):
        da = eager.decode(ids[:, i:i + 1])
        db = graphed.decode(ids[:, i:i + 1])
        assert torch.equal(da.logits, db.logits), f"step {i}"
        ref = model.dense_forward(ids[:, :i + 1])
        assert _cos(da.logits, ref) > 0.98
    nl = TINY.num_hidden_layers
    assert da.receipt.dense_attention_calls == 4 * nl and da.receipt.sparse_attention_calls == 0
    assert da.receipt.dense_late_loop_calls == 2 * nl and da.receipt.selected_keys_per_layer == ()


def test_graph_recapture_releases_old_graphs():
    """Each recapture destroys the superseded graph and its pool before capturing (no
    garbage-collector workaround): many recaptures with collections in between."""
    import gc

    model = OuroForCausalLM.random_init(TINY, seed=10, device="cuda")
    eng = FlashLoopEngine(model, config=FlashLoopConfig(decode_key_fraction=1.0), use_graphs=True)
    ids = _ids(400, seed=10)
    eng.prefill(ids[:, :200], decode_capacity=256)
    held = []
    first = None
    for i in range(200, 330):  # fraction 1: the selection capacity steps every 64 keys
        out = eng.decode(ids[:, i:i + 1])
        held.append(out)  # outputs held across recaptures stay valid tensors
        first = eng._runner.captures if first is None else first
        gc.collect()
    assert eng._runner.captures - first >= 2
    assert all(torch.isfinite(o.logits).all() for o in held[-3:])


def test_cfg4_full_model_prefill_and_decode():
    """BASELINE config 4 at its shape: the random-init 24-layer looped decoder (hidden
    2048, 16 heads x 128, SwiGLU 5632, vocab 49152), an 8192-token prompt, then 256 greedy
    decode steps (four rollovers of the BF16 tail, at steps 63, 127, 191 and 255).
    Checks the prefill receipts, the loop-2 key budget ceil((T+1)*0.1) actually selected
    by the top-k kernel at every step, finite logits, graph replay equal to eager
    launches bit for bit, the first 70 steps' logits against the torch-module decode step
    (fused_decode=False) by cosine, and -- sharing no reader with the engine -- layer 0's
    attention at the steps after the first three rollovers and at the last step, against
    the oracle run on layer 0's own K/V history (prefill K/V and masks, then every
    decoded token), with the packed streams of layer 0 bit-exact after the last rollover."""
    from gpu_util import assert_layer_matches_chain, np32, step_vs_oracle_rows

    print("case: cfg4 24L/2048/5632/49152, prompt 8192, 256 steps", flush=True)
    cfg = OuroConfig()
    assert (cfg.num_hidden_layers, cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size) == (24, 2048, 5632, 49152)
    model = OuroForCausalLM.random_init(cfg, seed=4, device="cuda")
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, cfg.vocab_size, (1, 8192), generator=g).cuda()
    graphed = FlashLoopEngine(model, use_graphs=True)
    eager = FlashLoopEngine(model, use_graphs=False)
    modules = FlashLoopEngine(model, use_graphs=False)
    modules.fused_decode = False
    heads = [0, 9]  # layer-0 heads held against the oracle
    # layer 0's prefill K/V and masks, as the eager engine packs them
    pre = {}
    from flashloop_amd import cache as cache_mod

    orig_fp = cache_mod.CrossLoopKVLayer.from_prefill.__func__

    def capture_prefill(cls, keys, values, **kw):
        if not pre:
            pre["k"] = [np32(k[:, heads]) for k in keys]
            pre["v"] = [np32(v[:, heads]) for v in values]
            pre["m"] = (kw["mask_loop3"].cpu().numpy().astype(bool), kw["mask_loop4"].cpu().numpy().astype(bool))
        return orig_fp(cls, keys, values, **kw)

    outs = [graphed.prefill(ids, decode_capacity=320)]
    cache_mod.CrossLoopKVLayer.from_prefill = classmethod(capture_prefill)
    try:
        outs.append(eager.prefill(ids, decode_capacity=320))
    finally:
        cache_mod.CrossLoopKVLayer.from_prefill = classmethod(orig_fp)
    outs.append(modules.prefill(ids, decode_capacity=320))
    for o in outs:
        assert [(r.loop, r.total_rows, r.active_rows) for r in o.state.prefill_receipts] == \
            [(1, 8192, 8192), (2, 8192, 8192), (3, 8192, 2048), (4, 8192, 820)]
        assert torch.isfinite(o.logits).all()
    assert torch.equal(outs[0].logits, outs[1].logits)
    assert pre["k"][0].shape == (1, 2, 8192, 128)
    lc = eager.state.cache.layers[0]
    assert lc.quantized_tokens == 8128
    seen = []
    rec = {}  # this step's layer-0 attention inputs and outputs, per loop

    def keep(loop, kw):
        rec[loop] = {n: kw[n].detach().clone() for n in ("query", "current_key", "current_value")}

    orig_dense, orig_sel = lc.dense_source_attention, lc.dense_source_attention_select
    orig_src, orig_delta = lc.cached_mass_sparse_attention_delta_with_source, lc.cached_mass_sparse_attention_delta
    check_sel = lc.select_decode_keys

    def spy_dense(loop, **kw):
        res = orig_dense(loop, **kw)
        keep(loop, kw)
        rec[loop]["out"] = res[0].clone()
        return res

    def spy_sel(loop, **kw):
        res = orig_sel(loop, **kw)
        check_sel(res[1], kw["fraction"], validate=True)  # NaN/inf logits would raise here
        seen.append(res[2][4])
        keep(loop, kw)
        rec[loop].update(out=res[0].clone(), logits=res[1].clone(), indices=res[2][0].clone())
        return res

    def spy_src(loop, **kw):
        res = orig_src(loop, **kw)
        keep(loop, kw)
        rec[loop]["out"] = res[0].clone()
        return res

    def spy_delta(loop, **kw):
        res = orig_delta(loop, **kw)
        keep(loop, kw)
        rec[loop]["out"] = res.clone()
        return res

    lc.dense_source_attention, lc.dense_source_attention_select = spy_dense, spy_sel
    lc.cached_mass_sparse_attention_delta_with_source, lc.cached_mass_sparse_attention_delta = spy_src, spy_delta
    hist_k = [[] for _ in range(4)]  # layer-0 K/V of every decoded token, per loop
    hist_v = [[] for _ in range(4)]
    tok = torch.argmax(outs[0].logits, dim=-1, keepdim=True)
    worst = 1.0
    rolled = []
    checked = []
    steps = 256
    for step in range(steps):
        pos = 8192 + step
        a = graphed.decode(tok)
        before = lc.quantized_tokens
        b = eager.decode(tok)
        if step < 70:
            c = modules.decode(tok)
            worst = min(worst, _cos(b.logits, c.logits))
            assert _cos(b.logits, c.logits) > 0.999, f"step {step}: fused vs torch-module step"
        elif step == 70:
            modules.reset()
        assert torch.isfinite(a.logits).all()
        assert torch.equal(a.logits, b.logits), f"step {step}: graph replay differs from eager"
        want_k = math.ceil((pos + 1) * 0.1)  # T = pos keys before the current token
        assert a.receipt.selected_keys_per_layer == (want_k,) * 24
        assert seen[-1].cpu().tolist() == [want_k] * 16, f"step {step}: observed top-k budget"
        if step in (64, 128, 192, steps - 1):
            torch.cuda.synchronize()
            T = pos
            nk = [np.concatenate([pre["k"][r]] + [x[None, :, None] for x in hist_k[r]], axis=2) for r in range(4)]
            nv = [np.concatenate([pre["v"][r]] + [x[None, :, None] for x in hist_v[r]], axis=2) for r in range(4)]
            assert nk[0].shape[2] == T
            ones = np.ones((1, step), bool)
            masks = (np.concatenate([pre["m"][0], ones], 1), np.concatenate([pre["m"][1], ones], 1))
            sub = lambda t: np32(t).reshape(16, 128)[heads]  # noqa: E731
            got = dict(out0=rec[0]["out"], out1=rec[1]["out"], logits1=rec[1]["logits"], indices=rec[1]["indices"],
                       delta2=rec[2]["out"], delta3=rec[3]["out"])
            step_vs_oracle_rows(got, heads, 16, nk, nv, masks, [sub(rec[r]["query"]) for r in range(4)],
                                [sub(rec[r]["current_key"]) for r in range(4)],
                                [sub(rec[r]["current_value"]) for r in range(4)], model.model.layers[0].self_attn.scaling,
                                0.10, what=f"cfg4 layer 0 step {step}")
            checked.append(step)
        for r in range(4):
            hist_k[r].append(np32(rec[r]["current_key"]).reshape(16, 128)[heads])
            hist_v[r].append(np32(rec[r]["current_value"]).reshape(16, 128)[heads])
        if lc.quantized_tokens != before:
            rolled.append(step)
        tok = torch.argmax(a.logits, dim=-1, keepdim=True)
    print(f"[parity] cfg4 worst cosine fused vs modules {worst:.6f} (70 steps)", flush=True)
    assert rolled == [63, 127, 191, 255] and checked == [64, 128, 192, 255]
    assert lc.quantized_tokens == 8384  # four 64-token groups rolled out of the tail
    # layer 0's packed streams (heads 0 and 9) after the fourth rollover, against the oracle
    # encoding of its whole K/V history
    from oracle import codec

    nk = [np.concatenate([pre["k"][r]] + [x[None, :, None] for x in hist_k[r]], axis=2) for r in range(4)]
    nv = [np.concatenate([pre["v"][r]] + [x[None, :, None] for x in hist_v[r]], axis=2) for r in range(4)]
    ones = np.ones((1, steps), bool)
    masks = (np.concatenate([pre["m"][0], ones], 1), np.concatenate([pre["m"][1], ones], 1))
    chain, tp = codec.compress_prefix(nk, nv, masks)  # 8448 tokens: 8384 packed, 64 in the tail
    assert tp == lc.quantized_tokens
    assert_layer_matches_chain(lc, chain, tp, 1, len(heads), row_ids=heads)


def test_hooks_route_forward_and_generate_with_observed_counters(tmp_path):
    """Inside flashloop(model) a plain forward prefills (all positions), a forward with the
    returned cache decodes, and generate runs the engine; the counters are what ran, and
    the kv audit's byte fields equal the reference's formulas (oracle restatement) over
    the rows the packed cache actually holds."""
    from oracle import accounting as OACC

    from test_model_cpu import _hf_dir

    src = OuroForCausalLM.random_init(TINY, seed=11, device="cuda")
    _hf_dir(tmp_path, src.cpu())
    eng_ref = FlashLoopEngine.from_pretrained(str(tmp_path), device="cuda")  # HF-style sharded directory
    model = eng_ref.model
    ids = _ids(200, seed=11)
    steps = 5
    ref_pre = eng_ref.prefill(ids, decode_capacity=64)
    tok = torch.argmax(ref_pre.logits, dim=-1, keepdim=True)
    ref_steps = []
    for _ in range(steps):
        d = eng_ref.decode(tok)
        ref_steps.append(d.logits.clone())
        tok = torch.argmax(d.logits, dim=-1, keepdim=True)
    with flashloop(model) as hooks:
        out = model(ids)
        assert out.logits.shape == (1, 200, TINY.vocab_size)
        # the last position of an all-positions lm_head (another GEMM shape: bf16 rounding)
        assert (out.logits[:, -1] - ref_pre.logits).abs().max().item() < 2e-2
        assert torch.equal(torch.argmax(out.logits[:, -1], -1), torch.argmax(ref_pre.logits, -1))
        cache = out.past_key_values
        tok = torch.argmax(out.logits[:, -1], dim=-1, keepdim=True)
        kept = []
        for i in range(steps):
            o = model(tok, past_key_values=cache)
            assert torch.equal(o.logits[:, 0], ref_steps[i]), f"routed decode step {i}"
            kept.append(o.logits)  # held as an HF caller holds them (graph replays follow)
            cache = o.past_key_values
            tok = torch.argmax(o.logits[:, 0], dim=-1, keepdim=True)
        # every kept step still holds its own logits after the later replays
        for i, lg in enumerate(kept):
            assert torch.equal(lg[:, 0], ref_steps[i]), f"kept logits of step {i} were overwritten"
        assert not torch.equal(kept[0], kept[-1])
        with pytest.raises(ValueError):
            model(tok, past_key_values=out.past_key_values)  # stale
        kv = hooks["kv"].audit()
        joint = hooks["attention_and_prefill"].audit()
        assert kv["forward_calls"] == 1 + steps and kv["cache_updates"] == 1 + steps
        nl = TINY.num_hidden_layers
        assert joint["attention"] == {"prefill_attention_calls": 4 * nl, "source_captures": steps * nl,
                                      "target_replacements": 2 * steps * nl}
        assert joint["token_sparse_prefill"] == {"active_counts": {"3": 50, "4": 20}, "mask_nested": True}
        st = hooks["kv"].engine.state
        m3 = st.mask_loop3.cpu().numpy()[0]
        m4 = st.mask_loop4.cpu().numpy()[0]
        tp = kv["quantized_tokens"]
        groups = []
        for _ in range(nl):
            for g in range(tp // 64):
                groups.append(OACC.temporal_group_bytes((1, TINY.num_attention_heads, 64, 128),
                                                        [64, int(m3[g * 64:(g + 1) * 64].sum()),
                                                         int(m4[g * 64:(g + 1) * 64].sum())])["packed_bytes"])
        want = OACC.compressor_audit(num_layers=nl, recurrent_steps=4, batch=1, heads=TINY.num_attention_heads,
                                     channels=128, total_tokens=200 + steps, current_tokens=200 + steps,
                                     next_start=[tp] * nl, packed_stream_bytes=sum(groups),
                                     quantized_groups=len(groups), mask_numel=200)
        for key, value in want.items():
            assert kv[key] == value, key
        lay = st.cache.layers[0]
        want_store = nl * OACC.kivi_layer_storage_bytes(
            batch=1, heads=TINY.num_attention_heads, channels=128, packed_tokens=tp, tail_tokens=200 + steps - tp,
            rows3=int(m3[:tp].sum()), rows4=int(m4[:tp].sum()))
        assert kv["reference_layout_storage_bytes"] == want_store
        assert kv["physical_storage_bytes"] == st.cache.storage_bytes
        gen = model.generate(ids, max_new_tokens=3)
        assert gen.shape == (1, 203)
        assert hooks["kv"].audit()["forward_calls"] == 1 + steps + 3
    assert lay.late_rows_host[0][0] == int(m3[:tp].sum())
