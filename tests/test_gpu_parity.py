"""GPU parity of the HIP path (through the C ABI) against the CPU oracle.

Bars: codes, scales/zeros and selected indices bit-exact;
attention outputs within 2e-2 max-abs and 1e-3 mean-abs.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import codec
from oracle import tokens as OT

from flashloop_amd import CrossLoopKVLayer, decode_attention_step, kernels
from flashloop_amd.synthetic import SCALING, decode_workload, ragged_lengths

from gpu_util import (
    assert_close,
    assert_layer_matches_chain,
    flat_rows,
    materialized,
    np32,
    oracle_prefix,
    restated_dense_logits,
    restated_selected_aggregate,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _masks(batch, tokens, seed, p3=0.3, p4=0.5):
    rng = np.random.default_rng(seed)
    m3 = rng.random((batch, tokens)) < p3
    m4 = m3 & (rng.random((batch, tokens)) < p4)
    m3[:, -1] = m4[:, -1] = True
    return m3, m4


def _build(w, m3=None, m4=None, recon=False, token_capacity=None):
    ks = [w.cache(r)[0].to(DEV) for r in range(4)]
    vs = [w.cache(r)[1].to(DEV) for r in range(4)]
    kw = {}
    if m3 is not None:
        kw = dict(mask_loop3=torch.from_numpy(m3).to(DEV), mask_loop4=torch.from_numpy(m4).to(DEV))
    layer = CrossLoopKVLayer.from_prefill(ks, vs, lengths=w.lengths, recon=recon, token_capacity=token_capacity, **kw)
    torch.cuda.synchronize()
    return layer


@pytest.mark.parametrize("masked", [False, True])
def test_pack_bit_exact(masked):
    print("case: pack B2 H3 T390 masked=%s" % masked, flush=True)
    w = decode_workload(2, 3, 390, seed=11)
    m3 = m4 = None
    if masked:
        m3, m4 = _masks(2, 390, 5)
    layer = _build(w, m3, m4, recon=True)
    nk, nv, chain, tp = oracle_prefix([w.cache(r)[0] for r in range(4)], [w.cache(r)[1] for r in range(4)], m3, m4)
    assert tp == layer.quantized_tokens == 320
    assert_layer_matches_chain(layer, chain, tp, 2, 3)
    for r in range(4):
        got_k = np32(layer.recon_keys[r]).reshape(2, 3, 390, 128)[:, :, :tp]
        got_v = np32(layer.recon_values[r]).reshape(2, 3, 390, 128)[:, :, :tp]
        assert np.array_equal(got_k, chain.recon_keys[r]), f"R_{r} keys differ"
        assert np.array_equal(got_v, chain.recon_values[r]), f"R_{r} values differ"


@pytest.mark.parametrize("loops", [1, 2, 3])
def test_pack_fewer_loops_match_the_four_loop_encode(loops):
    """The C-ABI's 1..3-loop packs (one kernel per loop count) write exactly the first
    streams of the 4-loop encode and leave the others untouched."""
    print("case: pack B2 H3 T390 masked loops=%d" % loops, flush=True)
    b, h, t = 2, 3, 390
    w = decode_workload(b, h, t, seed=13)
    m3, m4 = _masks(b, t, 7)
    full = _build(w, m3, m4)
    tp = full.quantized_tokens
    part = CrossLoopKVLayer(full.geometry, DEV)
    for s in range(2):
        part.rank[s].copy_(full.rank[s])
    ks = [w.cache(r)[0].to(DEV).reshape(b * h, t, 128).contiguous() for r in range(loops)]
    vs = [w.cache(r)[1].to(DEV).reshape(b * h, t, 128).contiguous() for r in range(loops)]
    mk = [torch.from_numpy(m).to(DEV).to(torch.uint8).contiguous() for m in (m3, m4)]
    kernels.pack_kv_groups(part.view(), loops, ks, vs, src_bh_stride=t, src_row_offset=0,
                           dst_group0=torch.zeros(b, dtype=torch.int32, device=DEV), n_groups=tp // 64,
                           masks=mk, mask_stride=t)
    torch.cuda.synchronize()
    for s in range(4):
        same = s < loops
        for name in ("codes", "key_meta", "value_meta", "key_meta_half", "value_meta_half"):
            got, ref = getattr(part, name)[s], getattr(full, name)[s]
            if same:
                assert torch.equal(got, ref), f"stream {s} {name} differs"
            else:
                assert not torch.any(got != 0), f"stream {s} {name} written by a {loops}-loop pack"
        rec_got, rec_ref = part.value_meta_token[..., s, :], full.value_meta_token[..., s, :]
        assert torch.equal(rec_got, rec_ref) if same else not torch.any(rec_got != 0)


def test_pack_closed_forms():
    """Constant and ramp groups through the GPU codec (known answers)."""
    print("case: pack closed forms", flush=True)
    t = 128
    k = torch.full((1, 1, t + 64, 128), 0.75, dtype=torch.bfloat16)
    ramp = (-1.0 + 0.125 * (torch.arange(t + 64) % 16)).to(torch.bfloat16)
    v = ramp[None, None, :, None].expand(1, 1, t + 64, 128).contiguous()
    layer = CrossLoopKVLayer.from_prefill([k.to(DEV)] * 4, [v.to(DEV)] * 4)
    kc = layer.key_codes[0].cpu().numpy()[0, :t]
    km = layer.key_meta[0].cpu().numpy()[0, : t // 64]
    assert np.all(kc == 0) and np.all(km[..., 0] == 1.0) and np.all(km[..., 1] == 0.75)
    # loops 2-4 reproduce loop 1 exactly: zero residual codes with scale 1
    for s in (1, 2, 3):
        assert np.all(layer.key_codes[s].cpu().numpy()[0, :t] == 0)
        assert np.all(layer.key_meta[s].cpu().numpy()[0, : t // 64, :, 0] == 1.0)


def _oracle_rows(w, m3=None, m4=None):
    """Per-(b,h) K_r/V_r rows ``[T_b, 128]`` for every loop, each sequence encoded on its own."""
    K = [[] for _ in range(4)]
    V = [[] for _ in range(4)]
    h = w.keys[0].shape[1]
    for b, t in enumerate(w.lengths):
        ks = [w.keys[r][b : b + 1, :, :t] for r in range(4)]
        vs = [w.values[r][b : b + 1, :, :t] for r in range(4)]
        mm3 = None if m3 is None else m3[b : b + 1, :t]
        mm4 = None if m4 is None else m4[b : b + 1, :t]
        nk, nv, chain, tp = oracle_prefix(ks, vs, mm3, mm4)
        Kb, Vb = materialized(nk, nv, chain, tp)
        for r in range(4):
            for j in range(h):
                K[r].append(Kb[r][0, j])
                V[r].append(Vb[r][0, j])
    return K, V


@pytest.mark.parametrize("masked", [False, True])
def test_dense_reader_all_loops(masked):
    print("case: dense reader B2 H3 T390 masked=%s" % masked, flush=True)
    w = decode_workload(2, 3, 390, seed=12)
    m3 = m4 = None
    if masked:
        m3, m4 = _masks(2, 390, 6)
    layer = _build(w, m3, m4)
    K, V = _oracle_rows(w, m3, m4)
    for loop in range(4):
        kc, vc = w.current(loop)
        out, logits = layer.dense_source_attention(
            loop, query=w.queries[loop].to(DEV), current_key=kc.to(DEV), current_value=vc.to(DEV),
            scaling=SCALING, return_logits=True)
        torch.cuda.synchronize()
        q = np32(w.queries[loop]).reshape(6, 128)
        want, want_lg = OA.dense_decode(q, K[loop], V[loop], np32(kc).reshape(6, 128),
                                        np32(vc).reshape(6, 128), SCALING)
        assert_close(np32(out).reshape(6, 128), want, what=f"loop {loop} output")
        got_lg = np32(logits).reshape(6, -1)
        assert got_lg.shape[1] >= want_lg.shape[1] and got_lg.shape[1] % 64 == 0  # padded, aligned row stride
        # two bars: the kernel's contraction against an fp64 restatement of its own
        # arithmetic (tight), and against the oracle's bf16 chain, whose per-stream
        # re-rounding the reader skips (~2e-3 on logits)
        rest = restated_dense_logits(layer, loop, range(6), q, np32(kc).reshape(6, 128), SCALING)
        assert_close(got_lg[:, : want_lg.shape[1]], np.stack(rest), max_abs=1e-4, mean_abs=1e-5,
                     what=f"loop {loop} logits vs restated reader arithmetic")
        assert_close(got_lg[:, : want_lg.shape[1]], want_lg, max_abs=2e-2, mean_abs=5e-3, what=f"loop {loop} logits")


def test_dense_logits_stay_within_their_stride():
    """A view whose host maxima undercount the device lengths (here: no tail counted) is
    accepted with a stride sized to those maxima; the reader still computes every key
    from the device lengths but writes no logit past a row's stride, so each row holds
    the first `stride` logits of a correctly sized read and nothing beyond is touched."""
    import ctypes as C

    from flashloop_amd import _lib

    print("case: dense logits stride guard B2 H3 T390", flush=True)
    w = decode_workload(2, 3, 390, seed=14)
    layer = _build(w)
    lib = _lib.load()
    kc, vc = w.current(1)
    q, k, v = (x.to(DEV).reshape(6, 128).contiguous() for x in (w.queries[1], kc, vc))
    view = layer.view()
    assert view.max_tail_tokens > 0
    stale = _lib.FlCacheView.from_buffer_copy(view)
    stale.max_tail_tokens = 0
    full_s = view.max_packed_tokens + view.max_tail_tokens + 1
    s = stale.max_packed_tokens + 1
    ref = torch.empty(6, full_s, dtype=torch.float32, device=DEV)
    buf = torch.full((6 * s + 256,), 7.0, dtype=torch.float32, device=DEV)
    out = torch.empty(6, 128, dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    for vw, lg, stride in ((view, ref, full_s), (stale, buf, s)):
        nbytes = lib.fl_decode_attn_dense_workspace(C.byref(vw))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        rc = lib.fl_decode_attn_dense(C.byref(vw), 1, q.data_ptr(), k.data_ptr(), v.data_ptr(), SCALING,
                                      out.data_ptr(), lg.data_ptr(), stride, ws.data_ptr(), nbytes, stream)
        assert rc == _lib.FL_OK, lib.fl_last_error()
    torch.cuda.synchronize()
    assert torch.equal(buf[: 6 * s].view(6, s), ref[:, :s])
    assert bool((buf[6 * s :] == 7.0).all())


def test_topk_bit_exact_with_ties():
    print("case: topk ties", flush=True)
    rng = np.random.default_rng(3)
    rows, n = 5, 3000
    lg = rng.integers(-40, 40, size=(rows, n)).astype(np.float32) / 8.0  # many exact ties
    lg[4] = 0.0  # all equal
    for frac in (0.1, 0.37, 1.0):
        sel = OA.decode_topk(lg, frac)
        cap = sel.indices.shape[1]
        t = torch.from_numpy(lg).to(DEV)
        nk = torch.full((rows,), n, dtype=torch.int32, device=DEV)
        idx, valid, mass, wts, counts = kernels.decode_topk(t, nk, frac, cap)
        torch.cuda.synchronize()
        assert np.array_equal(idx.cpu().numpy(), sel.indices), f"indices differ at fraction {frac}"
        assert np.array_equal(valid.cpu().numpy().astype(bool), sel.valid)
        assert np.array_equal(counts.cpu().numpy(), sel.count)
        assert np.allclose(mass.cpu().numpy(), sel.mass, rtol=2e-6, atol=1e-7)
        assert np.allclose(wts.cpu().numpy(), sel.selected_weights, rtol=2e-5, atol=1e-8)


@pytest.mark.parametrize("n", [32769, 40000])
def test_topk_ranks_fp32_softmax_weights(n):
    """Peaked rows (logits ~ N(0, 64^2): most weights underflow, so many distinct logits
    share one fp32 weight) and cfg3-shaped ordinary rows: indices bit-exact with the
    oracle's weight-image ranking, and equal to ranking torch's own fp32 softmax on this
    GPU with ties to the lower index.  n=40000 takes the global-memory kernel."""
    print("case: topk weight ranking n=%d" % n, flush=True)
    rng = np.random.default_rng(21)
    rows = 24
    lg = (rng.standard_normal((rows, n)) * np.repeat([1.0, 16.0, 64.0], rows // 3)[:, None]).astype(np.float32)
    lg[-1, :] = -300.0  # one row: a single finite winner among underflowing keys
    lg[-1, n // 2] = 0.0
    frac = 0.1
    cap = OA.padded_capacity(OA.decode_budget(n, frac))
    t = torch.from_numpy(lg).to(DEV)
    nk = torch.full((rows,), n, dtype=torch.int32, device=DEV)
    idx, valid, mass, wts, counts = kernels.decode_topk(t, nk, frac, cap)
    torch.cuda.synchronize()
    sel = OA.decode_topk(lg, frac, kpad=cap)
    got = idx.cpu().numpy()
    assert np.array_equal(got, sel.indices)
    assert np.allclose(mass.cpu().numpy(), sel.mass, rtol=2e-6)
    assert np.allclose(wts.cpu().numpy(), sel.selected_weights, rtol=2e-5, atol=1e-30)
    k = int(sel.count[0])
    # torch's fp32 softmax on the CPU keeps subnormal weights (IEEE); this GPU's torch
    # softmax flushes them to zero, so it ties more keys: reported, not asserted
    w_t = torch.softmax(t.cpu(), dim=-1, dtype=torch.float32).numpy()
    w_g = torch.softmax(t, dim=-1, dtype=torch.float32).cpu().numpy()
    d_torch = sum(not np.array_equal(got[r, :k], OA.topk_order(w_t[r], k)) for r in range(rows))
    d_gpu = sum(not np.array_equal(got[r, :k], OA.topk_order(w_g[r], k)) for r in range(rows))
    d_logit = sum(not np.array_equal(got[r, :k], OA.topk_order(lg[r], k)) for r in range(rows))
    print(f"[parity] topk n={n}: rows differing from torch-CPU fp32 softmax ranking {d_torch}, from "
          f"torch-GPU softmax ranking {d_gpu} (subnormals {int(((w_t > 0) & (w_t < 2**-126)).sum())} on CPU, "
          f"{int(((w_g > 0) & (w_g < 2**-126)).sum())} on GPU), from the logit ranking {d_logit} of {rows}",
          flush=True)
    assert d_torch == 0
    assert d_logit >= rows // 3 - 1  # the peaked rows (but the last): the logit order is not the reference's


@pytest.mark.parametrize("width", [5000, 4999])
def test_topk_ragged_rows_and_budget_edges(width):
    """Key counts that end mid-quad (one lane of the row's last 4-key quad reloads its keys)
    and, with width 4999, rows that start off the 16-byte alignment of a 4-key load."""
    print("case: topk ragged width=%d" % width, flush=True)
    rng = np.random.default_rng(4)
    n_keys = [1, 7, 64, 640, 641, 4097, width]
    rows = len(n_keys)
    lg = rng.standard_normal((rows, width)).astype(np.float32) * 3
    frac = 0.1
    cap = max(OA.padded_capacity(OA.decode_budget(n, frac)) for n in n_keys)
    t = torch.from_numpy(lg).to(DEV)
    idx, valid, mass, wts, counts = kernels.decode_topk(t, torch.tensor(n_keys, dtype=torch.int32, device=DEV), frac, cap)
    torch.cuda.synchronize()
    sel = OA.decode_topk([lg[r, :n] for r, n in enumerate(n_keys)], frac, kpad=cap)
    assert np.array_equal(idx.cpu().numpy(), sel.indices)
    assert np.array_equal(valid.cpu().numpy().astype(bool), sel.valid)
    assert np.allclose(mass.cpu().numpy(), sel.mass, rtol=2e-6)


def test_topk_long_rows_and_large_budgets():
    """Rows longer than the register-resident kernel holds (35840 keys) and budgets above
    its selected-list capacity (8192) take the global-memory kernel; same bits."""
    print("case: topk long rows", flush=True)
    rng = np.random.default_rng(6)
    n = 40000
    lg = (rng.standard_normal((3, n)) * 2.0).astype(np.float32)
    lg[1] = np.round(lg[1] * 4.0) / 4.0  # many exact ties
    n_keys = [n, 36001, 20000]
    for frac in (0.1, 0.3):
        cap = max(OA.padded_capacity(OA.decode_budget(k, frac)) for k in n_keys)
        t = torch.from_numpy(lg).to(DEV)
        idx, valid, mass, wts, counts = kernels.decode_topk(t, torch.tensor(n_keys, dtype=torch.int32, device=DEV),
                                                            frac, cap)
        torch.cuda.synchronize()
        sel = OA.decode_topk([lg[r, :k] for r, k in enumerate(n_keys)], frac, kpad=cap)
        assert np.array_equal(idx.cpu().numpy(), sel.indices), f"indices differ at fraction {frac}"
        assert np.array_equal(valid.cpu().numpy().astype(bool), sel.valid)
        assert np.array_equal(counts.cpu().numpy(), sel.count)
        assert np.allclose(mass.cpu().numpy(), sel.mass, rtol=2e-6)
        assert np.allclose(wts.cpu().numpy(), sel.selected_weights, rtol=2e-5, atol=1e-8)
    # a short row next to a long stride stays on its own key count
    t = torch.from_numpy(lg).to(DEV)
    short = torch.tensor([5, 64, 641], dtype=torch.int32, device=DEV)
    cap = OA.padded_capacity(OA.decode_budget(641, 0.1))
    idx, valid, mass, wts, counts = kernels.decode_topk(t, short, 0.1, cap)
    torch.cuda.synchronize()
    sel = OA.decode_topk([lg[r, :k] for r, k in enumerate([5, 64, 641])], 0.1, kpad=cap)
    assert np.array_equal(idx.cpu().numpy(), sel.indices)


def _step_vs_oracle(w, layer, m3=None, m4=None, frac=0.10):
    b, h = len(w.lengths), w.keys[0].shape[1]
    R = b * h
    Kr, Vr = _oracle_rows(w, m3, m4)
    qs = [w.queries[r].to(DEV) for r in range(4)]
    cur = [w.current(r) for r in range(4)]
    ks = [c[0].to(DEV) for c in cur]
    vs = [c[1].to(DEV) for c in cur]
    step = decode_attention_step(layer, qs, ks, vs, SCALING, frac)
    unfused = decode_attention_step(layer, qs, ks, vs, SCALING, frac, fused_source=False)
    torch.cuda.synchronize()
    # the fused loop-3 pass forms the same loop-2 aggregate as the separate selected-PV pass
    for a_, b_ in ((step.selected_output, unfused.selected_output), (step.delta2, unfused.delta2),
                   (step.delta3, unfused.delta3)):
        assert torch.allclose(a_, b_, atol=1e-5, rtol=1e-5)
    lengths = [x for x in w.lengths for _ in range(h)]
    q = [np32(w.queries[r]).reshape(R, 128) for r in range(4)]
    kc = [np32(c[0]).reshape(R, 128) for c in cur]
    vc = [np32(c[1]).reshape(R, 128) for c in cur]
    o0, _ = OA.dense_decode(q[0], Kr[0], Vr[0], kc[0], vc[0], SCALING)
    o1, lg1 = OA.dense_decode(q[1], Kr[1], Vr[1], kc[1], vc[1], SCALING)
    assert_close(np32(step.out0).reshape(R, 128), o0, what="loop-1 output")
    assert_close(np32(step.out1).reshape(R, 128), o1, what="loop-2 output")
    # selection: bit-exact on the kernel's own logits (identical inputs)
    g_lg = np32(step.logits1).reshape(R, -1)
    rows_lg = [g_lg[r, : lengths[r] + 1] for r in range(R)]
    cap = step.indices.shape[-1]
    sel = OA.decode_topk(rows_lg, frac, kpad=cap)
    assert np.array_equal(step.indices.cpu().numpy().reshape(R, cap), sel.indices), "selected indices differ"
    # end-to-end selection overlap against the oracle's own logits (reported, not bit-exact:
    # the kernel's logits differ from the bf16-chain oracle's by ~1e-3, which can swap keys
    # at a row's boundary).  One swap costs a row 1/k of its overlap, so the bound is per
    # row in swaps (at most 2, or 2% of k) and pooled over rows (> 99% once the rows
    # select 500 keys or more); measured pooled overlap >= 99.45% in every parity case.
    sel_o = OA.decode_topk(lg1, frac, kpad=cap)
    common = [len(set(sel.indices[r, : sel.count[r]]) & set(sel_o.indices[r, : sel_o.count[r]])) for r in range(R)]
    total = int(np.sum(sel_o.count[:R]))
    overlap = float(np.sum(common)) / total
    print(f"[parity] selection overlap with the oracle's own logits {overlap:.5f}", flush=True)
    for r in range(R):
        k = int(sel_o.count[r])
        assert k - common[r] <= max(2, math.ceil(0.02 * k)), f"row {r}: {k - common[r]} of {k} keys differ"
    if total >= 500:
        assert overlap > 0.99, f"selection overlap with oracle logits {overlap:.4f}"
    # selected aggregate and cached-mass deltas, oracle run on the kernel's selection
    so = OA.selected_value_aggregate(sel.indices, sel.valid, sel.selected_weights, Vr[1], vc[1], lengths)
    assert_close(np32(step.selected_output).reshape(R, 128), so, what="selected output")
    for loop, got in ((2, step.delta2), (3, step.delta3)):
        want = OA.sparse_delta(q[loop], Kr[loop], Vr[loop], kc[loop], vc[loop], lengths, sel.indices, sel.valid,
                               so, sel.mass, SCALING)
        assert_close(np32(got).reshape(R, 128), want, what=f"loop-{loop + 1} delta")
    return overlap


def test_decode_step_uniform():
    print("case: decode step B2 H4 T1200", flush=True)
    w = decode_workload(2, 4, 1200, seed=3)
    layer = _build(w)
    _step_vs_oracle(w, layer)


def test_decode_step_masked_late_loops():
    print("case: decode step masked B1 H4 T900", flush=True)
    w = decode_workload(1, 4, 900, seed=4)
    m3, m4 = _masks(1, 900, 8, p3=0.25, p4=0.4)
    layer = _build(w, m3, m4)
    _step_vs_oracle(w, layer, m3, m4)


def test_decode_step_late_loops_without_prefix_rows():
    """No prefix row is recomputed in loops 3/4 and the capacity leaves no room to grow:
    streams 2/3 hold a single unused row, which the readers read (and mask) in place of
    every absent row."""
    print("case: decode step empty late streams B2 H2 T640", flush=True)
    w = decode_workload(2, 2, 640, seed=13)
    m3 = np.zeros((2, 640), dtype=bool)
    layer = _build(w, m3, m3.copy())
    assert layer.geometry.row_capacity[2:] == (1, 1)
    assert layer.late_rows_host == [[0, 0], [0, 0]]
    _step_vs_oracle(w, layer, m3, m3.copy())


def _sparse_readers_case(B, H, T, cap, seed, with_counts):
    """Selected-PV sums, the fused loop-3 delta with its loop-2 aggregate and the loop-4
    delta over random sorted selections, against torch over the pack's reconstructed rows
    (pinned to the oracle by the pack tests).  With ``with_counts`` row r's valid slots lie
    below a random count (0, 1 and ``cap`` included) that the readers are given, and the
    results must also match the same calls without counts."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    R = B * H
    bf = torch.bfloat16
    keys = [torch.randn(B, H, T, 128, device=DEV, generator=g).to(bf) for _ in range(4)]
    values = [torch.randn(B, H, T, 128, device=DEV, generator=g).to(bf) for _ in range(4)]
    layer = CrossLoopKVLayer.from_prefill(keys, values, recon=True)
    tp = layer.quantized_tokens
    assert layer.tail_host[0] == T - tp
    cur_k = [torch.randn(B, H, 1, 128, device=DEV, generator=g).to(bf) for _ in range(4)]
    cur_v = [torch.randn(B, H, 1, 128, device=DEV, generator=g).to(bf) for _ in range(4)]
    q = [torch.randn(B, H, 1, 128, device=DEV, generator=g).to(bf) for _ in range(4)]
    # cap sorted distinct indices per row among the T + 1 keys (index T: the current token)
    idx = torch.argsort(torch.rand(R, T + 1, device=DEV, generator=g), dim=1)[:, :cap].sort(dim=1).values.int()
    valid = torch.rand(R, cap, device=DEV, generator=g) > 0.1
    counts = None
    if with_counts:
        # rows of cap/2..cap slots (1 to cap/16 tiles apart), and the tile-boundary rows
        counts = torch.randint(cap // 2, cap + 1, (R,), device=DEV, generator=g, dtype=torch.int32)
        counts[:8] = torch.tensor([0, cap, 1, cap - 1, 2, 7, 8, 9], dtype=torch.int32)
        valid &= torch.arange(cap, device=DEV)[None, :] < counts[:, None]
    valid = valid.to(torch.uint8)
    w = torch.rand(R, cap, device=DEV, generator=g) * valid
    w = w / w.sum(dim=1, keepdim=True).clamp_min(1e-30)
    live = valid.sum(dim=1) > 0  # rows with a selection (the softmax of an empty one is undefined)

    def rows(loop, recon, src, cur):  # [R, T + 1, 128] f32: prefix, tail, current token
        return torch.cat([recon[loop][:, :tp].float(), src[loop].reshape(R, T, 128)[:, tp:].float(),
                          cur[loop].reshape(R, 1, 128).float()], dim=1)

    def pick(x):
        return x.gather(1, idx.long()[..., None].expand(-1, -1, 128))

    def softmax_pv(loop):
        kr, vr = pick(rows(loop, layer.recon_keys, keys, cur_k)), pick(rows(loop, layer.recon_values, values, cur_v))
        lg = torch.einsum("rjc,rc->rj", kr, q[loop].reshape(R, 128).float()) * SCALING
        lg = lg.masked_fill(valid == 0, -float("inf"))
        return torch.einsum("rj,rjc->rc", torch.softmax(lg, dim=1), vr)

    v1 = pick(rows(1, layer.recon_values, values, cur_v))
    want_so = torch.einsum("rj,rjc->rc", w, v1)
    mass = torch.rand(R, device=DEV, generator=g) + 0.5

    def run(c):  # the C-ABI wrappers (the layer passes counts on for ragged batches only)
        view, kw = layer.view(), dict(device=DEV, workspace=layer.workspace, counts=c)
        so = kernels.fused_cross_loop_pv(view, 1, idx, valid, w, cur_v[1], **kw)
        d2, so2 = kernels.fused_sparse_attention_delta_with_source(
            view, 2, q[2], cur_k[2], cur_v[2], idx, valid, w, cur_v[1], mass, SCALING, **kw)
        d3 = kernels.fused_sparse_attention_delta(view, 3, q[3], cur_k[3], cur_v[3], idx, valid, so2, mass, SCALING,
                                                  **kw)
        torch.cuda.synchronize()
        return [t.reshape(R, 128) for t in (so, so2, d2, d3)]

    got = run(counts)
    if with_counts:
        # the partition over live tiles changes only the grouping of the partial sums
        for a_, b_, name in zip(got, run(None), ("pv", "aggregate", "loop-3 delta", "loop-4 delta")):
            print(f"[parity] {name}: counts vs none max abs {float((a_ - b_)[live].abs().max()):.3e}", flush=True)
            assert torch.allclose(a_, b_, atol=1e-5, rtol=1e-5, equal_nan=True), f"{name}: counts change the result"
    so, so2, d2, d3 = got
    # rows of >= 16 selected keys: the absolute bar.  Rows of a few keys average nothing
    # out (outputs of a few V rows reach |4|): a bar relative to the row's magnitude.
    full = valid.sum(dim=1) >= 16

    def check(got_, want_, what):
        assert_close(np32(got_[full]), np32(want_[full]), what=what)
        few = live & ~full
        if bool(few.any()):
            err = (got_[few] - want_[few]).abs().amax(dim=1) / want_[few].abs().amax(dim=1).clamp_min(1.0)
            print(f"[parity] {what}, rows of < 16 keys: max abs err / max(1, |want|) {float(err.max()):.3e}", flush=True)
            assert float(err.max()) <= 2e-2, f"{what}: few-key rows off by {float(err.max()):.3e} relative"

    check(so, want_so, "selected PV, loop 2")
    check(so2, want_so, "fused loop-2 aggregate")
    for loop, d in ((2, d2), (3, d3)):
        check(d, mass[:, None] * (softmax_pv(loop) - so2), f"loop-{loop + 1} delta")


def test_sparse_readers_many_rows_per_wave():
    """5000 rows of six 8-slot tiles: a reader wave's range spans up to four rows (its
    whole middle rows leave its staging early) and rows are split between the waves of a
    workgroup, whose partials of one row are combined before the merge."""
    print("case: sparse readers B625 H8 T130 capacity 48", flush=True)
    _sparse_readers_case(625, 8, 130, 48, seed=21, with_counts=False)


@pytest.mark.parametrize("b,h,t,cap", [(200, 8, 300, 96), (2, 4, 3000, 512), (300, 8, 130, 96)])
def test_sparse_readers_skip_padding_past_counts(b, h, t, cap):
    """Per-row selected counts: the readers split only the tiles below each row's count
    over the grid (rows of 0..cap slots, so rows of one tile sit next to full ones); 2400
    rows exceed the readers' 2048-row prefix and fall back to the padded partition."""
    print(f"case: sparse readers with counts B{b} H{h} T{t} capacity {cap}", flush=True)
    _sparse_readers_case(b, h, t, cap, seed=22 + b, with_counts=True)


def test_decode_step_ragged_batch():
    print("case: decode step ragged B3 H2", flush=True)
    lengths = ragged_lengths(3, 100, 900, seed=2)
    lengths[0] = 100  # packed prefix of one group
    w = decode_workload(3, 2, 0, seed=2, lengths=lengths)
    layer = _build(w)
    _step_vs_oracle(w, layer)


def test_decode_step_many_batches():
    """More sequences than the readers cache lengths for in LDS (1024 dense, 512 gather):
    the rows past the cache read their lengths from the device arrays."""
    print("case: decode step ragged B1030 H1", flush=True)
    lengths = ragged_lengths(1030, 65, 260, seed=5)
    w = decode_workload(1030, 1, 0, seed=5, lengths=lengths)
    layer = _build(w)
    _step_vs_oracle(w, layer)


def test_decode_step_query_and_key_ranges():
    """The sparse readers stage q*scale as fp16 factors normalised by the row's largest
    |q*scaling|: heads whose late-loop queries are 1e-3 .. 4 times the unit draw stay at
    the oracle bar (an unnormalised factor of a 1e-3 query falls into fp16's subnormal
    range).  Sharper rows (16x) leave the bar with fp32 factors too: the oracle's bf16
    residual chain, not the factors, sets that error."""
    print("case: decode step query/key ranges B2 H4 T700", flush=True)
    w = decode_workload(2, 4, 700, seed=12)
    f = torch.tensor([1e-3, 0.05, 1.0, 4.0]).view(1, 4, 1, 1)
    for r in (2, 3):
        w.queries[r] = (w.queries[r].float() * f).to(torch.bfloat16)
    layer = _build(w)
    _step_vs_oracle(w, layer)


def test_decode_step_tiny_selection():
    """A 0.1% retention keeps 3-4 keys per row.  The selection stays bit-exact on the
    kernel's own logits and the aggregate equals the sparse readers' own arithmetic to
    1e-5; against the oracle's bf16 chain the aggregate is then a few dequantised V rows,
    so its mean error is the per-row deviation of the fp32 stream sum (measured 1.2-1.3e-3
    in a randomised sweep), which a 10% selection averages down below 3e-4.  Bound here:
    2e-2 max, 2.5e-3 mean; the deltas keep the standard bound."""
    print("case: decode step tiny selection B2 H4 T3000 frac=0.001", flush=True)
    w = decode_workload(2, 4, 3000, seed=29)
    m3, m4 = _masks(2, 3000, 31, p3=0.3, p4=0.5)
    layer = _build(w, m3, m4)
    R, frac = 8, 0.001
    Kr, Vr = _oracle_rows(w, m3, m4)
    qs = [w.queries[r].to(DEV) for r in range(4)]
    cur = [w.current(r) for r in range(4)]
    step = decode_attention_step(layer, qs, [c[0].to(DEV) for c in cur], [c[1].to(DEV) for c in cur], SCALING, frac)
    torch.cuda.synchronize()
    lengths = [3000] * R
    q = [np32(w.queries[r]).reshape(R, 128) for r in range(4)]
    kc = [np32(c[0]).reshape(R, 128) for c in cur]
    vc = [np32(c[1]).reshape(R, 128) for c in cur]
    g_lg = np32(step.logits1).reshape(R, -1)
    cap = step.indices.shape[-1]
    sel = OA.decode_topk([g_lg[r, :3001] for r in range(R)], frac, kpad=cap)
    assert np.array_equal(step.indices.cpu().numpy().reshape(R, cap), sel.indices), "selected indices differ"
    assert int(sel.count.max()) <= 4
    got = np32(step.selected_output).reshape(R, 128)
    own = restated_selected_aggregate(layer, range(R), sel.indices, sel.valid, sel.selected_weights, vc[1])
    assert_close(got, own, max_abs=1e-5, mean_abs=2e-6, what="selected output vs the readers' arithmetic")
    so = OA.selected_value_aggregate(sel.indices, sel.valid, sel.selected_weights, Vr[1], vc[1], lengths)
    assert_close(got, so, max_abs=2e-2, mean_abs=2.5e-3, what="selected output vs the oracle")
    for loop, d in ((2, step.delta2), (3, step.delta3)):
        want = OA.sparse_delta(q[loop], Kr[loop], Vr[loop], kc[loop], vc[loop], lengths, sel.indices, sel.valid,
                               so, sel.mass, SCALING)
        assert_close(np32(d).reshape(R, 128), want, what=f"loop-{loop + 1} delta")


def test_decode_step_full_fraction_equals_dense():
    """fraction 1 selects every key: loop-2 output + delta == dense loop-3/4 output."""
    print("case: full fraction", flush=True)
    w = decode_workload(1, 2, 300, seed=9)
    layer = _build(w)
    qs = [w.queries[r].to(DEV) for r in range(4)]
    cur = [w.current(r) for r in range(4)]
    step = decode_attention_step(layer, qs, [c[0].to(DEV) for c in cur], [c[1].to(DEV) for c in cur], SCALING, 1.0)
    for loop, d in ((2, step.delta2), (3, step.delta3)):
        dense, _ = layer.dense_source_attention(loop, query=qs[loop], current_key=cur[loop][0].to(DEV),
                                                current_value=cur[loop][1].to(DEV), scaling=SCALING,
                                                return_logits=False)
        got = np32(step.out1 + d)
        assert np.abs(got - np32(dense)).max() < 2e-4


def test_decode_append_and_rollover_bit_exact():
    """Appending decode tokens rolls groups out of the tail (cfg1 semantics): the packed
    streams must equal the oracle's encoding of the whole sequence."""
    print("case: append/rollover", flush=True)
    t0, steps = 190, 75
    w = decode_workload(1, 2, t0, seed=1, extra=steps + 1)
    m3, m4 = _masks(1, t0, 9)
    ks = [w.keys[r][:, :, :t0].contiguous().to(DEV) for r in range(4)]
    vs = [w.values[r][:, :, :t0].contiguous().to(DEV) for r in range(4)]
    layer = CrossLoopKVLayer.from_prefill(ks, vs, mask_loop3=torch.from_numpy(m3).to(DEV),
                                          mask_loop4=torch.from_numpy(m4).to(DEV), token_capacity=512)
    for i in range(steps):
        p = t0 + i
        layer.append_decode_token([w.keys[r][:, :, p:p + 1].to(DEV) for r in range(4)],
                                  [w.values[r][:, :, p:p + 1].to(DEV) for r in range(4)])
    torch.cuda.synchronize()
    total = t0 + steps
    assert layer.quantized_tokens == codec.packed_prefix_tokens(total)
    nk = [np32(w.keys[r][:, :, :total]) for r in range(4)]
    nv = [np32(w.values[r][:, :, :total]) for r in range(4)]
    chain, tp = codec.compress_prefix(nk, nv, (m3, m4))
    assert_layer_matches_chain(layer, chain, tp, 1, 2)
    # and the reader over the rolled cache matches the oracle
    (K, V) = materialized(nk, nv, chain, tp)
    kc, vc = w.keys[1][:, :, total:total + 1], w.values[1][:, :, total:total + 1]
    out, _ = layer.dense_source_attention(1, query=w.queries[1].to(DEV), current_key=kc.to(DEV),
                                          current_value=vc.to(DEV), scaling=SCALING, return_logits=False)
    want, _ = OA.dense_decode(np32(w.queries[1]).reshape(2, 128), flat_rows(K[1]), flat_rows(V[1]),
                              np32(kc).reshape(2, 128), np32(vc).reshape(2, 128), SCALING)
    assert_close(np32(out).reshape(2, 128), want, what="post-rollover output")


def test_rollover_refused_at_row_capacity_changes_nothing():
    """A rollover that would overflow a loop-3/4 row capacity (the exact read-back check)
    raises before any device change: rank maps, row counts, lengths and codes are as
    before, and after the capacity is restored a retried rollover leaves the layer equal
    to one that never hit the limit (no row is counted twice)."""
    import dataclasses

    print("case: rollover at row capacity", flush=True)
    B, H, t0 = 2, 1, 200
    w = decode_workload(B, H, t0, seed=31, extra=80)
    m3, m4 = _masks(B, t0, 31)

    def build():
        ks = [w.keys[r][:, :, :t0].contiguous().to(DEV) for r in range(4)]
        vs = [w.values[r][:, :, :t0].contiguous().to(DEV) for r in range(4)]
        return CrossLoopKVLayer.from_prefill(ks, vs, mask_loop3=torch.from_numpy(m3).to(DEV),
                                             mask_loop4=torch.from_numpy(m4).to(DEV), token_capacity=t0 + 128)

    def append(layer, p, commit=True):
        args = ([w.keys[r][:, :, p:p + 1].to(DEV) for r in range(4)],
                [w.values[r][:, :, p:p + 1].to(DEV) for r in range(4)])
        if commit:
            layer.append_decode_token(*args)
        else:
            layer.append_rows(*args)

    limited, free = build(), build()
    assert limited.tail_host == [72, 72]
    for i in range(55):  # the 56th append fills the tails and rolls a group out
        append(limited, t0 + i)
        append(free, t0 + i)
    late = limited.late_rows_host
    g0 = limited.geometry
    # loop 4 (stream 3) can take only 5 more rows in any sequence; loop 3 has room
    limited.geometry = dataclasses.replace(g0, row_capacity=(*g0.row_capacity[:3], max(late[1]) + 5))
    snap = dict(rank=[r.clone() for r in limited.rank], late=limited.late_rows.clone(),
                packed=limited.packed_tokens.clone(), codes=[c.clone() for c in limited.codes])
    append(limited, t0 + 55, commit=False)
    with pytest.raises(RuntimeError, match="row capacity exhausted"):
        limited.commit_append()
    torch.cuda.synchronize()
    for a_, b_ in zip(limited.rank, snap["rank"]):
        assert torch.equal(a_, b_)
    assert torch.equal(limited.late_rows, snap["late"]) and torch.equal(limited.packed_tokens, snap["packed"])
    for a_, b_ in zip(limited.codes, snap["codes"]):
        assert torch.equal(a_, b_)
    assert limited.packed_host == [128, 128]
    # capacity restored: the retried rollover equals the rollover of the unlimited layer
    limited.geometry = g0
    limited._roll_groups()
    append(free, t0 + 55)
    torch.cuda.synchronize()
    assert limited.packed_host == free.packed_host == [192, 192] and limited.tail_host == free.tail_host
    assert limited.late_rows_host == free.late_rows_host
    for s in range(4):
        assert torch.equal(limited.codes[s], free.codes[s])
    for a_, b_ in zip(limited.rank, free.rank):
        assert torch.equal(a_, b_)


def test_rows_gather_scatter_round_trip():
    print("case: rows", flush=True)
    g = torch.Generator().manual_seed(0)
    hidden = torch.randn(1, 1000, 2048, generator=g).to(torch.bfloat16)
    kv = torch.randn(1, 16, 1000, 128, generator=g).to(torch.bfloat16)
    pos = torch.sort(torch.randperm(1000, generator=g)[:250]).values.to(torch.int32)
    hd, kvd, pd = hidden.to(DEV), kv.to(DEV), pos.to(DEV)
    gh, err = kernels.gather_rows(hd, pd, 1)
    gk, err2 = kernels.gather_rows(kvd, pd, 2)
    torch.cuda.synchronize()
    assert torch.equal(gh.cpu(), hidden.index_select(1, pos.long()))
    assert torch.equal(gk.cpu(), kv.index_select(2, pos.long()))
    assert int(err.item()) == 0 and int(err2.item()) == 0
    new = torch.randn_like(gk.cpu())
    dst = kvd.clone()
    kernels.scatter_rows_(dst, pd, new.to(DEV), 2)
    want = kv.clone().index_copy_(2, pos.long(), new)
    assert torch.equal(dst.cpu(), want)
    assert np.array_equal(dst.cpu().float().numpy(), OT.scatter_rows(np32(kv), pos.numpy(), np32(new), 2))
    # odd row size (4-byte path) and an out-of-range index is reported, not read
    small = torch.arange(2 * 10 * 6, dtype=torch.int16, device=DEV).reshape(2, 10, 6)
    bad = torch.tensor([0, 9, 10], dtype=torch.int32, device=DEV)
    got, err = kernels.gather_rows(small, bad, 1)
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    assert torch.equal(got[:, :2].cpu(), small.cpu()[:, [0, 9]])


def test_hidden_score_and_token_selection():
    print("case: token selection", flush=True)
    g = torch.Generator().manual_seed(1)
    h1 = torch.randn(2, 777, 2048, generator=g).to(torch.bfloat16)
    h2 = (h1.float() + 0.3 * torch.randn(2, 777, 2048, generator=g)).to(torch.bfloat16)
    s = kernels.hidden_delta_score(h2.to(DEV), h1.to(DEV))
    torch.cuda.synchronize()
    want = OT.hidden_delta_score(np32(h2), np32(h1))
    assert np.allclose(s.cpu().numpy(), want, rtol=1e-5)
    sc = s.cpu().numpy()
    mask3, pos3, cnt3, err = kernels.select_tokens(s, 0.25)
    torch.cuda.synchronize()
    want3 = OT.select_active_mask(sc, 0.25)
    assert np.array_equal(mask3.cpu().numpy(), want3)
    assert int(err.item()) == 0
    mask4, pos4, cnt4, err = kernels.select_tokens(s * 0.5, 0.10, eligible=mask3)
    torch.cuda.synchronize()
    want4 = OT.select_active_mask(sc * 0.5, 0.10, eligible=want3)
    assert np.array_equal(mask4.cpu().numpy(), want4)
    assert np.all(~want4 | want3)
    for b in range(2):
        n = int(cnt4[b].item())
        assert n == math.ceil(777 * 0.10)
        assert np.array_equal(pos4[b, :n].cpu().numpy(), np.nonzero(want4[b])[0])
    # ties: equal scores pick lower indices; an ineligible forced token is an error
    flat = torch.zeros(1, 50, device=DEV)
    m, p, c, err = kernels.select_tokens(flat, 0.1)
    torch.cuda.synchronize()
    assert np.array_equal(np.nonzero(m.cpu().numpy()[0])[0], [0, 1, 2, 3, 49])
    el = torch.ones(1, 50, dtype=torch.bool, device=DEV)
    el[0, 49] = False
    m, p, c, err = kernels.select_tokens(flat, 0.1, eligible=el)
    torch.cuda.synchronize()
    assert int(err.item()) == 1


def test_profile_hook_records_the_dense_reader():
    """fl_profile_dense_reader records events around the reader of the selected loop only."""
    import ctypes

    from flashloop_amd import _lib

    print("case: profile hook", flush=True)
    w = decode_workload(1, 2, 300, seed=5)
    layer = _build(w)
    qs = [w.queries[r].to(DEV) for r in range(4)]
    cur = [w.current(r) for r in range(4)]
    lib = _lib.load()
    _lib.check(lib.fl_profile_dense_reader(1, 3), "fl_profile_dense_reader")
    for loop in (0, 1, 1):
        layer.dense_source_attention(loop, query=qs[loop], current_key=cur[loop][0].to(DEV),
                                     current_value=cur[loop][1].to(DEV), scaling=SCALING, return_logits=loop == 1)
    tot, n = ctypes.c_float(0.0), ctypes.c_int32(0)
    _lib.check(lib.fl_profile_dense_reader_read(ctypes.byref(tot), ctypes.byref(n)), "read")
    _lib.check(lib.fl_profile_dense_reader(1, 0), "stop")
    assert n.value == 2 and tot.value > 0.0


@pytest.mark.parametrize("b,h,t", [(4, 4, 4000), (3, 2, 200), (5, 3, 7000), (2, 16, 20000), (9, 16, 32768)])
def test_dense_pair_matches_separate_launches(b, h, t):
    """fl_decode_attn_dense_pair (loops 1 and 2 in one launch) against the two single-loop
    launches: loop-2 logits bit-identical, outputs within 2e-5 (only the split points of
    the partial softmax sums differ), and, for the shapes the oracle finishes quickly,
    both outputs against the oracle at the output bar.  The shapes put the wave whose
    range crosses from loop 1 into loop 2 at different positions inside its workgroup,
    with multi-row ranges on both sides."""
    print("case: dense pair B%d H%d T%d" % (b, h, t), flush=True)
    w = decode_workload(b, h, t, seed=21, device=DEV)
    ks = [w.keys[r][:, :, :t].contiguous() for r in range(4)]
    vs = [w.values[r][:, :, :t].contiguous() for r in range(4)]
    layer = CrossLoopKVLayer.from_prefill(ks, vs)
    del ks, vs
    cur = [w.current(r) for r in range(2)]
    g = torch.Generator(device="cpu").manual_seed(5)
    q = [torch.randn(b, h, 1, 128, generator=g).bfloat16().to(DEV) for _ in range(2)]
    o0, _ = layer.dense_source_attention(0, query=q[0], current_key=cur[0][0], current_value=cur[0][1],
                                         scaling=SCALING, return_logits=False)
    o1, lg = layer.dense_source_attention(1, query=q[1], current_key=cur[1][0], current_value=cur[1][1],
                                          scaling=SCALING, return_logits=True)
    p0, p1, plg = layer.dense_source_attention_pair(queries=q, current_keys=[c[0] for c in cur],
                                                    current_values=[c[1] for c in cur], scaling=SCALING)
    torch.cuda.synchronize()
    keys = t + 1
    assert torch.equal(plg[..., :keys], lg[..., :keys])
    e0 = (p0 - o0).abs().max().item()
    e1 = (p1 - o1).abs().max().item()
    print(f"[parity] pair vs separate: loop 1 {e0:.2e}, loop 2 {e1:.2e}", flush=True)
    assert e0 < 2e-5 and e1 < 2e-5
    if b * h * t <= 64000:
        R = b * h
        nk, nv, chain, tp = oracle_prefix([k[:, :, :t] for k in w.keys], [v[:, :, :t] for v in w.values])
        K, V = materialized(nk, nv, chain, tp)
        for loop, got in ((0, p0), (1, p1)):
            want, _ = OA.dense_decode(np32(q[loop]).reshape(R, 128), flat_rows(K[loop]), flat_rows(V[loop]),
                                      np32(cur[loop][0]).reshape(R, 128), np32(cur[loop][1]).reshape(R, 128), SCALING)
            assert_close(np32(got).reshape(R, 128), want, what=f"pair loop {loop + 1} output vs oracle")


def _assert_half_copies(layer, chain, tp, batch, heads):
    """The fp16 metadata the readers stream, bit for bit: torch's/numpy's fp16 rounding
    (nearest even, overflow to inf; flashloop/packing.py:46) of the oracle's fp32
    scale/min, at the documented layouts: K [bh, group, channel, (scale, min)], V
    [bh, row, half, (scale, min)], and the per-token record [bh, token, half, stream,
    (scale, min)] in fp32."""
    with np.errstate(over="ignore"):  # fp16 copies overflow to inf by design
        bh = batch * heads
        G = tp // 64
        rec = layer.value_meta_token.cpu().numpy()
        for s in range(4):
            sc = chain.streams[s]
            kh = layer.key_meta_half[s].cpu().numpy()
            vh = layer.value_meta_half[s].cpu().numpy()
            want_ks = sc.k_scale.reshape(bh, G, 128).astype(np.float16)
            want_km = sc.k_min.reshape(bh, G, 128).astype(np.float16)
            assert np.array_equal(kh[:, :G, :, 0].view(np.uint16), want_ks.view(np.uint16)), f"stream {s}: fp16 K scale"
            assert np.array_equal(kh[:, :G, :, 1].view(np.uint16), want_km.view(np.uint16)), f"stream {s}: fp16 K min"
            ovs = sc.v_scale.reshape(batch, heads, tp, 2)
            ovm = sc.v_min.reshape(batch, heads, tp, 2)
            for b in range(batch):
                t_idx = np.nonzero(sc.active[b, :tp])[0]
                rows = t_idx if s < 2 else layer.rank[s - 2][b].cpu().numpy()[t_idx]
                for h in range(heads):
                    r = b * heads + h
                    for j, want in ((0, ovs), (1, ovm)):
                        got16 = vh[r, rows, :, j].view(np.uint16)
                        assert np.array_equal(got16, want[b, h, t_idx].astype(np.float16).view(np.uint16)), \
                            f"stream {s}: fp16 V meta {j} (b={b}, h={h})"
                        assert np.array_equal(rec[r, t_idx, :, s, j].view(np.uint32),
                                              want[b, h, t_idx].view(np.uint32)), \
                            f"stream {s}: per-token V record {j} (b={b}, h={h})"


@pytest.mark.parametrize("masked", [False, True])
def test_half_metadata_copies_bit_exact(masked):
    print("case: fp16 metadata copies B2 H3 T390 masked=%s" % masked, flush=True)
    w = decode_workload(2, 3, 390, seed=31)
    m3 = m4 = None
    if masked:
        m3, m4 = _masks(2, 390, 9)
    layer = _build(w, m3, m4)
    nk, nv, chain, tp = oracle_prefix([w.cache(r)[0] for r in range(4)], [w.cache(r)[1] for r in range(4)], m3, m4)
    _assert_half_copies(layer, chain, tp, 2, 3)


def test_extreme_ranges_codec_and_half_copies():
    """Groups whose spans reach the edges of fp32/fp16: huge spans (fp16 scale and min
    overflow to inf), tiny spans (fp16 subnormals and zero), and spans below 2^-100 whose
    scale is subnormal in fp32 (the pack kernel's IEEE-division path).  Codes, fp32
    metadata and reconstructions stay bit-exact with the oracle; the fp16 copies equal
    the fp16 rounding of the oracle's fp32 values."""
    print("case: extreme ranges B1 H4 T200", flush=True)
    b, h, t = 1, 4, 200
    g = torch.Generator().manual_seed(7)
    base = torch.randn(b, h, t, 128, generator=g)
    scales = torch.tensor([3e35, 1e-6, 1e-33, 3e-38]).view(1, h, 1, 1)
    ks, vs = [], []
    for r in range(4):
        drift = 1.0 + 0.1 * r * torch.randn(b, h, t, 128, generator=g)
        ks.append((base * drift * scales).bfloat16())
        vs.append((base.flip(-1) * drift * scales).bfloat16())
    layer = CrossLoopKVLayer.from_prefill([k.to(DEV) for k in ks], [v.to(DEV) for v in vs], recon=True)
    torch.cuda.synchronize()
    nk, nv, chain, tp = oracle_prefix(ks, vs)
    assert_layer_matches_chain(layer, chain, tp, b, h)
    for r in range(4):
        got_k = np32(layer.recon_keys[r]).reshape(b, h, t, 128)[:, :, :tp]
        got_v = np32(layer.recon_values[r]).reshape(b, h, t, 128)[:, :, :tp]
        assert np.array_equal(got_k, chain.recon_keys[r]), f"R_{r} keys differ"
        assert np.array_equal(got_v, chain.recon_values[r]), f"R_{r} values differ"
    # the cases are really reached: inf in fp16, fp32-subnormal scales
    k0 = chain.streams[0].k_scale
    assert np.isinf(k0.astype(np.float16)).any() and (k0[0, 3] < np.float32(2.0**-126)).any()
    _assert_half_copies(layer, chain, tp, b, h)


@pytest.mark.parametrize("masked", [False, True])
def test_signed_zero_minima(masked):
    """Groups whose smallest value is a zero, as +0, -0 or a mix of both (sparse data
    gives -0 from x * 0 with x < 0): the stored minimum is +0 in every copy (fp32 and
    fp16 K and V metadata, the per-token record), bit for bit with the oracle, and the
    codes and reconstructions are bit-exact too."""
    print(f"case: signed-zero minima B2 H2 T300 masked={masked}", flush=True)
    b, h, t = 2, 2, 300
    g = torch.Generator().manual_seed(31)
    ks, vs = [], []
    for r in range(4):
        x = torch.randn(b, h, t, 128, generator=g).abs()
        sign = torch.where(torch.rand(b, h, t, 128, generator=g) < 0.5, -1.0, 1.0)
        keep = torch.rand(b, h, t, 128, generator=g) < 0.3
        k = torch.where(keep, x, torch.zeros(()) * sign)  # >= 0 with +-0 zeros
        k[0, 0] = torch.zeros(()) * sign[0, 0]  # whole row of +-0: K groups and V tokens all zero
        k[1, 1, :, :64] = -0.0  # V halves of only -0
        ks.append(k.bfloat16())
        vs.append(k.flip(-2).bfloat16())
    assert (torch.signbit(ks[0]) & (ks[0] == 0)).any()
    kw, m3, m4 = {}, None, None
    if masked:
        m3, m4 = _masks(b, t, 31, p3=0.3, p4=0.5)
        kw = dict(mask_loop3=torch.from_numpy(m3).to(DEV), mask_loop4=torch.from_numpy(m4).to(DEV))
    layer = CrossLoopKVLayer.from_prefill([k.to(DEV) for k in ks], [v.to(DEV) for v in vs], recon=True, **kw)
    torch.cuda.synchronize()
    nk, nv, chain, tp = oracle_prefix(ks, vs, m3, m4)
    assert_layer_matches_chain(layer, chain, tp, b, h)
    for s_ in range(4):
        km = chain.streams[s_].k_min
        assert not np.signbit(km[km == 0]).any() and (km == 0).any()
    for r in range(4):
        got_k = np32(layer.recon_keys[r]).reshape(b, h, t, 128)[:, :, :tp]
        got_v = np32(layer.recon_values[r]).reshape(b, h, t, 128)[:, :, :tp]
        assert np.array_equal(got_k.view(np.uint32), chain.recon_keys[r].view(np.uint32)), f"R_{r} keys differ"
        assert np.array_equal(got_v.view(np.uint32), chain.recon_values[r].view(np.uint32)), f"R_{r} values differ"
    _assert_half_copies(layer, chain, tp, b, h)


@pytest.mark.parametrize("n", [3000, 40000])
def test_topk_signed_zeros_tie(n):
    """-0.0 and +0.0 are equal scores: their tie goes to the lower index, as in a stable
    sort on (-score, index) and torch.topk.  n=40000 takes the global-memory kernel."""
    print("case: topk signed zeros n=%d" % n, flush=True)
    rng = np.random.default_rng(8)
    lg = rng.standard_normal((2, n)).astype(np.float32)
    lg[:, : n // 2] = np.where(rng.random((2, n // 2)) < 0.5, np.float32(-0.0), np.float32(0.0))
    lg[:, n // 2 :] = -np.abs(lg[:, n // 2 :]) - 1.0  # the zeros are the top half
    frac = 0.1
    sel = OA.decode_topk(lg, frac)
    cap = sel.indices.shape[1]
    nk = torch.full((2,), n, dtype=torch.int32, device=DEV)
    idx, valid, mass, wts, counts = kernels.decode_topk(torch.from_numpy(lg).to(DEV), nk, frac, cap)
    torch.cuda.synchronize()
    k = int(sel.count[0])
    assert np.array_equal(sel.indices[:, :k], np.tile(np.arange(k), (2, 1)))  # oracle: lowest indices
    assert np.array_equal(idx.cpu().numpy(), sel.indices)
    assert np.allclose(mass.cpu().numpy(), sel.mass, rtol=2e-6)


@pytest.mark.parametrize("n", [3000, 40000])
def test_topk_reports_non_finite_scores(n):
    print("case: topk non-finite n=%d" % n, flush=True)
    rng = np.random.default_rng(9)
    lg = rng.standard_normal((5, n)).astype(np.float32)
    neg_nan = np.array([0xFFC00000], dtype=np.uint32).view(np.float32)[0]  # NaN with the sign bit set
    lg[1, 5] = np.nan
    lg[2, 7] = np.inf
    lg[2, 9] = -np.inf
    lg[3, 11] = neg_nan
    lg[4, [0, n - 1]] = np.nan
    lg[4, 100] = neg_nan
    nk = torch.full((5,), n, dtype=torch.int32, device=DEV)
    cap = OA.padded_capacity(OA.decode_budget(n, 0.1))
    nf = torch.full((5,), -1, dtype=torch.int32, device=DEV)
    t = torch.from_numpy(lg).to(DEV)
    kernels.decode_topk(t, nk, 0.1, cap, nonfinite=nf)
    torch.cuda.synchronize()
    assert nf.cpu().tolist() == [0, 1, 2, 1, 3]
    with pytest.raises(ValueError):
        kernels.decode_topk(t, nk, 0.1, cap, validate=True)
    kernels.decode_topk(t[:1], nk[:1], 0.1, cap, validate=True)  # finite row passes


def test_topk_crowded_boundary_bin_and_very_long_rows():
    """Scores clustered in one narrow range (more keys in the boundary bin than the
    resident kernel's 512-entry candidate list: its exact radix ranking within the bin
    runs instead), with exact ties at the boundary; and 70000-key rows (past the 35840
    keys the resident kernel holds: the global-memory kernel)."""
    print("case: topk crowded bin / 70000-key rows", flush=True)
    rng = np.random.default_rng(12)
    n = 40000
    lg = np.empty((3, n), np.float32)
    lg[0] = 1.0 + rng.random(n).astype(np.float32) * 0.1  # one prefix bin [1, 1.125)
    lg[1] = 1.0 + np.round(rng.random(n) * 64).astype(np.float32) / 1024  # one bin, heavy ties
    lg[2] = np.float32(1.0)  # all equal
    for frac in (0.1, 0.5):
        cap = OA.padded_capacity(OA.decode_budget(n, frac))
        idx, valid, mass, wts, counts = kernels.decode_topk(torch.from_numpy(lg).to(DEV),
                                                            torch.full((3,), n, dtype=torch.int32, device=DEV),
                                                            frac, cap)
        torch.cuda.synchronize()
        sel = OA.decode_topk(lg, frac, kpad=cap)
        assert np.array_equal(idx.cpu().numpy(), sel.indices), f"crowded indices differ at {frac}"
        assert np.allclose(mass.cpu().numpy(), sel.mass, rtol=2e-6)
        assert np.allclose(wts.cpu().numpy(), sel.selected_weights, rtol=2e-5, atol=1e-8)
    n = 70000
    lg = (rng.standard_normal((2, n)) * 2.0).astype(np.float32)
    lg[1] = np.round(lg[1] * 4.0) / 4.0
    cap = OA.padded_capacity(OA.decode_budget(n, 0.1))
    idx, valid, mass, wts, counts = kernels.decode_topk(torch.from_numpy(lg).to(DEV),
                                                        torch.full((2,), n, dtype=torch.int32, device=DEV), 0.1, cap)
    torch.cuda.synchronize()
    sel = OA.decode_topk(lg, 0.1, kpad=cap)
    assert np.array_equal(idx.cpu().numpy(), sel.indices)
    assert np.allclose(mass.cpu().numpy(), sel.mass, rtol=2e-6)


@pytest.mark.parametrize("case", ["uniform", "ragged", "many-batches", "full-fraction"])
def test_dense_select_matches_separate_calls(case):
    """fl_decode_attn_dense_select (reader launch, then the top-k and the row merges in one
    launch) against fl_decode_attn_dense + fl_decode_topk: outputs, logits and the whole
    selection bit for bit, for equal and ragged lengths (key counts read from the cache
    view), more batches than the length caches, and fraction 1."""
    print("case: dense select %s" % case, flush=True)
    frac = 1.0 if case == "full-fraction" else 0.10
    if case == "ragged":
        w = decode_workload(5, 3, 0, seed=31, lengths=ragged_lengths(5, 70, 3000, seed=31))
    elif case == "many-batches":
        w = decode_workload(1030, 1, 0, seed=32, lengths=ragged_lengths(1030, 65, 260, seed=32))
    else:
        w = decode_workload(2, 16, 4000, seed=33)
    layer = _build(w)
    q = w.queries[1].to(DEV)
    kc, vc = (x.to(DEV) for x in w.current(1))
    out_a, lg_a = layer.dense_source_attention(1, query=q, current_key=kc, current_value=vc, scaling=SCALING,
                                               return_logits=True)
    sel_a = layer.select_decode_keys(lg_a, frac)
    out_b, lg_b, sel_b = layer.dense_source_attention_select(1, query=q, current_key=kc, current_value=vc,
                                                             scaling=SCALING, fraction=frac)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b), "outputs differ"
    nk = layer.key_counts().cpu().tolist()
    la, lb = lg_a.reshape(layer.rows, -1), lg_b.reshape(layer.rows, -1)
    for r in range(layer.rows):
        n = nk[r // layer.heads]
        assert torch.equal(la[r, :n], lb[r, :n]), f"logits row {r}"
    for name, a, b in zip(("indices", "valid", "mass", "weights", "counts"), sel_a, sel_b):
        assert torch.equal(a, b), f"{name} differ"
