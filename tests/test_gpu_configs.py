"""GPU parity at the shapes of BASELINE.json configs 0-3.

cfg0: B1 H16 T2048, one dense decode step over all four loops, fp32 outputs vs the oracle.
cfg1: T8192 followed by 256 decode appends (a rollover every 64): the packed streams equal
      the oracle's encoding of the whole 8448-token sequence, and a decode step over the
      rolled cache matches the oracle.  Heads are reduced to 2 to keep the CPU oracle in
      seconds; each head is encoded independently, so H does not change the arithmetic.
cfg2: B32 H16, per-sequence contexts drawn from U[1024, 16384] (seeded): one decode step
      over the full ragged batch on the GPU; the rows of the shortest and the longest
      sequence (heads 0 and 15) are checked against the oracle.
cfg3: B8 H16 T32768 (the benchmark shape): one decode step over every row; the first and
      the last row are checked against the oracle (k = 3277 keys in loops 3-4).
"""

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import codec

from flashloop_amd import CrossLoopKVLayer, decode_attention_step
from flashloop_amd.synthetic import SCALING, decode_workload, ragged_lengths

from gpu_util import assert_close, assert_layer_matches_chain, flat_rows, materialized, np32, oracle_prefix

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(keys, values, lengths=None, token_capacity=None):
    layer = CrossLoopKVLayer.from_prefill([k.to(DEV) for k in keys], [v.to(DEV) for v in values], lengths=lengths,
                                          token_capacity=token_capacity)
    torch.cuda.synchronize()
    return layer


def test_cfg0_dense_all_loops():
    print("case: cfg0 B1 H16 T2048 dense, all loops", flush=True)
    B, H, T = 1, 16, 2048
    w = decode_workload(B, H, T, seed=0)
    keys = [w.cache(r)[0] for r in range(4)]
    values = [w.cache(r)[1] for r in range(4)]
    layer = _layer(keys, values)
    nk, nv, chain, tp = oracle_prefix(keys, values)
    assert tp == layer.quantized_tokens == 1984
    assert_layer_matches_chain(layer, chain, tp, B, H)
    K, V = materialized(nk, nv, chain, tp)
    for loop in range(4):
        kc, vc = w.current(loop)
        out, _ = layer.dense_source_attention(loop, query=w.queries[loop].to(DEV), current_key=kc.to(DEV),
                                              current_value=vc.to(DEV), scaling=SCALING, return_logits=False)
        want, _ = OA.dense_decode(np32(w.queries[loop]).reshape(H, 128), flat_rows(K[loop]), flat_rows(V[loop]),
                                  np32(kc).reshape(H, 128), np32(vc).reshape(H, 128), SCALING)
        assert_close(np32(out).reshape(H, 128), want, what=f"cfg0 loop {loop + 1} output")


def test_cfg1_appends_and_rollover():
    print("case: cfg1 T8192 + 256 appends (H2)", flush=True)
    H, T, steps = 2, 8192, 256
    w = decode_workload(1, H, T, seed=1, extra=steps + 1)
    keys = [w.keys[r][:, :, :T].contiguous() for r in range(4)]
    values = [w.values[r][:, :, :T].contiguous() for r in range(4)]
    layer = _layer(keys, values, token_capacity=T + steps + 64)
    seen = {layer.quantized_tokens}
    for i in range(steps):
        p = T + i
        layer.append_decode_token([w.keys[r][:, :, p:p + 1].to(DEV) for r in range(4)],
                                  [w.values[r][:, :, p:p + 1].to(DEV) for r in range(4)])
        seen.add(layer.quantized_tokens)
    torch.cuda.synchronize()
    total = T + steps
    assert layer.quantized_tokens == codec.packed_prefix_tokens(total)
    assert len(seen) == 1 + steps // 64  # one rollover per 64 appends
    nk = [np32(w.keys[r][:, :, :total]) for r in range(4)]
    nv = [np32(w.values[r][:, :, :total]) for r in range(4)]
    chain, tp = codec.compress_prefix(nk, nv, None)
    assert_layer_matches_chain(layer, chain, tp, 1, H)
    K, V = materialized(nk, nv, chain, tp)
    # one decode step over the rolled cache (loops 1-2 dense, 3-4 sparse)
    qs = [w.queries[r].to(DEV) for r in range(4)]
    kc = [w.keys[r][:, :, total:total + 1] for r in range(4)]
    vc = [w.values[r][:, :, total:total + 1] for r in range(4)]
    step = decode_attention_step(layer, qs, [k.to(DEV) for k in kc], [v.to(DEV) for v in vc], SCALING, 0.10)
    torch.cuda.synchronize()
    q = [np32(w.queries[r]).reshape(H, 128) for r in range(4)]
    kcn = [np32(k).reshape(H, 128) for k in kc]
    vcn = [np32(v).reshape(H, 128) for v in vc]
    Kr = [flat_rows(K[r]) for r in range(4)]
    Vr = [flat_rows(V[r]) for r in range(4)]
    o1, _ = OA.dense_decode(q[1], Kr[1], Vr[1], kcn[1], vcn[1], SCALING)
    assert_close(np32(step.out1).reshape(H, 128), o1, what="cfg1 loop-2 output")
    g_lg = np32(step.logits1).reshape(H, -1)[:, : total + 1]
    cap = step.indices.shape[-1]
    sel = OA.decode_topk(list(g_lg), 0.10, kpad=cap)
    assert np.array_equal(step.indices.cpu().numpy().reshape(H, cap), sel.indices)
    lengths = [total] * H
    so = OA.selected_value_aggregate(sel.indices, sel.valid, sel.selected_weights, Vr[1], vcn[1], lengths)
    for loop, got in ((2, step.delta2), (3, step.delta3)):
        want = OA.sparse_delta(q[loop], Kr[loop], Vr[loop], kcn[loop], vcn[loop], lengths, sel.indices, sel.valid,
                               so, sel.mass, SCALING)
        assert_close(np32(got).reshape(H, 128), want, what=f"cfg1 loop-{loop + 1} delta")


def test_cfg2_ragged_batch32():
    print("case: cfg2 B32 H16 ragged [1024, 16384]", flush=True)
    B, H = 32, 16
    lengths = ragged_lengths(B, 1024, 16384, seed=2)
    w = decode_workload(B, H, 0, seed=2, lengths=lengths)
    Tmax = max(lengths)
    layer = _layer([w.cache(r)[0] for r in range(4)], [w.cache(r)[1] for r in range(4)], lengths=lengths)
    qs = [w.queries[r].to(DEV) for r in range(4)]
    cur = [w.current(r) for r in range(4)]
    step = decode_attention_step(layer, qs, [c[0].to(DEV) for c in cur], [c[1].to(DEV) for c in cur], SCALING, 0.10)
    torch.cuda.synchronize()
    R = B * H
    out1 = np32(step.out1).reshape(R, 128)
    d2 = np32(step.delta2).reshape(R, 128)
    d3 = np32(step.delta3).reshape(R, 128)
    g_lg = np32(step.logits1).reshape(R, -1)
    cap = step.indices.shape[-1]
    idx = step.indices.cpu().numpy().reshape(R, cap)
    assert np.isfinite(out1).all() and np.isfinite(d2).all() and np.isfinite(d3).all()
    heads = [0, H - 1]
    for b in (int(np.argmin(lengths)), int(np.argmax(lengths))):
        t = lengths[b]
        ks = [w.keys[r][b:b + 1, heads, :t] for r in range(4)]
        vs = [w.values[r][b:b + 1, heads, :t] for r in range(4)]
        nk, nv, chain, tp = oracle_prefix(ks, vs)
        Kb, Vb = materialized(nk, nv, chain, tp)
        rows = [b * H + h for h in heads]
        q = [np32(w.queries[r]).reshape(R, 128)[rows] for r in range(4)]
        kc = [np32(c[0]).reshape(R, 128)[rows] for c in cur]
        vc = [np32(c[1]).reshape(R, 128)[rows] for c in cur]
        Kr = [flat_rows(Kb[r]) for r in range(4)]
        Vr = [flat_rows(Vb[r]) for r in range(4)]
        o1, _ = OA.dense_decode(q[1], Kr[1], Vr[1], kc[1], vc[1], SCALING)
        assert_close(out1[rows], o1, what=f"cfg2 b={b} (T={t}) loop-2 output")
        sel = OA.decode_topk([g_lg[r, : t + 1] for r in rows], 0.10, kpad=cap)
        assert np.array_equal(idx[rows], sel.indices), f"cfg2 b={b} selection"
        so = OA.selected_value_aggregate(sel.indices, sel.valid, sel.selected_weights, Vr[1], vc[1], [t, t])
        for loop, got in ((2, d2), (3, d3)):
            want = OA.sparse_delta(q[loop], Kr[loop], Vr[loop], kc[loop], vc[loop], [t, t], sel.indices, sel.valid,
                                   so, sel.mass, SCALING)
            assert_close(got[rows], want, what=f"cfg2 b={b} loop-{loop + 1} delta")
    assert Tmax <= 16384


def test_cfg3_full_shape_rows():
    """cfg3 at its full shape (B8 H16 T32768, the benchmark workload): one decode step over
    every row on the GPU; two rows (first and last) are checked against the oracle."""
    print("case: cfg3 B8 H16 T32768", flush=True)
    B, H, T = 8, 16, 32768
    w = decode_workload(B, H, T, seed=3)
    layer = _layer([w.cache(r)[0] for r in range(4)], [w.cache(r)[1] for r in range(4)])
    qs = [w.queries[r].to(DEV) for r in range(4)]
    cur = [w.current(r) for r in range(4)]
    step = decode_attention_step(layer, qs, [c[0].to(DEV) for c in cur], [c[1].to(DEV) for c in cur], SCALING, 0.10)
    torch.cuda.synchronize()
    R = B * H
    out0 = np32(step.out0).reshape(R, 128)
    out1 = np32(step.out1).reshape(R, 128)
    d2 = np32(step.delta2).reshape(R, 128)
    d3 = np32(step.delta3).reshape(R, 128)
    g_lg = np32(step.logits1).reshape(R, -1)
    cap = step.indices.shape[-1]
    idx = step.indices.cpu().numpy().reshape(R, cap)
    for a in (out0, out1, d2, d3):
        assert np.isfinite(a).all()
    for b, h in ((0, 0), (B - 1, H - 1)):
        ks = [w.keys[r][b:b + 1, h:h + 1, :T] for r in range(4)]
        vs = [w.values[r][b:b + 1, h:h + 1, :T] for r in range(4)]
        nk, nv, chain, tp = oracle_prefix(ks, vs)
        Kb, Vb = materialized(nk, nv, chain, tp)
        rows = [b * H + h]
        q = [np32(w.queries[r]).reshape(R, 128)[rows] for r in range(4)]
        kc = [np32(c[0]).reshape(R, 128)[rows] for c in cur]
        vc = [np32(c[1]).reshape(R, 128)[rows] for c in cur]
        Kr = [flat_rows(Kb[r]) for r in range(4)]
        Vr = [flat_rows(Vb[r]) for r in range(4)]
        o0, _ = OA.dense_decode(q[0], Kr[0], Vr[0], kc[0], vc[0], SCALING)
        o1, _ = OA.dense_decode(q[1], Kr[1], Vr[1], kc[1], vc[1], SCALING)
        assert_close(out0[rows], o0, what=f"cfg3 row {rows[0]} loop-1 output")
        assert_close(out1[rows], o1, what=f"cfg3 row {rows[0]} loop-2 output")
        sel = OA.decode_topk([g_lg[r, : T + 1] for r in rows], 0.10, kpad=cap)
        assert np.array_equal(idx[rows], sel.indices), f"cfg3 row {rows[0]} selection"
        assert sel.count[0] == 3277
        so = OA.selected_value_aggregate(sel.indices, sel.valid, sel.selected_weights, Vr[1], vc[1], [T])
        for loop, got in ((2, d2), (3, d3)):
            want = OA.sparse_delta(q[loop], Kr[loop], Vr[loop], kc[loop], vc[loop], [T], sel.indices, sel.valid,
                                   so, sel.mass, SCALING)
            assert_close(got[rows], want, what=f"cfg3 row {rows[0]} loop-{loop + 1} delta")
