"""GPU parity at the shapes of BASELINE.json configs 0-3.

cfg0: B1 H16 T2048, one dense decode step over all four loops, fp32 outputs vs the oracle.
cfg1: T8192 followed by 256 decode appends (a rollover every 64): the packed streams equal
      the oracle's encoding of the whole 8448-token sequence, and a decode step over the
      rolled cache matches the oracle (H2); and at H16 a decode step before every append,
      checked against the oracle after each of the four rollovers (three heads; each head
      is encoded independently, so a subset of heads is exact).
cfg2: B32 H16, per-sequence contexts drawn from U[1024, 16384] (seeded): one decode step
      over the full ragged batch on the GPU; every head of the shortest and of the longest
      sequence is checked against the oracle.
cfg3: B8 H16 T32768 (the benchmark shape): one decode step over every row; 16 rows, chosen
      where the dense readers' persistent-wave ranges start or end (tail/prefix splits),
      are checked against the oracle (k = 3277 keys in loops 3-4).
The full-shape workloads are drawn on the device (same distributions; the oracle reads
the rows it checks back from it).  Logits are held twice: within 1e-4 of an fp64
restatement of the reader's own contraction over the (oracle-pinned) codes and fp16
metadata, and within 2e-2 max / 5e-3 mean of the oracle's bf16-chain logits.
"""

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import codec

from flashloop_amd import CrossLoopKVLayer, decode_attention_step
from flashloop_amd.synthetic import SCALING, decode_workload, ragged_lengths

from gpu_util import (
    assert_close,
    step_vs_oracle_rows,
    assert_layer_matches_chain,
    flat_rows,
    materialized,
    np32,
    oracle_prefix,
    restated_dense_logits,
)

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


def test_cfg1_decode_every_step_across_rollovers():
    """BASELINE config 1 as configured: B1 H16 T8192, 256 consecutive decode steps, each a
    full 4-loop decode step over the cache followed by the append of its token (a tail
    rollover every 64 appends).  The step after each of the four rollovers (steps 64,
    128, 192, 256) is checked against the oracle at heads 0, 7 and 15, and at the end
    the packed streams of those heads equal the oracle's encoding of all 8448 tokens."""
    print("case: cfg1 H16 T8192, decode + append x256", flush=True)
    H, T, steps = 16, 8192, 256
    heads = [0, 7, 15]
    w = decode_workload(1, H, T, seed=11, extra=steps + 1)
    keys = [w.keys[r][:, :, :T].contiguous() for r in range(4)]
    values = [w.values[r][:, :, :T].contiguous() for r in range(4)]
    layer = _layer(keys, values, token_capacity=T + steps + 64)
    gen = torch.Generator().manual_seed(111)
    rolled = []
    checked = 0
    for i in range(steps + 1):
        p = T + i
        qs = [torch.randn((1, H, 1, 128), generator=gen).to(torch.bfloat16) for _ in range(4)]
        kc = [w.keys[r][:, :, p:p + 1] for r in range(4)]
        vc = [w.values[r][:, :, p:p + 1] for r in range(4)]
        step = decode_attention_step(layer, [x.to(DEV) for x in qs], [k.to(DEV) for k in kc],
                                     [v.to(DEV) for v in vc], SCALING, 0.10)
        if i in (64, 128, 192, 256):
            torch.cuda.synchronize()
            assert layer.quantized_tokens == codec.packed_prefix_tokens(p), f"step {i}"
            nk = [np32(w.keys[r][:, heads, :p]) for r in range(4)]
            nv = [np32(w.values[r][:, heads, :p]) for r in range(4)]
            q = [np32(x)[0, heads].reshape(len(heads), 128) for x in qs]
            kcn = [np32(k)[0, heads].reshape(len(heads), 128) for k in kc]
            vcn = [np32(v)[0, heads].reshape(len(heads), 128) for v in vc]
            got = dict(out0=step.out0, out1=step.out1, logits1=step.logits1, indices=step.indices,
                       delta2=step.delta2, delta3=step.delta3)
            chain, tp = step_vs_oracle_rows(got, heads, H, nk, nv, None, q, kcn, vcn, SCALING, 0.10,
                                            what=f"cfg1 step {i}")
            checked += 1
        else:
            assert bool(torch.isfinite(step.out1).all()) and bool(torch.isfinite(step.delta3).all()), f"step {i}"
        if i < steps:
            before = layer.quantized_tokens
            layer.append_decode_token([k.to(DEV) for k in kc], [v.to(DEV) for v in vc])
            if layer.quantized_tokens != before:
                rolled.append(i)
    torch.cuda.synchronize()
    assert rolled == [63, 127, 191, 255] and checked == 4
    # the packed streams of the checked heads, after the last rollover
    assert tp == layer.quantized_tokens
    assert_layer_matches_chain(layer, chain, tp, 1, len(heads), row_ids=heads)


def _check_rows(w, layer, step, rows, H, lengths, what):
    """Oracle parity of the decode step at the (b,h) rows ``rows`` (one vectorised oracle
    encode of those rows): loop-1/2 outputs, logits (restated and oracle bars), the
    selection bit for bit on the kernel's logits, the selected aggregate and both deltas."""
    R = step.out1.numel() // 128
    cur = [w.current(r) for r in range(4)]
    tmax = max(lengths[r // H] for r in rows)
    ks = [torch.stack([w.keys[r][x // H, x % H, :tmax] for x in rows])[None] for r in range(4)]
    vs = [torch.stack([w.values[r][x // H, x % H, :tmax] for x in rows])[None] for r in range(4)]
    Kr = [[] for _ in range(4)]
    Vr = [[] for _ in range(4)]
    # rows of one length share one oracle call (each row is encoded independently)
    by_len = {}
    for i, x in enumerate(rows):
        by_len.setdefault(lengths[x // H], []).append(i)
    per_row = {}
    for t, idxs in by_len.items():
        nk, nv, chain, tp = oracle_prefix([k[:, idxs, :t] for k in ks], [v[:, idxs, :t] for v in vs])
        Kb, Vb = materialized(nk, nv, chain, tp)
        for j, i in enumerate(idxs):
            per_row[i] = ([Kb[r][0, j] for r in range(4)], [Vb[r][0, j] for r in range(4)])
    for r in range(4):
        Kr[r] = [per_row[i][0][r] for i in range(len(rows))]
        Vr[r] = [per_row[i][1][r] for i in range(len(rows))]
    q = [np32(w.queries[r]).reshape(R, 128)[rows] for r in range(4)]
    kc = [np32(c[0]).reshape(R, 128)[rows] for c in cur]
    vc = [np32(c[1]).reshape(R, 128)[rows] for c in cur]
    lens = [lengths[x // H] for x in rows]
    o0, _ = OA.dense_decode(q[0], Kr[0], Vr[0], kc[0], vc[0], SCALING)
    o1, lg1 = OA.dense_decode(q[1], Kr[1], Vr[1], kc[1], vc[1], SCALING)
    assert_close(np32(step.out0).reshape(R, 128)[rows], o0, what=f"{what} loop-1 output")
    assert_close(np32(step.out1).reshape(R, 128)[rows], o1, what=f"{what} loop-2 output")
    g_lg = np32(step.logits1).reshape(R, -1)
    got_lg = [g_lg[x, : lens[i] + 1] for i, x in enumerate(rows)]
    rest = restated_dense_logits(layer, 1, rows, q[1], kc[1], SCALING)
    assert_close(np.concatenate(got_lg), np.concatenate(rest), max_abs=1e-4, mean_abs=1e-5,
                 what=f"{what} logits vs restated reader arithmetic")
    assert_close(np.concatenate(got_lg), np.concatenate([np.asarray(x) for x in lg1]), max_abs=2e-2, mean_abs=5e-3,
                 what=f"{what} logits vs oracle bf16 chain")
    cap = step.indices.shape[-1]
    idx = step.indices.cpu().numpy().reshape(R, cap)
    sel = OA.decode_topk(got_lg, 0.10, kpad=cap)
    assert np.array_equal(idx[rows], sel.indices), f"{what} selection"
    so = OA.selected_value_aggregate(sel.indices, sel.valid, sel.selected_weights, Vr[1], vc[1], lens)
    assert_close(np32(step.selected_output).reshape(R, 128)[rows], so, what=f"{what} selected output")
    for loop, got in ((2, step.delta2), (3, step.delta3)):
        want = OA.sparse_delta(q[loop], Kr[loop], Vr[loop], kc[loop], vc[loop], lens, sel.indices, sel.valid,
                               so, sel.mass, SCALING)
        assert_close(np32(got).reshape(R, 128)[rows], want, what=f"{what} loop-{loop + 1} delta")
    return sel


def _run_step(w, layer):
    qs = [q.contiguous() for q in w.queries]
    cur = [w.current(r) for r in range(4)]
    step = decode_attention_step(layer, qs, [c[0] for c in cur], [c[1] for c in cur], SCALING, 0.10)
    torch.cuda.synchronize()
    for t in (step.out0, step.out1, step.delta2, step.delta3, step.selected_output):
        assert bool(torch.isfinite(t).all())
    return step


@pytest.mark.parametrize("which", ["shortest", "longest"])
def test_cfg2_ragged_batch32(which):
    """cfg2 at its shape; every head of the shortest / the longest sequence."""
    print(f"case: cfg2 B32 H16 ragged [1024, 16384], {which} sequence", flush=True)
    B, H = 32, 16
    lengths = ragged_lengths(B, 1024, 16384, seed=2)
    assert max(lengths) <= 16384 and min(lengths) >= 1024
    w = decode_workload(B, H, 0, seed=2, lengths=lengths, device=DEV)
    layer = _layer([w.cache(r)[0] for r in range(4)], [w.cache(r)[1] for r in range(4)], lengths=lengths)
    step = _run_step(w, layer)
    b = int(np.argmin(lengths)) if which == "shortest" else int(np.argmax(lengths))
    rows = [b * H + h for h in range(H)]
    sel = _check_rows(w, layer, step, rows, H, lengths, f"cfg2 b={b} (T={lengths[b]})")
    assert list(sel.count) == [OA.decode_budget(lengths[b] + 1, 0.10)] * H


def cfg3_boundary_rows(B=8, H=16, T=32768, per_split=8):
    """Rows of cfg3 where a dense reader's persistent-wave range begins: a row spans
    3 tail units + Tp/64 prefix groups of the global work sequence, and the waves split
    it into contiguous ranges of ceil(U / waves) units.  For both reader grids on a
    256-CU part (1024 waves: loop 2, one workgroup per CU; 2048 waves: loop 1, two) the
    rows whose first range boundary falls earliest after the row start -- at the tail, or
    between the tail and the first prefix group -- are taken; every row also has
    boundaries mid-prefix (a row spans 8-16 ranges)."""
    span = 3 + (T - 64) // 64
    U = B * H * span
    out = []
    for waves in (1024, 2048):
        chunk = -(-U // waves)
        off = [(-(r * span)) % chunk for r in range(B * H)]
        for r in sorted(range(B * H), key=lambda r: (off[r], r)):
            if r not in out:
                out.append(r)
            if len(out) % per_split == 0 and len(out) >= per_split * (1 + (waves == 2048)):
                break
    return out


@pytest.mark.parametrize("half", [0, 1])
def test_cfg3_full_shape_rows(half):
    """cfg3 at its full shape (B8 H16 T32768, the benchmark workload): one decode step over
    every row on the GPU; 8 of the 16 wave-boundary rows per half are checked."""
    B, H, T = 8, 16, 32768
    rows = cfg3_boundary_rows(B, H, T)[8 * half: 8 * half + 8]
    print(f"case: cfg3 B8 H16 T32768 rows {rows}", flush=True)
    w = decode_workload(B, H, T, seed=3, device=DEV)
    layer = _layer([w.cache(r)[0] for r in range(4)], [w.cache(r)[1] for r in range(4)])
    step = _run_step(w, layer)
    sel = _check_rows(w, layer, step, rows, H, [T] * B, "cfg3")
    assert list(sel.count) == [3277] * len(rows)
