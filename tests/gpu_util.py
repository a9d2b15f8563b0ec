"""Helpers shared by the GPU parity tests (host-side conversions only)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import attention as OA
from oracle import codec


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def unpack_codes(codes: torch.Tensor) -> np.ndarray:
    """u8 ``[..., 64]`` rows (channel 2j low nibble, 2j+1 high) -> ``[..., 128]``."""
    c = codes.cpu().numpy()
    out = np.empty(c.shape[:-1] + (128,), np.uint8)
    out[..., 0::2] = c & 0xF
    out[..., 1::2] = c >> 4
    return out


def oracle_prefix(keys, values, m3=None, m4=None):
    """Oracle chain over the packed prefix of [B,H,T,128] bf16 torch tensors."""
    nk = [np32(k) for k in keys]
    nv = [np32(v) for v in values]
    masks = None if m3 is None else (np.asarray(m3, bool), np.asarray(m4, bool))
    chain, tp = codec.compress_prefix(nk, nv, masks)
    return nk, nv, chain, tp


def assert_layer_matches_chain(layer, chain, tp, batch, heads, row_ids=None):
    """Bit-exact codes, K/V metadata (compared as bit patterns, so the sign of a zero counts) of all four streams against the oracle chain.
    ``row_ids``: the layer's (b,h) rows of the chain's rows (default: the same rows)."""
    bh = batch * heads
    ids = np.arange(bh) if row_ids is None else np.asarray(row_ids)
    G = tp // 64
    for s in range(4):
        sc = chain.streams[s]
        kc = unpack_codes(layer.key_codes[s])
        vc = unpack_codes(layer.value_codes[s])
        kmeta = layer.key_meta[s].cpu().numpy()
        vmeta = layer.value_meta[s].cpu().numpy()
        ks = sc.k_scale.reshape(bh, G, 128)
        km = sc.k_min.reshape(bh, G, 128)
        assert np.array_equal(kmeta[ids, :G, :, 0].view(np.uint32), ks.view(np.uint32)), f"stream {s}: K scale mismatch"
        assert np.array_equal(kmeta[ids, :G, :, 1].view(np.uint32), km.view(np.uint32)), f"stream {s}: K min mismatch"
        okc = sc.k_codes.reshape(batch, heads, tp, 128)
        ovc = sc.v_codes.reshape(batch, heads, tp, 128)
        ovs = sc.v_scale.reshape(batch, heads, tp, 2)
        ovm = sc.v_min.reshape(batch, heads, tp, 2)
        for b in range(batch):
            act = sc.active[b, :tp]
            t_idx = np.nonzero(act)[0]
            if s < 2:
                rows = t_idx
            else:
                rank = layer.rank[s - 2][b].cpu().numpy()
                rows = rank[t_idx]
                assert np.all(rows >= 0), "active row without a rank"
                assert np.all(rank[:tp][~act] == -1)
            for h in range(heads):
                r = ids[b * heads + h]
                assert np.array_equal(kc[r, rows], okc[b, h, t_idx]), f"stream {s}: K codes mismatch (b={b}, h={h})"
                assert np.array_equal(vc[r, rows], ovc[b, h, t_idx]), f"stream {s}: V codes mismatch (b={b}, h={h})"
                assert np.array_equal(vmeta[r, rows, :, 0].view(np.uint32), ovs[b, h, t_idx].view(np.uint32)), f"stream {s}: V scale mismatch"
                assert np.array_equal(vmeta[r, rows, :, 1].view(np.uint32), ovm[b, h, t_idx].view(np.uint32)), f"stream {s}: V min mismatch"


def materialized(nk, nv, chain, tp):
    """Per-loop K_r/V_r the reference attends to: reconstructed prefix + raw tail."""
    return codec.materialize_loop_cache(nk, nv, chain, tp)


def flat_rows(x: np.ndarray, lengths=None):
    """[B,H,T,C] -> list over (b,h) of [T_b, C] arrays."""
    b, h = x.shape[:2]
    out = []
    for i in range(b):
        t = x.shape[2] if lengths is None else lengths[i]
        for j in range(h):
            out.append(x[i, j, :t])
    return out


def assert_close(got: np.ndarray, want: np.ndarray, max_abs: float = 2e-2, mean_abs: float = 1e-3, what: str = ""):
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    print(f"[parity] {what}: max abs {err.max():.3e} mean abs {err.mean():.3e}", flush=True)
    assert err.max() <= max_abs, f"{what}: max abs err {err.max():.3e} > {max_abs}"
    assert err.mean() <= mean_abs, f"{what}: mean abs err {err.mean():.3e} > {mean_abs}"
    return float(err.max()), float(err.mean())


def restated_dense_logits(layer, loop: int, rows, q, k_cur, scaling: float) -> list:
    """fp64 logits of the dense reader's own arithmetic for the (b,h) rows ``rows``:
    prefix keys K[t] = sum_{s<=loop} (code_s[t] * scale16_s + min16_s) from the packed
    codes and the fp16 metadata copies (streams 2/3 only at tokens with a rank), with no
    bf16 rounding between streams; then the raw BF16 tail rows and the current key.

    The codes and the fp16 copies are themselves pinned bit for bit against the oracle
    (``assert_layer_matches_chain``, the fp16 copy tests), so this pins the kernel's
    contraction to ~1e-6 -- the oracle comparison then bounds what the skipped bf16
    re-rounding of the reference chain adds (~2e-3 on logits).  ``q``/``k_cur``:
    float arrays ``[len(rows), 128]``."""
    out = []
    heads = layer.heads
    for i, r in enumerate(rows):
        b = r // heads
        tp = layer.packed_host[b]
        tl = layer.tail_host[b]
        G = tp // 64
        qd = np.asarray(q[i], np.float64) * scaling
        lg = np.zeros(tp + tl + 1, np.float64)
        for s in range(loop + 1):
            meta = layer.key_meta_half[s][r, :G].float().cpu().numpy().astype(np.float64)  # [G, 128, 2]
            if s < 2:
                rows_s = np.arange(tp)
                present = np.ones(tp, bool)
            else:
                rank = layer.rank[s - 2][b, :tp].cpu().numpy()
                present = rank >= 0
                rows_s = np.where(present, rank, 0)
            codes = unpack_codes(layer.key_codes[s][r])[rows_s].astype(np.float64)  # [tp, 128]
            scale = np.repeat(meta[:, :, 0], 64, axis=0)
            mn = np.repeat(meta[:, :, 1], 64, axis=0)
            lg[:tp] += np.where(present, (codes * scale + mn) @ qd, 0.0)
        tail = layer.tail_key[loop][r, :tl].float().cpu().numpy().astype(np.float64)
        lg[tp:tp + tl] = tail @ qd
        lg[tp + tl] = np.asarray(k_cur[i], np.float64) @ qd
        out.append(lg)
    return out


def restated_selected_aggregate(layer, rows, indices, valid, weights, v_cur) -> np.ndarray:
    """fp64 loop-2 selected aggregate ``sum_j w_j V[t_j]`` of the sparse readers' own
    arithmetic for the (b,h) rows ``rows``: a prefix token's V is
    ``sum_{s<=1} code_s * scale_s + min_s`` from the packed codes and the fp32 per-token
    metadata, with no bf16 rounding between the streams; tail rows and the current token
    are the raw BF16 rows.  ``indices``/``valid``/``weights``: ``[len(rows), cap]``;
    ``v_cur``: ``[len(rows), 128]``."""
    out = []
    heads = layer.heads
    for i, r in enumerate(rows):
        b = r // heads
        tp, tl = layer.packed_host[b], layer.tail_host[b]
        acc = np.zeros(128, np.float64)
        for j in np.nonzero(valid[i])[0]:
            t, wt = int(indices[i, j]), float(weights[i, j])
            if t < tp:
                v = np.zeros(128, np.float64)
                for s in range(2):
                    codes = unpack_codes(layer.value_codes[s][r, t]).astype(np.float64)  # [128]
                    meta = layer.value_meta[s][r, t].cpu().numpy().astype(np.float64)  # [half, (scale, min)]
                    v += codes * np.repeat(meta[:, 0], 64) + np.repeat(meta[:, 1], 64)
            elif t < tp + tl:
                v = layer.tail_value[1][r, t - tp].float().cpu().numpy().astype(np.float64)
            else:
                v = np.asarray(v_cur[i], np.float64)
            acc += wt * v
        out.append(acc)
    return np.stack(out)


def step_vs_oracle_rows(got, rows, H, nk, nv, masks, q, kc, vc, scaling, fraction, what=""):
    """One decode step of a batch-one cache against the oracle at the head rows ``rows``.

    ``got``: the step's tensors (``out0``, ``out1`` [H,128]-shaped, ``logits1`` [H, >= T+1],
    ``indices`` [H, cap], ``delta2``, ``delta3``); ``nk``/``nv``: per loop, float32
    ``[1, len(rows), T, 128]`` K/V of every cached token of those heads; ``masks``: the
    loop-3/4 active rows ``(m3, m4)`` ``[1, T]`` or None; ``q``/``kc``/``vc``: per loop,
    ``[len(rows), 128]``.  Checks the loop-1/2 outputs, the selection bit for bit on the
    kernel's logits and the loop-3/4 deltas.  Returns the oracle chain and its prefix."""
    chain, tp = codec.compress_prefix(nk, nv, masks)
    K, V = materialized(nk, nv, chain, tp)
    T = nk[0].shape[2]
    idx = np.asarray(rows)
    Kr = [flat_rows(K[r]) for r in range(4)]
    Vr = [flat_rows(V[r]) for r in range(4)]
    o0, _ = OA.dense_decode(q[0], Kr[0], Vr[0], kc[0], vc[0], scaling)
    o1, _ = OA.dense_decode(q[1], Kr[1], Vr[1], kc[1], vc[1], scaling)
    assert_close(np32(got["out0"]).reshape(H, 128)[idx], o0, what=f"{what} loop-1 output")
    assert_close(np32(got["out1"]).reshape(H, 128)[idx], o1, what=f"{what} loop-2 output")
    g_lg = np32(got["logits1"]).reshape(H, -1)[idx, : T + 1]
    cap = got["indices"].shape[-1]
    sel = OA.decode_topk(list(g_lg), fraction, kpad=cap)
    assert np.array_equal(got["indices"].cpu().numpy().reshape(H, cap)[idx], sel.indices), f"{what}: selection"
    lengths = [T] * len(rows)
    so = OA.selected_value_aggregate(sel.indices, sel.valid, sel.selected_weights, Vr[1], vc[1], lengths)
    for loop in (2, 3):
        want = OA.sparse_delta(q[loop], Kr[loop], Vr[loop], kc[loop], vc[loop], lengths, sel.indices, sel.valid,
                               so, sel.mass, scaling)
        assert_close(np32(got[f"delta{loop}"]).reshape(H, 128)[idx], want, what=f"{what} loop-{loop + 1} delta")
    return chain, tp
