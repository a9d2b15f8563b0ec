"""Decode attention, decode top-k and the cached-mass sparse delta, restated in numpy.

Test infrastructure: the checker for ``fl_decode_attn_dense``, ``fl_decode_topk``,
``fl_decode_selected_pv`` and ``fl_decode_attn_sparse_delta``.

Vectors are float32/float64 numpy arrays, rows flattened over ``(batch, head)``.
Attention is evaluated in float64 (the reference evaluates the same formulas in
float32; the float64 value is the closer ground truth for both).

Pinned by (tests/test_oracle_attention.py): brute-force nested loops on tiny
inputs, the identity ``cached-mass delta == mass_scaled_sparse_output`` of
flashloop_torch (attention_utils.py:216-248) with ``cached_source_mass`` scales,
sparse == dense when the fraction is 1 (config.py:73-77), ``sum softmax == 1``,
``mass in (0, 1]``, the budget formula, and top-k == a stable argsort on
``(-score, index)`` / the 3x3 known-answer of attention_utils.py:638-654.  The fp32
softmax weight image the selection ranks is pinned in tests/test_oracle_topk_weights.py.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


def _softmax64(x: np.ndarray, axis: int = -1) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def dense_decode(q, keys, values, k_cur, v_cur, scaling):
    """One-query attention over ``[past ; current]`` keys.

    Restates ``CrossLoopKVLayer.dense_source_attention``'s reference branch
    (flashloop/cache.py:1735-1756): ``logits = q.K^T * scaling`` over the logical
    prefix, the tail and the current token; fp32 softmax; ``out = P.V``.

    q, k_cur, v_cur: ``[R, C]``; keys/values: ``[R, T, C]`` (a list of per-row arrays
    of differing T is accepted for ragged batches).  Returns ``(out [R, C],
    logits list or [R, T+1])`` as float64.
    """
    outs, logits = [], []
    for r in range(len(q)):
        k = np.concatenate([np.asarray(keys[r], np.float64), np.asarray(k_cur[r], np.float64)[None]], 0)
        v = np.concatenate([np.asarray(values[r], np.float64), np.asarray(v_cur[r], np.float64)[None]], 0)
        lg = (k @ np.asarray(q[r], np.float64)) * float(scaling)
        p = _softmax64(lg)
        outs.append(p @ v)
        logits.append(lg)
    out = np.stack(outs)
    if all(len(x) == len(logits[0]) for x in logits):
        return out, np.stack(logits)
    return out, logits


def decode_budget(keys: int, fraction: float) -> int:
    """``min(T+1, max(1, ceil((T+1) * f)))`` (engine.py:443-452; attention_utils.py:143-144)."""
    return min(keys, max(1, math.ceil(keys * fraction)))


def padded_capacity(count: int, block: int = 64) -> int:
    """``_pad_decode_indices`` capacity (engine.py:84-109): one spare block at exact multiples."""
    return (count // block + 1) * block


@dataclass
class DecodeSelection:
    indices: np.ndarray  # int32 [R, kpad], ascending, zero padded
    valid: np.ndarray  # bool [R, kpad]
    mass: np.ndarray  # float64 [R]
    selected_weights: np.ndarray  # float64 [R, kpad] = w / mass, 0 where invalid
    count: np.ndarray  # int [R]


def topk_order(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices of the ``k`` largest scores, ties broken by lower index, returned ascending.

    ``torch.topk`` leaves the tie order unspecified (engine.py:453); the workload
    definition fixes it to the lower index.  A stable argsort on ``-score`` yields
    exactly that order.
    """
    s = np.asarray(scores)
    order = np.argsort(-s.astype(np.float64), kind="stable")
    return np.sort(order[:k]).astype(np.int32)


# ---- the fp32 softmax weight image that the decode selection ranks ----------------------
# engine.py:439-453 (and selection.py:85) rank ``w = softmax(logits, dtype=float32)``: two
# different logits whose fp32 weights are equal tie, and ties go to the lower index.  The
# image below is the one the HIP top-k forms, op for op in float32:
#   e = softmax_exp(RN(x - max)), Z = the sum of e in the kernels' fixed order,
#   w = RN(e * RN(1 / Z)).
# Pinned (tests/test_oracle_topk_weights.py) by: fma32 against exact rational arithmetic,
# softmax_exp within 2 ulp of the float64 exp (and exact at 0 and in the underflow range),
# Z and w within a few ulp of the float64 softmax, and the ranking equal to torch's own
# fp32 softmax ranking on rows where the logit ranking differs from it.

_F = np.float32
LN2_HI = _F(float.fromhex("0x1.62e430p-1"))
LN2_LO = _F(float.fromhex("-0x1.05c610p-29"))
INV_LN2 = _F(float.fromhex("0x1.715476p+0"))
_POLY = [_F(float.fromhex(h)) for h in ("0x1.a01a02p-13", "0x1.6c16c2p-10", "0x1.111112p-7",
                                         "0x1.555556p-5", "0x1.555556p-3")] + [_F(0.5), _F(1.0), _F(1.0)]
TOPK_THREADS = 1024
TOPK_WAVE = 64


def fma32(a, b, c) -> np.ndarray:
    """Correctly rounded float32 ``a*b + c``: the product is exact in float64, the sum is
    formed in float64 rounded to odd (TwoSum error, then the last bit forced odd when
    inexact), and one rounding to float32 follows (Boldo & Melquiond, 2008: round-to-odd
    with >= 2 extra bits makes the double rounding exact)."""
    a = np.asarray(a, np.float32).astype(np.float64)
    b = np.asarray(b, np.float32).astype(np.float64)
    c = np.asarray(c, np.float32).astype(np.float64)
    p = a * b  # exact: 48 significant bits
    with np.errstate(invalid="ignore", over="ignore"):
        s = p + c
        bb = s - p
        err = (p - (s - bb)) + (c - bb)
    bits = s.view(np.int64)
    fix = (err != 0) & ((bits & 1) == 0) & np.isfinite(s)
    toward = np.where(err > 0, np.inf, -np.inf)
    s = np.where(fix, np.nextafter(s, toward), s)
    return s.astype(np.float32)


def softmax_exp32(d) -> np.ndarray:
    """The kernels' fp32 ``exp(d)`` for ``d <= 0`` (topk.hip ``softmax_exp``): Cody-Waite
    reduction with ``n = rint(d / ln2)``, degree-7 Taylor polynomial by Horner in fma, and
    the scale ``2^n`` as an exact multiply by ``2^(n+64)`` then a rounding multiply by
    ``2^-64``."""
    d = np.maximum(np.asarray(d, np.float32), _F(-112.0))
    n = np.rint(d * INV_LN2)
    r = fma32(n, -LN2_HI, d)
    r = fma32(n, -LN2_LO, r)
    p = np.full_like(r, _POLY[0])
    for c in _POLY[1:]:
        p = fma32(p, r, c)
    up = ((n.astype(np.int32) + 64 + 127) << 23).astype(np.uint32).view(np.float32)
    return (p * up) * _F(2.0 ** -64)


def weight_sum_fixed(e: np.ndarray) -> np.float32:
    """The kernels' normaliser: thread t of 1024 sums indices q*4096 + 4t + e in (q, e)
    order (4 contiguous keys per thread per 4096-key chunk); each wave of 64 threads adds
    lane pairs at distance 32, 16, ..., 1; the 16 wave sums are added in wave order."""
    e = np.asarray(e, np.float32)
    n = e.shape[0]
    chunk = 4 * TOPK_THREADS
    rows = max(1, -(-n // chunk))
    buf = np.zeros(rows * chunk, np.float32)
    buf[:n] = e
    buf = buf.reshape(rows, TOPK_THREADS, 4)
    z = buf[0, :, 0].copy()
    for q in range(rows):
        for j in range(4):
            if q or j:
                z = z + buf[q, :, j]
    v = z.reshape(TOPK_THREADS // TOPK_WAVE, TOPK_WAVE)
    lanes = np.arange(TOPK_WAVE)
    off = TOPK_WAVE // 2
    while off >= 1:
        v = v + v[:, lanes ^ off]
        off //= 2
    total = v[0, 0]
    for w in range(1, v.shape[0]):
        total = np.float32(total + v[w, 0])
    return np.float32(total)


def weight_image(x) -> np.ndarray | None:
    """fp32 softmax weights of one logits row as the top-k ranks them, or ``None`` when the
    row holds a NaN or +inf (or only -inf): torch's fp32 softmax is NaN throughout then,
    and the kernels rank the scores themselves (ties to the lower index, -inf as -FLT_MAX)."""
    x = np.asarray(x, np.float32)
    if x.size == 0 or np.isnan(x).any() or np.isposinf(x).any() or not np.isfinite(x.max()):
        return None
    m = x.max()
    e = softmax_exp32(x - m)
    inv = np.float32(np.float32(1.0) / weight_sum_fixed(e))
    return e * inv


def score_order_key(x) -> np.ndarray:
    """Ranking key of a row without finite weights (topk.hip ``score_key``): the float's
    order-preserving unsigned image (``-0.0`` folded into ``+0.0`` by adding ``+0.0``;
    NaN keeps its sign), floored at the image of ``-FLT_MAX``."""
    u = (np.asarray(x, np.float32) + np.float32(0.0)).view(np.uint32)
    key = np.where((u & np.uint32(0x80000000)) != 0, ~u, u | np.uint32(0x80000000))
    return np.maximum(key, np.uint32(0x00800000))


def decode_topk(logits, fraction: float, kpad: int | None = None) -> DecodeSelection:
    """Loop-2 key selection of ``FlashLoopEngine.decode`` (engine.py:438-498).

    ``w = softmax_fp32(logits)`` (the image of ``weight_image``); ``k = budget``; top-k of
    ``w`` with ties to the lower index -> ascending sort -> pad to a 64 multiple with a
    validity mask; ``mass = sum w_S``; ``selected_weights = w_S / mass``.  A row without
    finite weights (``weight_image`` is ``None``) is ranked by its scores and gets NaN
    mass and weights.  ``logits``: ``[R, N]`` array or a list of 1-D arrays (ragged rows).
    """
    rows = [np.asarray(x, dtype=np.float32) for x in logits]
    counts = [decode_budget(len(x), fraction) for x in rows]
    if kpad is None:
        kpad = max(padded_capacity(c) for c in counts)
    R = len(rows)
    idx = np.zeros((R, kpad), np.int32)
    valid = np.zeros((R, kpad), bool)
    mass = np.zeros(R, np.float64)
    sw = np.zeros((R, kpad), np.float64)
    for r, x in enumerate(rows):
        k = counts[r]
        w = weight_image(x)
        if w is None:
            sel = topk_order(score_order_key(x).astype(np.int64), k)
            mass[r] = np.nan
            sw[r, :k] = np.nan
        else:
            sel = topk_order(w, k)
            mass[r] = w[sel].astype(np.float64).sum()
            sw[r, :k] = w[sel] / mass[r]
        idx[r, :k] = sel
        valid[r, :k] = True
    return DecodeSelection(idx, valid, mass, sw, np.asarray(counts))


def selected_value_aggregate(indices, valid, weights, values, v_cur, past_tokens):
    """``_selected_value_aggregate`` (engine.py:346-371): ``sum_S w_i V[i]`` where index
    ``past_tokens`` is the current token (``v_cur``).  ``values``: ``[R, T, C]`` or list."""
    out = []
    for r in range(len(indices)):
        acc = np.zeros(np.asarray(v_cur[r]).shape[-1], np.float64)
        T = past_tokens[r] if np.ndim(past_tokens) else past_tokens
        for j in np.nonzero(valid[r])[0]:
            i = int(indices[r, j])
            row = v_cur[r] if i == T else values[r][i]
            acc += float(weights[r, j]) * np.asarray(row, np.float64)
        out.append(acc)
    return np.stack(out)


def sparse_delta(q, keys, values, k_cur, v_cur, past_tokens, indices, valid, source_output, mass, scaling):
    """Cached-mass late-loop correction (flashloop/cache.py:1592-1617).

    Over the selected keys ``S`` (index ``past_tokens`` is the current token):
    ``delta = mass * (softmax_S(scaling * q.K[S]) . V[S] - source_output)``.
    """
    out = []
    for r in range(len(q)):
        T = past_tokens[r] if np.ndim(past_tokens) else past_tokens
        sel = [int(indices[r, j]) for j in np.nonzero(valid[r])[0]]
        kr = np.stack([np.asarray(k_cur[r] if i == T else keys[r][i], np.float64) for i in sel])
        vr = np.stack([np.asarray(v_cur[r] if i == T else values[r][i], np.float64) for i in sel])
        lg = (kr @ np.asarray(q[r], np.float64)) * float(scaling)
        p = _softmax64(lg)
        target = p @ vr
        out.append(float(mass[r]) * (target - np.asarray(source_output[r], np.float64)))
    return np.stack(out)


def mass_scaled_sparse_output(source_logits, target_logits, source_values, target_values, mask, mass):
    """flashloop_torch ``mass_scaled_sparse_output`` before ``o_proj`` with the
    ``cached_source_mass`` scales (attention_utils.py:216-238, attention.py:101-107):
    ``mass * softmax_S(target) V_t - mass * softmax_S(source) V_s`` for one row."""

    def subset(lg, m):
        x = np.where(m, np.asarray(lg, np.float64), -np.inf)
        p = _softmax64(x)
        return np.where(m, p, 0.0)

    ts = subset(target_logits, mask) @ np.asarray(target_values, np.float64)
    ss = subset(source_logits, mask) @ np.asarray(source_values, np.float64)
    return mass * ts - mass * ss


@dataclass
class LayerStep:
    out0: np.ndarray
    out1: np.ndarray
    logits1: object
    selection: DecodeSelection
    selected_output: np.ndarray
    delta2: np.ndarray
    delta3: np.ndarray


def decode_layer_step(qs, kcur, vcur, keys, values, scaling, fraction=0.10, sparse=True):
    """One layer of ``FlashLoopEngine.decode`` attention over all four loops
    (engine.py:422-531), before ``o_proj``.

    ``qs/kcur/vcur``: 4 arrays ``[R, C]`` (per loop); ``keys/values``: 4 arrays
    ``[R, T, C]`` (per loop: reconstructed prefix + BF16 tail).  Loops 1-2 dense; loop 2
    also selects keys; loops 3-4 return the cached-mass delta.  With ``sparse=False``
    loops 3-4 are dense too (``enable_sparse_decode=False``) and ``delta*`` hold their
    dense outputs.
    """
    out0, _ = dense_decode(qs[0], keys[0], values[0], kcur[0], vcur[0], scaling)
    out1, lg1 = dense_decode(qs[1], keys[1], values[1], kcur[1], vcur[1], scaling)
    if not sparse:
        d2, _ = dense_decode(qs[2], keys[2], values[2], kcur[2], vcur[2], scaling)
        d3, _ = dense_decode(qs[3], keys[3], values[3], kcur[3], vcur[3], scaling)
        return LayerStep(out0, out1, lg1, None, None, d2, d3)
    sel = decode_topk(lg1, fraction)
    T = [len(keys[1][r]) for r in range(len(qs[1]))]
    so = selected_value_aggregate(sel.indices, sel.valid, sel.selected_weights, values[1], vcur[1], T)
    d2 = sparse_delta(qs[2], keys[2], values[2], kcur[2], vcur[2], T, sel.indices, sel.valid, so, sel.mass, scaling)
    d3 = sparse_delta(qs[3], keys[3], values[3], kcur[3], vcur[3], T, sel.indices, sel.valid, so, sel.mass, scaling)
    return LayerStep(out0, out1, lg1, sel, so, d2, d3)
