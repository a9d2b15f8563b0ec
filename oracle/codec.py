"""int4 asymmetric min/max codec and the cross-loop residual chain, restated in numpy.

Test infrastructure: the checker for ``fl_pack_kv_group`` (flashloop_amd/csrc/pack.hip).

All arithmetic is float32 with one IEEE rounding per operation, exactly as the
reference's eager torch-CPU ops perform it:

* ``work = values.float()``; ``amin``/``amax`` over the group (exact: inputs are bf16);
* ``span = max - min``; ``scale = span / 15`` when ``span > 0`` else ``1``;
* ``code = round_half_even((work - min) / scale)`` clamped to ``[0, 15]``;
* ``recon = bf16(code * scale + min)`` -- a float32 multiply, then a float32 add
  (two roundings, never a fused multiply-add), then round-to-nearest-even to bf16.

bf16 tensors are carried as float32 arrays whose values are exactly representable
in bf16.  bf16 ``a - b`` and ``a + b`` are computed as float32 then rounded to bf16,
which is what torch's CPU bf16 binary ops do.

Pinned by (tests/test_oracle_codec.py): closed forms (constant group -> scale 1,
codes 0; ramps -> codes j; half-way values -> half-even; clamping), a literal
per-group compaction loop for masked deltas (``_quantize_active_delta``
semantics), the chain invariants of ``encode_temporal_group`` (inactive rows
carry the previous loop exactly), and reconstruction error bounds
(|x - recon| <= scale/2 + bf16 rounding).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

GROUP = 64
LEVELS = np.float32(15.0)
F32 = np.float32


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bf16 value (ties to even), returned as float32.

    Matches ``tensor.to(torch.bfloat16)`` for finite values and infinities.
    """
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    out = r.view(F32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.float32("nan")
    return out


def bf16_sub(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """bf16 ``a - b`` as torch CPU computes it (float32 op, then RNE to bf16)."""
    return bf16_round(a.astype(F32) - b.astype(F32))


def bf16_add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return bf16_round(a.astype(F32) + b.astype(F32))


@dataclass
class FakeQuant:
    codes: np.ndarray  # uint8, same shape as the input
    scale: np.ndarray  # float32, keepdims along the reduced axis
    minimum: np.ndarray  # float32, keepdims along the reduced axis
    recon: np.ndarray  # float32 holding bf16 values


def asymmetric_fake_quant(values: np.ndarray, axis: int, active: np.ndarray | None = None) -> FakeQuant:
    """``_asymmetric_fake_quant`` (flashloop_torch/kv_quantization.py:395-414), 4 bits.

    ``active`` (broadcastable to ``values``) restricts the min/max to active entries;
    inactive entries get code 0 and reconstruction 0.  A reduction with no active
    entry gets the convention scale 1, min 0 (the reference skips such groups,
    kv_quantization.py:468-469, so they carry no metadata).
    """
    work = np.asarray(values, dtype=F32)
    if active is None:
        mn = work.min(axis=axis, keepdims=True)
        mx = work.max(axis=axis, keepdims=True)
        any_active = None
    else:
        act = np.broadcast_to(active, work.shape)
        mn = np.where(act, work, np.float32(np.inf)).min(axis=axis, keepdims=True)
        mx = np.where(act, work, np.float32(-np.inf)).max(axis=axis, keepdims=True)
        any_active = act.any(axis=axis, keepdims=True)
        mn = np.where(any_active, mn, F32(0.0)).astype(F32)
        mx = np.where(any_active, mx, F32(0.0)).astype(F32)
    # A zero minimum is stored as +0 (-0 + 0 = +0): torch's amin returns either zero
    # over a mix of +0 and -0, depending on its evaluation order.  The codes and the
    # reconstruction do not depend on that sign.
    mn = (mn + F32(0.0)).astype(F32)
    span = (mx - mn).astype(F32)
    scale = np.where(span > 0, span / LEVELS, F32(1.0)).astype(F32)
    q = np.rint((work - mn) / scale).astype(F32)  # np.rint: round half to even
    q = np.clip(q, F32(0.0), LEVELS)
    recon = bf16_round((q * scale).astype(F32) + mn)
    codes = q.astype(np.uint8)
    if active is not None:
        act = np.broadcast_to(active, work.shape)
        codes = np.where(act, codes, np.uint8(0)).astype(np.uint8)
        recon = np.where(act, recon, F32(0.0)).astype(F32)
    return FakeQuant(codes=codes, scale=scale, minimum=mn, recon=recon)


@dataclass
class StreamCodes:
    """Layout-neutral codes and metadata of one packed stream (one loop).

    ``k_codes``/``v_codes``: uint8 ``[B, H, T, C]`` (0 at inactive rows);
    ``k_scale``/``k_min``: float32 ``[B, H, T/64, C]`` (per channel, per 64-token group);
    ``v_scale``/``v_min``: float32 ``[B, H, T, C/64]`` (per token, per 64-channel group);
    ``active``: bool ``[B, T]`` rows this stream stores.
    """

    k_codes: np.ndarray
    k_scale: np.ndarray
    k_min: np.ndarray
    v_codes: np.ndarray
    v_scale: np.ndarray
    v_min: np.ndarray
    active: np.ndarray


def quantize_k_per_channel(x: np.ndarray, active: np.ndarray | None = None) -> tuple[FakeQuant, np.ndarray]:
    """``quantize_dequantize_k_per_channel`` (kv_quantization.py:417-433) over whole groups.

    ``x``: ``[B, H, T, C]`` with ``T % 64 == 0``; ``active``: ``[B, T]`` or None.
    Returns the fake-quant result (codes/recon ``[B,H,T,C]``) and meta ``[B,H,T/64,C]``.
    With a mask, the min/max of each group runs over its active rows only, which is
    what compacting a <=64-row temporal group and quantizing it does
    (``_quantize_active_delta``, kv_quantization.py:455-486).
    """
    b, h, t, c = x.shape
    assert t % GROUP == 0
    g = t // GROUP
    xr = x.reshape(b, h, g, GROUP, c)
    act = None
    if active is not None:
        act = active.reshape(b, 1, g, GROUP, 1)
    fq = asymmetric_fake_quant(xr, axis=3, active=act)
    return (
        FakeQuant(
            codes=fq.codes.reshape(b, h, t, c),
            scale=fq.scale.reshape(b, h, g, c),
            minimum=fq.minimum.reshape(b, h, g, c),
            recon=fq.recon.reshape(b, h, t, c),
        ),
        fq.scale.reshape(b, h, g, c),
    )


def quantize_v_per_token(x: np.ndarray, active: np.ndarray | None = None) -> FakeQuant:
    """``quantize_dequantize_v_per_token`` (kv_quantization.py:436-452): 64-channel groups.

    ``x``: ``[B, H, T, C]`` with ``C % 64 == 0``.  Meta shape ``[B, H, T, C/64]``.
    """
    b, h, t, c = x.shape
    assert c % GROUP == 0
    gc = c // GROUP
    xr = x.reshape(b, h, t, gc, GROUP)
    act = None
    if active is not None:
        act = active.reshape(b, 1, t, 1, 1)
    fq = asymmetric_fake_quant(xr, axis=4, active=act)
    return FakeQuant(
        codes=fq.codes.reshape(b, h, t, c),
        scale=fq.scale.reshape(b, h, t, gc),
        minimum=fq.minimum.reshape(b, h, t, gc),
        recon=fq.recon.reshape(b, h, t, c),
    )


@dataclass
class ChainResult:
    recon_keys: list[np.ndarray]  # per loop, bf16-valued float32 [B,H,T,C]
    recon_values: list[np.ndarray]
    streams: list[StreamCodes]


def encode_temporal_groups(
    keys: list[np.ndarray],
    values: list[np.ndarray],
    masks: list[np.ndarray | None] | None = None,
) -> ChainResult:
    """``encode_temporal_group`` (kv_quantization.py:531-650), profile ``kivi4_channel``.

    Applied to every 64-token group of ``[B, H, T, C]`` at once (the groups are
    independent).  ``R_1 = fq(L_1)``; ``R_r = R_{r-1} + fq_masked(L_r - R_{r-1})`` with
    all additions and subtractions in bf16.  ``masks[r-1]`` (``[B, T]`` bool or None
    for all-active) selects the rows whose loop-(r) delta is stored
    (kv_quantization.py:580-602).  K: per-channel over tokens; V: per-token over
    64-channel groups (kv_quantization.py:40-45).
    """
    loops = len(keys)
    assert 1 <= loops <= 4 and len(values) == loops
    b, h, t, c = keys[0].shape
    if masks is None:
        masks = [None] * (loops - 1)
    assert len(masks) == loops - 1
    rk: list[np.ndarray] = []
    rv: list[np.ndarray] = []
    streams: list[StreamCodes] = []
    for r in range(loops):
        if r == 0:
            xk = bf16_round(keys[0])
            xv = bf16_round(values[0])
            m = None
        else:
            xk = bf16_sub(keys[r], rk[-1])
            xv = bf16_sub(values[r], rv[-1])
            m = masks[r - 1]
        fk, _ = quantize_k_per_channel(xk, m)
        fv = quantize_v_per_token(xv, m)
        if r == 0:
            rk.append(fk.recon)
            rv.append(fv.recon)
        else:
            # inactive rows get an exact zero delta; bf16(R + 0) == R except -0 -> +0
            rk.append(bf16_add(rk[-1], fk.recon))
            rv.append(bf16_add(rv[-1], fv.recon))
        act = np.ones((b, t), dtype=bool) if m is None else m.astype(bool)
        streams.append(
            StreamCodes(
                k_codes=fk.codes,
                k_scale=fk.scale,
                k_min=fk.minimum,
                v_codes=fv.codes,
                v_scale=fv.scale,
                v_min=fv.minimum,
                active=act,
            )
        )
    return ChainResult(recon_keys=rk, recon_values=rv, streams=streams)


def packed_prefix_tokens(tokens: int, group: int = GROUP, residual: int = 64) -> int:
    """Tokens held in packed streams; the rest stay in the BF16 tail.

    ``compress_available`` encodes ``[s, s+64)`` while ``T - s >= residual + group``
    (kv_quantization.py:215); the engine uses the same count (cache.py:385-387).
    """
    return max(0, ((tokens - residual) // group) * group)


def transition_masks(batch: int, start: int, stop: int, prefill_masks: tuple[np.ndarray, np.ndarray] | None, loops: int = 4):
    """``_transition_masks`` (kv_quantization.py:171-196): loop-1->2 is always dense,
    loops 3/4 use the prefill masks over the prompt and are dense beyond it."""
    width = stop - start
    masks = [np.ones((batch, width), dtype=bool) for _ in range(loops - 1)]
    if prefill_masks is not None:
        for ti, src in enumerate(prefill_masks, start=1):
            if ti >= len(masks):
                break
            ov = min(stop, src.shape[1])
            if ov > start:
                masks[ti][:, : ov - start] = src[:, start:ov]
    return masks


def compress_prefix(
    keys: list[np.ndarray],
    values: list[np.ndarray],
    prefill_masks: tuple[np.ndarray, np.ndarray] | None = None,
    residual: int = 64,
) -> tuple[ChainResult, int]:
    """``CrossLoopKVCacheCompressor.compress_available`` (kv_quantization.py:198-244).

    Encodes every complete group that has left the ``residual``-token BF16 tail.
    Returns the chain result over the packed prefix and its length ``Tp``.
    """
    b, h, t, c = keys[0].shape
    tp = packed_prefix_tokens(t, GROUP, residual)
    masks = transition_masks(b, 0, tp, prefill_masks, loops=len(keys))
    res = encode_temporal_groups(
        [k[:, :, :tp] for k in keys],
        [v[:, :, :tp] for v in values],
        [m for m in masks],
    )
    return res, tp


def materialize_loop_cache(keys: list[np.ndarray], values: list[np.ndarray], chain: ChainResult, tp: int):
    """The K_r/V_r every loop attends to: reconstructed prefix, raw BF16 tail
    (the in-place overwrite at kv_quantization.py:233-239)."""
    ks, vs = [], []
    for r in range(len(keys)):
        k = bf16_round(keys[r]).copy()
        v = bf16_round(values[r]).copy()
        k[:, :, :tp] = chain.recon_keys[r]
        v[:, :, :tp] = chain.recon_values[r]
        ks.append(k)
        vs.append(v)
    return ks, vs
