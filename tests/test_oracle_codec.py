"""Pins for the numpy codec oracle (oracle/codec.py) -- CPU only.

Each test is chosen so that a plausible restatement mistake (mean instead of min,
round-half-up, fused multiply-add, wrong reduction axis, dropped bf16 rounding, a
mask applied to the wrong loop) fails at least one of them.
"""

import numpy as np
import pytest

from oracle import codec

F32 = np.float32


def _bf16(x):
    return codec.bf16_round(np.asarray(x, F32))


def test_bf16_round_known_values():
    # 1 + 2^-8 is half-way between 1 and 1 + 2^-7: ties to even -> 1
    assert codec.bf16_round(np.array([1 + 2**-8], F32))[0] == 1.0
    # 1 + 3*2^-8 is half-way between 1+2^-7 and 1+2^-6: ties to even -> 1 + 2^-6
    assert codec.bf16_round(np.array([1 + 3 * 2**-8], F32))[0] == F32(1 + 2**-6)
    # just above half-way rounds up
    assert codec.bf16_round(np.array([1 + 2**-8 + 2**-20], F32))[0] == F32(1 + 2**-7)
    assert codec.bf16_round(np.array([-3.0], F32))[0] == -3.0
    assert np.isinf(codec.bf16_round(np.array([3.4e38], F32))[0])


def test_constant_group_scale_one_codes_zero():
    x = np.full((1, 1, 64, 128), 0.75, F32)
    fq, _ = codec.quantize_k_per_channel(x)
    assert np.all(fq.scale == 1.0) and np.all(fq.minimum == 0.75)
    assert np.all(fq.codes == 0) and np.all(fq.recon == 0.75)


def test_zero_minimum_is_positive_zero():
    """A group whose smallest value is a zero stores +0 as its minimum, whether its
    zeros are +0, -0 or a mix (numpy's and torch's min over a mix return either);
    codes and reconstructions are those of a +0 minimum, and no reconstruction is -0."""
    x = np.zeros((1, 1, 64, 128), F32)
    x[0, 0, :, 0] = -0.0  # all -0
    x[0, 0, ::2, 1] = -0.0  # mixed
    x[0, 0, 1::3, 2] = -0.0
    x[0, 0, 5, 2] = 2.0  # mixed zeros with one non-zero above them
    x[0, 0, :, 3] = -0.0
    x[0, 0, 7, 3] = -1.0  # a negative minimum keeps its value
    fq, _ = codec.quantize_k_per_channel(x)
    mn = fq.minimum.reshape(-1)
    assert mn[3] == -1.0
    zero = mn == 0
    assert zero[[0, 1, 2]].all() and not np.signbit(mn[zero]).any()
    assert fq.scale.reshape(-1)[2] == F32(2.0) / F32(15)
    assert fq.codes[0, 0, 5, 2] == 15 and fq.codes[0, 0, :5, 2].max() == 0
    assert not np.signbit(fq.recon[fq.recon == 0]).any()
    v = codec.quantize_v_per_token(np.where(np.arange(128) % 3 == 0, F32(-0.0), F32(0.0))[None, None, None, :]
                                   * np.ones((1, 1, 4, 1), F32))
    assert np.all(v.minimum == 0) and not np.signbit(v.minimum).any()


def test_ramp_gives_codes_j():
    # per-channel ramp over 16 tokens repeated: min=-1, step 0.125 -> span 1.875, scale 0.125
    j = np.arange(64) % 16
    x = (-1.0 + 0.125 * j).astype(F32)[None, None, :, None].repeat(128, axis=3)
    fq, _ = codec.quantize_k_per_channel(x)
    assert np.all(fq.scale == F32(1.875) / F32(15))
    assert np.array_equal(fq.codes[0, 0, :, 0], j.astype(np.uint8))
    assert np.array_equal(fq.recon, _bf16(x))


def test_round_half_even_and_clamp():
    # V group over 64 channels: min 0, max 15 -> scale 1; values n + 0.5 round to even
    row = np.zeros(64, F32)
    row[0], row[1] = 0.0, 15.0
    row[2:6] = [0.5, 1.5, 2.5, 13.5]
    x = np.concatenate([row, row])[None, None, None, :]
    fq = codec.quantize_v_per_token(x)
    assert fq.scale[0, 0, 0, 0] == 1.0
    assert list(fq.codes[0, 0, 0, 2:6]) == [0, 2, 2, 14]
    assert fq.codes.max() == 15 and fq.codes.min() == 0


def test_k_reduces_over_tokens_v_over_channels():
    rng = np.random.default_rng(0)
    x = _bf16(rng.standard_normal((2, 3, 128, 128)))
    fk, _ = codec.quantize_k_per_channel(x)
    fv = codec.quantize_v_per_token(x)
    g = x.reshape(2, 3, 2, 64, 128)
    assert np.array_equal(fk.minimum, g.min(axis=3))
    assert np.array_equal(fv.minimum, x.reshape(2, 3, 128, 2, 64).min(axis=4))
    # error bound |x - recon| <= scale/2 + one bf16 rounding of recon
    for fq, scale in ((fk, np.repeat(fk.scale, 64, axis=2)), (fv, np.repeat(fv.scale, 64, axis=3))):
        err = np.abs(x - fq.recon)
        assert np.all(err <= scale * 0.5 + np.abs(fq.recon) * 2**-8 + 1e-7)


def test_reconstruction_is_mul_then_add_not_fma():
    # pick a case where fma(code, scale, min) != (code*scale)+min in float32
    rng = np.random.default_rng(1)
    hits = 0
    for _ in range(200):
        x = _bf16(rng.standard_normal((1, 1, 64, 128)) * 3)
        fq, _ = codec.quantize_k_per_channel(x)
        code = fq.codes.astype(np.float64)
        s = np.repeat(fq.scale, 64, axis=2).astype(np.float64)
        m = np.repeat(fq.minimum, 64, axis=2).astype(np.float64)
        fused = codec.bf16_round((code * s + m).astype(F32))  # one rounding to f32
        two = codec.bf16_round((code.astype(F32) * s.astype(F32)).astype(F32) + m.astype(F32))
        assert np.array_equal(fq.recon, two)
        hits += int(np.any(fused != two))
        if hits:
            break
    assert hits, "no sample distinguishes fma from mul+add; widen the search"


def _literal_active_delta(delta, mask, axis):
    """Literal restatement of ``_quantize_active_delta`` (kv_quantization.py:455-486):
    compact the active rows, chunk by 64, quantize, scatter back."""
    out = np.zeros_like(delta)
    for b in range(delta.shape[0]):
        pos = np.nonzero(mask[b])[0]
        if pos.size == 0:
            continue
        sel = delta[b : b + 1][:, :, pos, :]
        if axis == "k":
            chunks = []
            for s in range(0, sel.shape[2], 64):
                part = sel[:, :, s : s + 64, :]
                mn = part.min(axis=2, keepdims=True)
                mx = part.max(axis=2, keepdims=True)
                span = mx - mn
                sc = np.where(span > 0, span / F32(15), F32(1)).astype(F32)
                q = np.clip(np.rint((part - mn) / sc), 0, 15).astype(F32)
                chunks.append(codec.bf16_round(q * sc + mn))
            rec = np.concatenate(chunks, axis=2)
        else:
            rec = codec.quantize_v_per_token(sel).recon
        out[b : b + 1][:, :, pos, :] = rec
    return out


@pytest.mark.parametrize("axis", ["k", "v"])
def test_masked_delta_equals_literal_compaction(axis):
    rng = np.random.default_rng(2)
    d = _bf16(rng.standard_normal((2, 2, 64, 128)) * 0.1)
    mask = rng.random((2, 64)) < 0.3
    mask[1] = False  # an empty row
    if axis == "k":
        got, _ = codec.quantize_k_per_channel(d, mask)
    else:
        got = codec.quantize_v_per_token(d, mask)
    want = _literal_active_delta(d, mask, axis)
    assert np.array_equal(got.recon, want)
    assert np.all(got.codes[1] == 0)


def test_chain_invariants():
    rng = np.random.default_rng(3)
    b, h, t, c = 1, 2, 128, 128
    l1 = _bf16(rng.standard_normal((b, h, t, c)))
    ks = [l1]
    for _ in range(3):
        ks.append(_bf16(ks[-1] + 0.1 * rng.standard_normal((b, h, t, c))))
    vs = [_bf16(k[:, ::-1]) for k in ks]
    m3 = rng.random((b, t)) < 0.25
    m3[:, -1] = True
    m4 = m3 & (rng.random((b, t)) < 0.4)
    res = codec.encode_temporal_groups(ks, vs, [None, m3, m4])
    # loop-2 deltas are dense; loop-3/4 reconstructions equal the previous loop at inactive rows
    r2, r3, r4 = res.recon_keys[1:]
    assert np.array_equal(r3[:, :, ~m3[0]], r2[:, :, ~m3[0]])
    assert np.array_equal(r4[:, :, ~m4[0]], r3[:, :, ~m4[0]])
    # each loop reconstruction is closer to its target than the previous loop's
    for r in range(1, 4):
        e_prev = np.abs(ks[r] - res.recon_keys[r - 1])
        e_new = np.abs(ks[r] - res.recon_keys[r])
        act = np.ones((b, t), bool) if r == 1 else (m3 if r == 2 else m4)
        sel = act[0]
        assert e_new[:, :, sel].mean() < e_prev[:, :, sel].mean()
    # residual codes really are residual: stream r decodes to recon_r - recon_{r-1} (bf16)
    s1 = res.streams[1]
    dec = codec.bf16_round(
        np.repeat(s1.k_scale, 64, axis=2) * s1.k_codes.astype(F32) + np.repeat(s1.k_min, 64, axis=2)
    )
    assert np.array_equal(codec.bf16_add(res.recon_keys[0], dec), res.recon_keys[1])


def test_packed_prefix_and_transition_masks():
    assert codec.packed_prefix_tokens(2048) == 1984
    assert codec.packed_prefix_tokens(8192) == 8128
    assert codec.packed_prefix_tokens(32768) == 32704
    assert codec.packed_prefix_tokens(127) == 0
    assert codec.packed_prefix_tokens(128) == 64
    m3 = np.zeros((1, 100), bool)
    m3[0, 70] = True
    m4 = np.zeros((1, 100), bool)
    masks = codec.transition_masks(1, 64, 128, (m3, m4))
    assert masks[0].all()
    assert masks[1][0, 6] and masks[1][0, :36].sum() == 1 and masks[1][0, 36:].all()
    assert masks[2][0, :36].sum() == 0 and masks[2][0, 36:].all()
