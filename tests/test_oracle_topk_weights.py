"""Pins for the fp32 softmax weight image that the decode selection ranks
(oracle/attention.py ``fma32``, ``softmax_exp32``, ``weight_sum_fixed``, ``weight_image``,
``decode_topk``) -- CPU only.

The reference ranks ``torch.softmax(logits, dtype=float32)`` with ``torch.topk``
(flashloop/engine.py:439-453, flashloop/selection.py:85); the workload fixes ties to the
lower index.  The last tests count, on cfg3-shaped rows (32,769 keys), the rows where
ranking the logits and ranking the weight image each differ from ranking torch's own fp32
softmax weights on this CPU.
"""

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import attention as A


def _round_f32(q: Fraction) -> np.float32:
    """Round-to-nearest-even of an exact rational to float32 (subnormals included)."""
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    e = max(e, -126)  # subnormals share the exponent of the smallest normal
    scale = Fraction(2) ** (23 - e)
    m = q * scale
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return np.float32(sign * math.ldexp(fl, e - 23))


def test_fma32_is_correctly_rounded():
    rng = np.random.default_rng(0)
    n = 4000
    a = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 2.0 ** rng.integers(-20, 20, n)).astype(np.float32)
    c = -(a.astype(np.float64) * b).astype(np.float32)  # cancellation: the residual decides
    c[: n // 2] = (rng.standard_normal(n // 2) * 2.0 ** rng.integers(-30, 30, n // 2)).astype(np.float32)
    # results in the subnormal range
    a[:200] = np.float32(2.0 ** -70)
    b[:200] = (rng.random(200) * 2.0 ** -60).astype(np.float32)
    c[:200] = (rng.random(200) * 2.0 ** -130).astype(np.float32)
    got = A.fma32(a, b, c)
    for i in range(n):
        want = _round_f32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i].view(np.uint32) == want.view(np.uint32) or (got[i] == 0 and want == 0), (i, a[i], b[i], c[i])
    # an exact half-way case that float64 double rounding gets wrong: 1 + 2^-24 + 2^-60
    x = A.fma32(np.float32(1.0 + 2.0 ** -23), np.float32(1.0 + 2.0 ** -23), np.float32(-(2.0 ** -23)))
    want = _round_f32(Fraction(1 + Fraction(1, 2 ** 23)) ** 2 - Fraction(1, 2 ** 23))
    assert x.view(np.uint32) == want.view(np.uint32)


def _ulp32(y: np.ndarray) -> np.ndarray:
    y = np.abs(y).astype(np.float32)
    return np.maximum(np.spacing(y).astype(np.float64), 2.0 ** -149)


def test_softmax_exp_accuracy_and_special_values():
    rng = np.random.default_rng(1)
    d = np.concatenate([
        -rng.random(1_000_000).astype(np.float32) * 120.0,
        -rng.random(200_000).astype(np.float32) * 1.0,
        -(2.0 ** -rng.integers(1, 40, 50_000) * rng.random(50_000)).astype(np.float32),
        np.linspace(-104.5, -86.0, 100_000, dtype=np.float32),  # subnormal range
    ])
    got = A.softmax_exp32(d).astype(np.float64)
    want = np.exp(d.astype(np.float64))
    err = np.abs(got - want) / _ulp32(want)
    assert err.max() <= 2.0, f"max error {err.max():.3f} ulp"
    assert np.mean(err) < 0.3
    assert A.softmax_exp32(np.float32(0.0)) == np.float32(1.0)
    assert A.softmax_exp32(np.float32(-np.inf)) == 0.0
    assert np.all(A.softmax_exp32(np.linspace(-200, -104.0, 1000, dtype=np.float32)) == 0.0)
    # the smallest subnormal appears where exp(d) crosses 2^-150
    edge = np.float32(math.log(2.0 ** -149))
    assert A.softmax_exp32(edge) == np.float32(2.0 ** -149)


def test_weight_sum_order_is_the_kernels():
    """The vectorised fixed-order sum equals the literal per-thread / per-wave loops."""
    rng = np.random.default_rng(2)
    for n in (1, 63, 1024, 3000, 5000, 9001):
        e = (rng.random(n) * 3).astype(np.float32)
        threads = [np.float32(0.0)] * 1024
        for t in range(1024):
            acc = np.float32(0.0)
            base = 4 * t
            while base < n:
                for i in range(base, min(base + 4, n)):
                    acc = np.float32(acc + e[i])
                base += 4096
            threads[t] = acc
        waves = []
        for w in range(16):
            v = [threads[w * 64 + l] for l in range(64)]
            off = 32
            while off >= 1:
                v = [np.float32(v[l] + v[l ^ off]) for l in range(64)]
                off //= 2
            waves.append(v[0])
        total = waves[0]
        for w in range(1, 16):
            total = np.float32(total + waves[w])
        assert A.weight_sum_fixed(e).view(np.uint32) == np.float32(total).view(np.uint32)
        assert abs(float(total) - float(e.astype(np.float64).sum())) <= 1e-6 * max(1.0, float(total))


def test_weight_image_matches_softmax():
    rng = np.random.default_rng(3)
    for scale in (1.0, 8.0, 40.0):
        x = (rng.standard_normal(20000) * scale).astype(np.float32)
        w = A.weight_image(x).astype(np.float64)
        d = (x - x.max()).astype(np.float64)  # RN(x - max) in fp32, as torch forms it too
        ref = np.exp(d)
        ref /= ref.sum()
        normal = ref >= 2.0 ** -126
        rel = np.abs(w[normal] - ref[normal]) / ref[normal]
        assert rel.max() < 8 * 2.0 ** -24
        assert np.all(np.abs(w[~normal] - ref[~normal]) <= 2.0 ** -148)
    assert A.weight_image(np.array([1.0, np.nan], np.float32)) is None
    assert A.weight_image(np.array([1.0, np.inf], np.float32)) is None
    assert A.weight_image(np.array([-np.inf, -np.inf], np.float32)) is None
    w = A.weight_image(np.array([0.0, -np.inf, 0.0], np.float32))
    assert w[1] == 0.0 and w[0] == w[2] == np.float32(0.5)


def test_decode_topk_ranks_weights_not_logits():
    """Distinct logits whose weights underflow to one value tie at the lower index."""
    x = np.array([0.0, -200.0, -150.0, -120.0, -1.0], np.float32)  # weights 1, 0, 0, 0, e^-1
    sel = A.decode_topk([x], 0.6)  # k = 3
    assert list(sel.indices[0, :3]) == [0, 1, 4]  # index 1 wins the 0-weight tie
    assert list(A.topk_order(x, 3)) == [0, 3, 4]  # the logit order would take index 3


def _torch_rank(x: np.ndarray, k: int) -> np.ndarray:
    """torch's fp32 softmax on this CPU, ranked with ties to the lower index."""
    w = torch.softmax(torch.from_numpy(x), dim=-1, dtype=torch.float32).numpy()
    return A.topk_order(w, k)


def _count_differences(x: np.ndarray, frac: float = 0.1):
    k = A.decode_budget(x.shape[-1], frac)
    sel = A.decode_topk(x, frac)
    d_image = d_logit = 0
    for r in range(x.shape[0]):
        ref = _torch_rank(x[r], k)
        d_image += not np.array_equal(sel.indices[r, :k], ref)
        d_logit += not np.array_equal(A.topk_order(x[r], k), ref)
    return d_image, d_logit


@pytest.mark.parametrize("scale,logit_rows", [(1.0, 0), (16.0, 0), (64.0, 32)])
def test_selection_matches_torch_fp32_softmax_ranking(scale, logit_rows):
    """cfg3-shaped rows (32 of them, 32,769 keys, budget 3,277).  At scale 64 (peaked
    rows: most weights underflow) ranking the logits picks a different set in every row,
    ranking the weight image matches torch's fp32 softmax ranking in every row."""
    rng = np.random.default_rng(int(scale))
    x = (rng.standard_normal((32, 32769)) * scale).astype(np.float32)
    d_image, d_logit = _count_differences(x)
    assert d_image == 0
    assert d_logit == logit_rows


def test_selection_matches_torch_on_the_golden_fixture():
    import os

    f = dict(np.load(os.path.join(os.path.dirname(__file__), "golden", "decode_small.npz"), allow_pickle=False))
    d_image, d_logit = _count_differences(np.asarray(f["logits1"], np.float32), float(f["fraction"]))
    assert d_image == 0 and d_logit == 0
