"""Pins for the attention / selection oracle (oracle/attention.py) -- CPU only."""

import math

import numpy as np

from oracle import attention as A


def _rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


def test_dense_decode_brute_force():
    rng = np.random.default_rng(0)
    R, T, C = 3, 17, 8
    q, K, V, kc, vc = _rand(rng, R, C), _rand(rng, R, T, C), _rand(rng, R, T, C), _rand(rng, R, C), _rand(rng, R, C)
    out, lg = A.dense_decode(q, K, V, kc, vc, 0.3)
    for r in range(R):
        logits = []
        for t in range(T + 1):
            k = kc[r] if t == T else K[r, t]
            logits.append(sum(float(q[r, c]) * float(k[c]) for c in range(C)) * 0.3)
        m = max(logits)
        e = [math.exp(x - m) for x in logits]
        z = sum(e)
        for c in range(C):
            want = sum(e[t] / z * float((vc[r] if t == T else V[r, t])[c]) for t in range(T + 1))
            assert abs(out[r, c] - want) < 1e-12
        assert np.allclose(lg[r], logits, atol=1e-12)


def test_budget_and_padding():
    assert A.decode_budget(32769, 0.1) == 3277
    assert A.padded_capacity(3277) == 3328
    assert A.padded_capacity(64) == 128  # one spare block at exact multiples
    assert A.decode_budget(5, 0.1) == 1
    assert A.decode_budget(3, 1.0) == 3


def test_topk_known_answer_and_ties():
    # attention_utils.py:646-648: top-1 of each row of [[3,2,1],[1,4,2],[1,2,5]] is its diagonal
    s = np.array([[3.0, 2.0, 1.0], [1.0, 4.0, 2.0], [1.0, 2.0, 5.0]], np.float32)
    for r in range(3):
        assert list(A.topk_order(s[r], 1)) == [r]
    # ties -> lower index
    t = np.array([1.0, 5.0, 5.0, 5.0, 0.0], np.float32)
    assert list(A.topk_order(t, 2)) == [1, 2]
    # equals a brute-force stable sort on (-score, index)
    rng = np.random.default_rng(1)
    x = rng.integers(0, 6, 200).astype(np.float32)
    for k in (1, 7, 50, 200):
        want = sorted(sorted(range(200), key=lambda i: (-x[i], i))[:k])
        assert list(A.topk_order(x, k)) == want


def test_decode_topk_mass_and_weights():
    rng = np.random.default_rng(2)
    lg = _rand(rng, 4, 300) * 3
    sel = A.decode_topk(lg, 0.1)
    assert sel.indices.shape == (4, 64) and sel.count.tolist() == [30] * 4
    for r in range(4):
        w = np.exp(lg[r].astype(np.float64) - lg[r].max())
        w /= w.sum()
        k = sel.count[r]
        assert np.all(np.diff(sel.indices[r, :k]) > 0)
        assert np.all(sel.indices[r, k:] == 0) and not sel.valid[r, k:].any()
        assert abs(sel.mass[r] - w[sel.indices[r, :k]].sum()) < 1e-6  # fp32 weight image
        assert 0 < sel.mass[r] <= 1
        assert abs(sel.selected_weights[r].sum() - 1) < 1e-12
        # the selected set is the k largest weights
        assert w[sel.indices[r, :k]].min() >= np.sort(w)[-k]


def test_sparse_delta_matches_mass_scaled_sparse_output():
    """engine cached-mass delta == flashloop_torch mass_scaled_sparse_output
    (cached_source_mass: source and target scales both the loop-2 mass)."""
    rng = np.random.default_rng(3)
    R, T, C = 2, 40, 16
    keys = [_rand(rng, R, T, C) for _ in range(4)]
    vals = [_rand(rng, R, T, C) for _ in range(4)]
    qs = [_rand(rng, R, C) for _ in range(4)]
    kc = [_rand(rng, R, C) for _ in range(4)]
    vc = [_rand(rng, R, C) for _ in range(4)]
    step = A.decode_layer_step(qs, kc, vc, keys, vals, 0.25, fraction=0.3)
    for r in range(R):
        mask = np.zeros(T + 1, bool)
        mask[step.selection.indices[r, step.selection.valid[r]]] = True
        src_lg = step.logits1[r]
        for loop, delta in ((2, step.delta2), (3, step.delta3)):
            Kt = np.concatenate([keys[loop][r], kc[loop][r][None]])
            Vt = np.concatenate([vals[loop][r], vc[loop][r][None]])
            tgt_lg = (Kt.astype(np.float64) @ qs[loop][r].astype(np.float64)) * 0.25
            Vs = np.concatenate([vals[1][r], vc[1][r][None]])
            want = A.mass_scaled_sparse_output(src_lg, tgt_lg, Vs, Vt, mask, step.selection.mass[r])
            assert np.allclose(delta[r], want, atol=1e-12)


def test_full_fraction_sparse_equals_dense():
    """With fraction 1, loop-2 output + delta equals the dense loop-3/4 output."""
    rng = np.random.default_rng(4)
    R, T, C = 2, 30, 8
    keys = [_rand(rng, R, T, C) for _ in range(4)]
    vals = [_rand(rng, R, T, C) for _ in range(4)]
    qs = [_rand(rng, R, C) for _ in range(4)]
    kc = [_rand(rng, R, C) for _ in range(4)]
    vc = [_rand(rng, R, C) for _ in range(4)]
    sp = A.decode_layer_step(qs, kc, vc, keys, vals, 0.5, fraction=1.0)
    dn = A.decode_layer_step(qs, kc, vc, keys, vals, 0.5, sparse=False)
    assert np.allclose(sp.selected_output, sp.out1, atol=1e-12)
    assert np.allclose(sp.out1 + sp.delta2, dn.delta2, atol=1e-12)
    assert np.allclose(sp.out1 + sp.delta3, dn.delta3, atol=1e-12)
