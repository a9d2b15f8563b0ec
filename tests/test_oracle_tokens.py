"""Pins for the token-sparse update oracle (oracle/tokens.py) -- CPU only."""

import math

import numpy as np
import pytest

from oracle import tokens as OT


def test_hidden_delta_score_closed_forms():
    cur = np.array([[[3.0, 4.0], [1.0, 0.0], [0.0, 0.0]]], np.float32)
    prev = np.array([[[0.0, 0.0], [1.0, 0.0], [1.0, 0.0]]], np.float32)
    s = OT.hidden_delta_score(cur, prev)
    assert s[0, 0] == pytest.approx(1.0)  # ||h|| / ||h||
    assert s[0, 1] == 0.0  # unchanged row
    assert s[0, 2] == pytest.approx(1.0 / 1e-12)  # zero current row: clamped denominator


def test_select_active_mask_budget_nesting_forced_last():
    rng = np.random.default_rng(0)
    scores = rng.random((3, 101)).astype(np.float32)
    m3 = OT.select_active_mask(scores, 0.25)
    assert np.all(m3.sum(1) == math.ceil(101 * 0.25))
    assert np.all(m3[:, -1])
    m4 = OT.select_active_mask(scores * 2, 0.10, eligible=m3)
    assert np.all(m4.sum(1) == math.ceil(101 * 0.10))
    assert np.all(~m4 | m3) and np.all(m4[:, -1])
    # brute force: the selected non-forced rows are the top-scoring eligible candidates
    for b in range(3):
        cand = [i for i in range(100) if m3[b, i]]
        want = sorted(sorted(cand, key=lambda i: (-scores[b, i] * 2, i))[: math.ceil(101 * 0.10) - 1])
        assert list(np.nonzero(m4[b, :100])[0]) == want


def test_select_active_mask_small_and_errors():
    s = np.array([[5.0, 1.0, 3.0]], np.float32)
    assert OT.select_active_mask(s, 0.01).tolist() == [[False, False, True]]  # budget 1 = forced last
    assert OT.select_active_mask(s, 1.0).tolist() == [[True, True, True]]
    with pytest.raises(ValueError):
        OT.select_active_mask(s, 0.5, eligible=np.array([[True, True, False]]))
    with pytest.raises(ValueError):
        OT.select_active_mask(s, 0.5, eligible=np.zeros((1, 3), bool), force_last_token=False)


def test_gather_scatter_round_trip_and_identity():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 4, 50, 8)).astype(np.float32)
    pos = np.sort(rng.choice(50, 13, replace=False))
    g = OT.gather_rows(x, pos, axis=2)
    assert g.shape == (2, 4, 13, 8) and np.array_equal(g[:, :, 3], x[:, :, pos[3]])
    y = OT.scatter_rows(np.zeros_like(x), pos, g, axis=2)
    assert np.array_equal(y[:, :, pos], x[:, :, pos])
    rest = np.setdiff1d(np.arange(50), pos)
    assert np.all(y[:, :, rest] == 0)
    ident = np.arange(50)
    assert np.array_equal(OT.gather_rows(x, ident, 2), x)
    assert np.array_equal(OT.scatter_rows(np.zeros_like(x), ident, x, 2), x)


def test_carry_and_replace_frozen():
    prev = np.zeros((1, 4, 3), np.float32)
    comp = np.ones((1, 4, 3), np.float32)
    act = np.array([[True, False, True, False]])
    out = OT.carry_frozen_hidden(prev, comp, act)
    assert out[0, :, 0].tolist() == [1, 0, 1, 0]
    kv_prev = np.zeros((1, 2, 4, 3), np.float32)
    kv_cur = np.ones((1, 2, 4, 3), np.float32)
    out = OT.replace_frozen_cache(kv_prev, kv_cur, act)
    assert out[0, 1, :, 2].tolist() == [1, 0, 1, 0]
