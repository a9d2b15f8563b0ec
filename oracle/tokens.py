"""Token-sparse prefill selection and row gather/scatter, restated in numpy.

Test infrastructure: the checker for ``fl_hidden_delta_score``, ``fl_select_tokens``,
``fl_gather_rows`` and ``fl_scatter_rows``.

Pinned by (tests/test_oracle_tokens.py): nesting and forced-last invariants, the
budget formula, brute-force ranking on small inputs, and gather/scatter round trips
(scatter(gather(x)) restores the selected rows, identity permutations).
"""

from __future__ import annotations

import math

import numpy as np


def hidden_delta_score(current: np.ndarray, previous: np.ndarray) -> np.ndarray:
    """``_hidden_delta_score`` (flashloop/engine.py:78-81), also the ``hidden_delta``
    selector of ``LoopFreezeIntervention._choose_mask`` (token_updates.py:294-296):
    ``||h_r - h_{r-1}|| / max(||h_r||, 1e-12)`` per row, float32 inputs."""
    c = np.asarray(current, np.float64)
    p = np.asarray(previous, np.float64)
    num = np.sqrt(((c - p) ** 2).sum(-1))
    den = np.maximum(np.sqrt((c**2).sum(-1)), 1e-12)
    return num / den


def select_active_mask(scores: np.ndarray, fraction: float, eligible: np.ndarray | None = None, force_last_token: bool = True) -> np.ndarray:
    """``select_prefill_tokens`` (flashloop/selection.py:26-69) / ``select_active_mask``
    (flashloop_torch/token_updates.py:24-62).

    Global budget ``max(1, ceil(T * f))`` over all tokens; candidates are the eligible
    rows minus the forced last token; the top ``count - forced`` candidates by score are
    chosen (ties: lower index; ``torch.topk`` leaves them unspecified); the last token is
    always selected.  ``scores``: ``[B, T]``.  Returns bool ``[B, T]``.
    """
    s = np.asarray(scores, np.float32)
    b, t = s.shape
    if eligible is None:
        eligible = np.ones((b, t), bool)
    budget = max(1, math.ceil(t * float(fraction)))
    out = np.zeros((b, t), bool)
    for bi in range(b):
        cand = np.nonzero(eligible[bi])[0]
        if cand.size == 0:
            raise ValueError("eligible contains an empty batch row")
        forced = []
        if force_last_token:
            if not eligible[bi, t - 1]:
                raise ValueError("the forced final token must be eligible")
            forced = [t - 1]
            cand = cand[cand != t - 1]
        count = min(budget, cand.size + len(forced))
        rem = count - len(forced)
        if rem > 0:
            order = np.argsort(-s[bi, cand].astype(np.float64), kind="stable")[:rem]
            out[bi, cand[order]] = True
        if forced:
            out[bi, forced] = True
    return out


def gather_rows(x: np.ndarray, positions: np.ndarray, axis: int) -> np.ndarray:
    """``index_select`` of active rows (flashloop/prefill.py:158, engine.py:284-316)."""
    return np.take(x, np.asarray(positions, np.int64), axis=axis)


def scatter_rows(dst: np.ndarray, positions: np.ndarray, rows: np.ndarray, axis: int) -> np.ndarray:
    """``index_copy_`` of computed rows back (flashloop/prefill.py:193-194, 237)."""
    out = np.array(dst, copy=True)
    idx = [slice(None)] * out.ndim
    idx[axis] = np.asarray(positions, np.int64)
    out[tuple(idx)] = rows
    return out


def carry_frozen_hidden(previous: np.ndarray, computed: np.ndarray, active: np.ndarray) -> np.ndarray:
    """``carry_frozen_hidden`` (token_updates.py:65-71): computed rows where active."""
    return np.where(active[..., None], computed, previous)


def replace_frozen_cache(previous: np.ndarray, current: np.ndarray, active: np.ndarray) -> np.ndarray:
    """``replace_frozen_cache`` (token_updates.py:74-82): ``[B,H,T,D]`` rows by ``[B,T]`` mask."""
    return np.where(active[:, None, :, None], current, previous)
