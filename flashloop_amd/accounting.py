"""Algorithmic (unique, compulsory) HBM bytes of each decode-step kernel.

The roofline numerator: bytes a kernel must move at minimum, not what it happens to
move.  Per (b,h) row, with packed prefix ``Tp`` and tail ``tl``; the readers stream the
fp16 copies of the metadata (the fp32 values are the stored codec state):

* packed stream, dense read: K codes ``Tp*64`` + V codes ``Tp*64``
  + K (scale,min) ``Tp/64 * 128 * 4`` + V (scale,min) ``Tp * 2 * 4``;
* BF16 tail: ``tl * 128 * 2`` each for K and V; vectors q/k_cur/v_cur ``3 * 256``;
  output ``128 * 4``; logits (loop 2) ``(T+1) * 4``;
* top-k: logits read ``(T+1) * 4`` + indices/valid/weights written ``cap * 9`` + mass;
* sparse readers: per selected prefix row and stream, K codes 64 + V codes 64 +
  V metadata 16, plus 512 B of K metadata per touched (group, stream) -- these readers
  stream the fp16 copy of the K metadata; selected tail or current rows 256 per K or V;
  the selection itself ``cap * 5`` (+ weights 4).
"""

from __future__ import annotations

import numpy as np

KMETA_GROUP = 128 * 8  # (scale, min) f32 per channel of one 64-token group
KMETA_GROUP_F16 = 128 * 4  # the fp16 copy the readers stream
VMETA_ROW_F16 = 2 * 4  # the fp16 copy the dense readers stream
VMETA_ROW = 2 * 8  # (scale, min) f32 per 64-channel half of one token
CODE_ROW = 64  # int4 x 128 channels
BF16_ROW = 256


def dense_bytes(packed, tail, streams: int, logits: bool) -> int:
    """Sum over rows of one dense reader call; ``packed``/``tail`` per row."""
    p = np.asarray(packed, np.int64)
    t = np.asarray(tail, np.int64)
    per_stream = p * 2 * CODE_ROW + (p // 64) * KMETA_GROUP_F16 + p * VMETA_ROW_F16
    tot = streams * per_stream + t * 2 * BF16_ROW + 3 * BF16_ROW + 128 * 4
    if logits:
        tot = tot + (p + t + 1) * 4
    return int(tot.sum())


def topk_bytes(packed, tail, cap: int) -> int:
    p = np.asarray(packed, np.int64)
    t = np.asarray(tail, np.int64)
    return int(((p + t + 1) * 4 + cap * 9 + 4).sum())


def selection_stats(indices: np.ndarray, counts: np.ndarray, packed, rank3=None, rank4=None, batch_of_row=None):
    """Per row: selected prefix rows, selected tail/current rows, touched groups, and the
    prefix rows present in streams 2/3 (through the rank maps)."""
    rows = indices.shape[0]
    out = []
    for r in range(rows):
        k = int(counts[r])
        sel = indices[r, :k].astype(np.int64)
        p = int(packed[r])
        pre = sel[sel < p]
        g = np.unique(pre // 64)
        b = batch_of_row[r] if batch_of_row is not None else 0
        n3 = int((rank3[b][pre] >= 0).sum()) if rank3 is not None else len(pre)
        n4 = int((rank4[b][pre] >= 0).sum()) if rank4 is not None else len(pre)
        out.append(dict(prefix=len(pre), other=k - len(pre), groups=len(g), s2=n3, s3=n4))
    return out


def selected_pv_bytes(stats, cap: int, streams: int = 2) -> int:
    tot = 0
    for s in stats:
        tot += s["prefix"] * streams * (CODE_ROW + VMETA_ROW) + s["other"] * BF16_ROW
        tot += cap * 9 + 128 * 4
    return tot


def sparse_bytes(stats, cap: int, loop: int, with_source: bool = False) -> int:
    """Cached-mass sparse reader of loop index ``loop`` (2 or 3): streams 0..loop.
    ``with_source``: the pass also forms the loop-2 selected aggregate -- its V rows of
    streams 0/1 are already counted; add the weights, loop-2 tail/current V rows and
    the aggregate written."""
    tot = 0
    for s in stats:
        if with_source:
            tot += cap * 4 + s["other"] * BF16_ROW + 128 * 4
        rows_per_stream = [s["prefix"], s["prefix"], s["s2"], s["s3"]][: loop + 1]
        for n in rows_per_stream:
            tot += n * (2 * CODE_ROW + VMETA_ROW)
        tot += s["groups"] * KMETA_GROUP_F16 * (loop + 1)
        tot += s["other"] * 2 * BF16_ROW
        tot += 3 * BF16_ROW + 128 * 4 + 4 + 128 * 4 + cap * 5
    return tot
