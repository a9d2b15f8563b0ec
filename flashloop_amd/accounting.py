"""Algorithmic (unique, compulsory) HBM bytes of each decode-step kernel.

The roofline numerator: bytes a kernel must move at minimum, not what it happens to
move.  Per (b,h) row, with packed prefix ``Tp`` and tail ``tl``; the readers stream the
fp16 copies of the metadata (the fp32 values are the stored codec state):

* packed stream, dense read: K codes ``Tp*64`` + V codes ``Tp*64``
  + K (scale,min) ``Tp/64 * 128 * 4`` + V (scale,min) ``Tp * 2 * 4``;
* BF16 tail: ``tl * 128 * 2`` each for K and V; vectors q/k_cur/v_cur ``3 * 256``;
  output ``128 * 4``; logits (loop 2) ``(T+1) * 4``;
* top-k: logits read ``(T+1) * 4`` + indices/valid/weights written ``cap * 9`` + mass;
* pack (cache build, J1): reads the bf16 K and V of every loop, ``Tp * 4 * 2 * 256``
  (plus, with loop-3/4 masks, one mask byte and one int32 rank per token and masked
  loop of each sequence); writes per stream and stored row K and V codes ``2 * 64``,
  V (scale, min) in fp32 and fp16 ``2 * (8 + 4)`` and the per-token record ``2 * 8``,
  and per 64-token group K (scale, min) in fp32 and fp16 ``128 * (8 + 4)``;
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


def pack_bytes(packed, stream_rows, masked_tokens: int = 0) -> tuple[int, int]:
    """(read, written) algorithmic bytes of one cache build: ``packed`` = packed prefix
    per (b,h) row, ``stream_rows[s]`` = rows stored in stream s per (b,h) row (the
    packed prefix for loops 1/2, the active tokens for loops 3/4), ``masked_tokens`` =
    tokens x masked loops summed over sequences (mask byte + rank entry each)."""
    p = np.asarray(packed, np.int64)
    read = int((p * 4 * 2 * BF16_ROW).sum()) + masked_tokens * (1 + 4)
    written = 0
    for rows in stream_rows:
        r = np.asarray(rows, np.int64)
        written += int((r * (2 * CODE_ROW + 2 * (VMETA_ROW // 2 + VMETA_ROW_F16 // 2) + VMETA_ROW)).sum())
        written += int(((p // 64) * (KMETA_GROUP + KMETA_GROUP_F16)).sum())
    return read, written


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


# ---------------------------------------------------------------------------------
# The reference's own accounting, for the audit fields a drop-in must report with the
# reference's values: the codec's byte count of a temporal group
# (flashloop_torch/kv_quantization.py:489-527, 606-620), the streaming compressor's
# audit (kv_quantization.py:246-322) and the storage of a reference cache layer in its
# KIVI layout (flashloop/cache.py:1084-1101; tensor shapes kivi_backend.py:346-360).
# ---------------------------------------------------------------------------------
def codec_group_bytes(batch: int, heads: int, channels: int, group_tokens: int, transition_active,
                      bits: int = 4, group_size: int = 64) -> int:
    """Packed bytes of one temporal group of the residual chain: the anchor and every
    transition's active rows, K per channel (one 4-byte fp16 (scale, min) pair per
    channel of each stream holding a row) and V per token (one pair per 64 channels of
    each active token)."""
    pairs_v = -(-channels // group_size)
    total = 0
    for tokens in [batch * group_tokens, *[int(x) for x in transition_active]]:
        if tokens == 0:
            continue
        payload = -(-tokens * heads * channels * bits // 8)
        total += 2 * payload + 4 * (batch * heads * channels) + 4 * (tokens * heads * pairs_v)
    return total


def codec_audit(*, num_layers: int, batch: int, heads: int, channels: int, total_tokens: int,
                current_tokens: int, quantized_tokens: int, group_bytes, mask_numel: int | None,
                recurrent_steps: int = 4) -> dict:
    """The compressor audit's byte fields from the per-(layer, group) packed bytes."""
    packed = int(sum(group_bytes))
    tail = total_tokens - quantized_tokens
    per_token = num_layers * recurrent_steps * 2 * batch * heads * channels * 2
    residual = per_token * tail
    dense = per_token * total_tokens
    masks = -(-2 * int(mask_numel) // 8) if mask_numel is not None else 0
    total = packed + residual + masks
    return {
        "quantized_groups": len(group_bytes),
        "quantized_tokens": quantized_tokens,
        "bf16_tail_tokens": tail,
        "total_cache_tokens": total_tokens,
        "current_cache_tokens": current_tokens,
        "packed_stream_bytes": packed,
        "residual_bf16_bytes": residual,
        "mask_bytes": masks,
        "total_packed_bytes": total,
        "dense_recurrent_bf16_bytes": dense,
        "dense_r4_bf16_bytes": dense if recurrent_steps == 4 else None,
        "dense_recurrent_ratio": total / dense if dense else None,
        "dense_r4_ratio": total / dense if recurrent_steps == 4 and dense else None,
    }


def reference_layer_storage_bytes(*, batch: int, heads: int, channels: int, packed_tokens: int, tail_tokens: int,
                                  rows_loop3: int, rows_loop4: int, group_size: int = 64) -> int:
    """What ``CrossLoopKVLayer.storage_bytes`` of the reference reports for the same
    cache built by prefill with the KIVI reader: per packed stream (anchor and loop-2
    residual over the prefix, loop-3/4 residuals over their compact rows) an int32
    payload of 8 codes per word (K token-packed, V channel-packed) and fp16 minimum and
    scale (K per channel per 64 rows, V per token per 64 channels); the four loops' BF16
    tails; int64 override positions, int32 rank maps over the prefix and the two bool
    tail-activity rows."""
    total = 0
    for rows in (packed_tokens, packed_tokens, rows_loop3, rows_loop4):
        if rows == 0:
            continue
        k_payload = 4 * batch * heads * (-(-rows // 8)) * channels
        k_meta = 2 * 2 * batch * heads * (-(-rows // group_size)) * channels
        v_payload = 4 * batch * heads * (-(-channels // 8)) * rows
        v_meta = 2 * 2 * batch * heads * rows * (-(-channels // group_size))
        total += k_payload + k_meta + v_payload + v_meta
    total += 4 * 2 * 2 * batch * heads * tail_tokens * channels
    total += 8 * (rows_loop3 + rows_loop4) + 4 * 2 * packed_tokens + 2 * batch * tail_tokens
    return total
