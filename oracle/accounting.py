"""The reference's byte accounting of the cross-loop cache, restated.

Test infrastructure: the checker for the audit fields ``flashloop_amd`` reports with
the reference's values.  Pinned by hand-computed cases in
``tests/test_oracle_accounting.py``.

* ``stream_bytes`` -- ``_payload_bytes``/``_k_stream_bytes``/``_v_stream_bytes``
  (flashloop_torch/kv_quantization.py:489-527);
* ``temporal_group_bytes`` -- ``packed_bytes`` of ``encode_temporal_group``
  (kv_quantization.py:600-620);
* ``compressor_audit`` -- ``CrossLoopKVCacheCompressor.audit`` (kv_quantization.py:246-322);
* ``kivi_layer_storage_bytes`` -- ``CrossLoopKVLayer.storage_bytes``
  (flashloop/cache.py:1084-1101) of a prefill-built layer with the KIVI reader: payload,
  minimum and scale of ``KiviPacked4Bit`` (flashloop/kivi_backend.py:328-360), tails
  (cache.py:690-702), override positions and rank maps (cache.py:880-910, 281-289).
"""

from __future__ import annotations

import math


def stream_bytes(shape, active_values: int, bits: int, axis: str, group_size: int = 64) -> int:
    batch, heads, _tokens, channels = (int(x) for x in shape)
    if active_values == 0:
        return 0
    payload = math.ceil(active_values * bits / 8)
    active_tokens = active_values // (heads * channels)
    if axis == "per_channel":
        groups = batch * heads * channels if active_tokens else 0
    elif axis == "per_token":
        groups = active_tokens * heads * math.ceil(channels / group_size)
    else:
        raise ValueError(axis)
    return payload + 4 * groups


def temporal_group_bytes(shape, transition_tokens, bits: int = 4, group_size: int = 64) -> dict:
    """``shape`` [B, H, group, C]; ``transition_tokens``: active tokens of loops 2..4."""
    batch, heads, tokens, channels = (int(x) for x in shape)
    counts = [batch * heads * tokens * channels] + [int(t) * heads * channels for t in transition_tokens]
    k = [stream_bytes(shape, c, bits, "per_channel", group_size) for c in counts]
    v = [stream_bytes(shape, c, bits, "per_token", group_size) for c in counts]
    return {"k_stream_bytes": k, "v_stream_bytes": v, "packed_bytes": sum(k) + sum(v)}


def compressor_audit(*, num_layers, recurrent_steps, batch, heads, channels, total_tokens, current_tokens,
                     next_start, packed_stream_bytes, quantized_groups, mask_numel=None) -> dict:
    unique = min(next_start)
    tail = total_tokens - unique
    residual = num_layers * recurrent_steps * 2 * batch * heads * tail * channels * 2
    dense = num_layers * recurrent_steps * 2 * batch * heads * total_tokens * channels * 2
    mask_bytes = math.ceil(2 * mask_numel / 8) if mask_numel is not None else 0
    total = packed_stream_bytes + residual + mask_bytes
    return {
        "quantized_groups": quantized_groups,
        "quantized_tokens": unique,
        "bf16_tail_tokens": tail,
        "total_cache_tokens": total_tokens,
        "current_cache_tokens": current_tokens,
        "packed_stream_bytes": packed_stream_bytes,
        "residual_bf16_bytes": residual,
        "mask_bytes": mask_bytes,
        "total_packed_bytes": total,
        "dense_recurrent_bf16_bytes": dense,
        "dense_r4_bf16_bytes": dense if recurrent_steps == 4 else None,
        "dense_recurrent_ratio": total / dense if dense else None,
        "dense_r4_ratio": total / dense if recurrent_steps == 4 and dense else None,
    }


def _nbytes(shape, itemsize: int) -> int:
    return math.prod(int(x) for x in shape) * itemsize


def kivi_layer_storage_bytes(*, batch, heads, channels, packed_tokens, tail_tokens, rows3, rows4,
                             group_size: int = 64) -> int:
    total = 0
    for rows in (packed_tokens, packed_tokens, rows3, rows4):
        if rows == 0:
            continue  # no stream was packed
        # K: per channel over tokens -> payload [B, H, ceil(T/8), C] i32, meta [B, H, ceil(T/g), C] f16
        total += _nbytes((batch, heads, (rows + 7) // 8, channels), 4)
        total += 2 * _nbytes((batch, heads, math.ceil(rows / group_size), channels), 2)
        # V: per token over channels -> payload [B, H, ceil(C/8), T] i32, meta [B, H, T, ceil(C/g)] f16
        total += _nbytes((batch, heads, (channels + 7) // 8, rows), 4)
        total += 2 * _nbytes((batch, heads, rows, math.ceil(channels / group_size)), 2)
    total += 2 * 4 * _nbytes((batch, heads, tail_tokens, channels), 2)  # 4 loops x (K, V) bf16 tails
    total += _nbytes((rows3,), 8) + _nbytes((rows4,), 8)  # override positions
    total += 2 * _nbytes((packed_tokens,), 4)  # rank maps
    total += 2 * _nbytes((batch, tail_tokens), 1)  # tail activity
    return total
