"""``flashloop(model)``: the hook-style entry point of ``flashloop_torch`` (flashloop_torch/__init__.py:5-22).

    with flashloop(model) as hooks:
        out = model.generate(input_ids, max_new_tokens=64)
        hooks["attention_and_prefill"].audit(); hooks["kv"].audit()

The reference installs forward hooks on the Hugging Face Ouro modules (token-sparse
prefill freezing, loop-2 key capture and loop-3/4 cached-mass replacement, and a KV
fake-quantizer, flashloop_torch/integration.py:179-246, kv_quantization.py:325-392).
Here the same three lazy updates run through ``FlashLoopEngine`` on the HIP kernels:
inside the context ``model.generate`` is routed through the engine; on exit the original
method is restored.  The two yielded objects keep the reference's ``audit()`` /
``close()`` interface and counters.
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Any

import torch

from .config import FlashLoopConfig
from .engine import FlashLoopEngine


class TokenSparsePrefillCachedMassIntervention:
    """Counters of the decode cached-mass attention and the token-sparse prefill
    (flashloop_torch/integration.py:179-246)."""

    def __init__(self, engine: FlashLoopEngine, attention_fraction: float, fraction_loop3: float,
                 fraction_loop4: float) -> None:
        self.engine = engine
        self.attention_fraction = attention_fraction
        self.fraction_loop3 = fraction_loop3
        self.fraction_loop4 = fraction_loop4
        self.prefill_attention_calls = 0
        self.source_captures = 0
        self.target_replacements = 0
        self.active_counts: dict[str, int] = {}
        self.mask_nested = False
        self.closed = False

    def _record_prefill(self) -> None:
        st = self.engine.state
        nl = len(self.engine.layers)
        self.prefill_attention_calls += 4 * nl
        self.active_counts = {"3": int(st.mask_loop3.sum().item()), "4": int(st.mask_loop4.sum().item())}
        self.mask_nested = bool(torch.all(~st.mask_loop4 | st.mask_loop3).item())

    def _record_decode(self) -> None:
        nl = len(self.engine.layers)
        self.source_captures += nl
        self.target_replacements += 2 * nl

    def audit(self) -> dict[str, Any]:
        return {
            "attention": {
                "prefill_attention_calls": self.prefill_attention_calls,
                "source_captures": self.source_captures,
                "target_replacements": self.target_replacements,
            },
            "token_sparse_prefill": {"active_counts": dict(self.active_counts), "mask_nested": self.mask_nested},
        }

    def close(self) -> None:
        self.closed = True


class CrossLoopKVQuantizationIntervention:
    """Codec accounting of the packed cross-loop cache (flashloop_torch/kv_quantization.py:325-392)."""

    def __init__(self, engine: FlashLoopEngine) -> None:
        self.engine = engine
        self.forward_calls = 0
        self.cache_updates = 0
        self.closed = False

    def audit(self) -> dict[str, Any]:
        base = {"forward_calls": self.forward_calls, "cache_updates": self.cache_updates, "closed": self.closed}
        if self.engine._state is None:
            return {"status": "PENDING", "quantized_groups": 0, "quantized_tokens": 0, **base}
        layers = [l for l in self.engine.state.cache.layers if l is not None]
        first = layers[0]
        storage = sum(l.storage_bytes for l in layers)
        dense = sum(l.dense_bf16_bytes for l in layers)
        h = first.heads
        tails = sum(first.tail_host)
        # kv_quantization.py:246-322 field by field: packed streams (codes + fp32 metadata
        # + rank maps), the BF16 tails of every loop, and the two prefill masks as bits
        tail_bytes = len(layers) * 4 * 2 * h * tails * 128 * 2
        st = self.engine.state
        mask_bytes = -(-2 * int(st.mask_loop3.numel()) // 8) if st.mask_loop3 is not None else 0
        packed_stream_bytes = storage - tail_bytes
        return {
            "status": "PASS",
            "kind": "asymmetric_cross_loop_innovation_int4",
            "codec_profile": "kivi4_channel",
            "recurrent_steps": 4,
            "key_axes": ["per_channel"] * 4,
            "value_axes": ["per_token"] * 4,
            "k_bits": [4] * 4,
            "v_bits": [4] * 4,
            "group_size": 64,
            "residual_length": 64,
            "quantized_groups": sum(sum(l.packed_host) // 64 for l in layers),
            "quantized_tokens": first.quantized_tokens,
            "bf16_tail_tokens": first.tail_tokens_max,
            "total_cache_tokens": first.token_count,
            "current_cache_tokens": first.token_count,
            "packed_stream_bytes": packed_stream_bytes,
            "residual_bf16_bytes": tail_bytes,
            "mask_bytes": mask_bytes,
            "total_packed_bytes": storage + mask_bytes,
            "dense_recurrent_bf16_bytes": dense,
            "dense_r4_bf16_bytes": dense,
            "dense_recurrent_ratio": (storage + mask_bytes) / dense if dense else None,
            "dense_r4_ratio": (storage + mask_bytes) / dense if dense else None,
            "reference_cache_materialized": False,
            **base,
        }

    def close(self) -> None:
        self.closed = True


@contextmanager
def flashloop(model, *, attention_fraction: float = 0.10, fraction_loop3: float = 0.25, fraction_loop4: float = 0.10):
    config = FlashLoopConfig(prefill_fraction_loop3=fraction_loop3, prefill_fraction_loop4=fraction_loop4,
                             decode_key_fraction=attention_fraction)
    engine = FlashLoopEngine(model, config=config)
    joint = TokenSparsePrefillCachedMassIntervention(engine, attention_fraction, fraction_loop3, fraction_loop4)
    kv = CrossLoopKVQuantizationIntervention(engine)
    had_own = "generate" in model.__dict__
    original = model.__dict__.get("generate")

    def generate(input_ids, *, max_new_tokens: int, eos_token_id=None, **_ignored):
        engine.reset()
        out = engine.generate(input_ids, max_new_tokens=max_new_tokens, eos_token_id=eos_token_id)
        joint._record_prefill()
        steps = out.shape[1] - input_ids.shape[1] - 1  # decode calls (the first token comes from prefill)
        for _ in range(max(0, steps)):
            joint._record_decode()
        kv.forward_calls += 1 + max(0, steps)
        kv.cache_updates += 1 + max(0, steps)
        return out

    model.generate = generate
    try:
        yield {"attention_and_prefill": joint, "kv": kv}
    finally:
        if had_own:
            model.generate = original
        else:
            del model.generate
        kv.close()
        joint.close()
