"""``flashloop(model)``: the hook-style entry point of ``flashloop_torch`` (flashloop_torch/__init__.py:5-22).

    with flashloop(model) as hooks:
        out = model.generate(input_ids, max_new_tokens=64)
        step = model(input_ids)                        # any forward, too
        hooks["attention_and_prefill"].audit(); hooks["kv"].audit()

The reference registers forward hooks on the Hugging Face Ouro modules, so every
forward or generate inside the context runs with FlashLoop's lazy updates: token-sparse
prefill freezing, loop-2 key capture and loop-3/4 cached-mass replacement, and the KV
codec (flashloop_torch/attention.py:290-295, kv_quantization.py:352,
integration.py:179-246).  Here those updates are the engine's HIP path, so inside the
context both entry points of the model are routed through ``FlashLoopEngine``:

* ``model(input_ids)`` without a cache prefills (logits of every position) and returns
  a ``FlashLoopCache`` as ``past_key_values``; ``model(next_ids, past_key_values=cache)``
  with one token decodes one step on it (logits ``[1, 1, vocab]``);
* ``model.generate(input_ids, max_new_tokens=...)`` is greedy generation on the engine.

Arguments the engine cannot honour raise (``TypeError`` for unknown ones, ``ValueError``
for unsupported values) instead of being dropped.  The audit counters count what the
engine actually ran (its prefill receipts, decode receipts and cache updates), and the
``kv`` audit reports the reference's byte accounting next to this layout's physical
bytes.  On exit the model's own methods are restored.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
from typing import Any

import torch

from . import accounting
from .config import FlashLoopConfig
from .engine import DecodeOutput, FlashLoopEngine, PrefillOutput


class FlashLoopCache:
    """``past_key_values`` of a routed forward: a handle on the engine's packed cache at
    one position (the reference returns the Hugging Face cache object)."""

    def __init__(self, engine: FlashLoopEngine, position: int) -> None:
        self.engine = engine
        self.position = int(position)

    def get_seq_length(self) -> int:
        return self.position


@dataclass
class FlashLoopOutput:
    logits: torch.Tensor
    past_key_values: FlashLoopCache


class TokenSparsePrefillCachedMassIntervention:
    """Counters of the decode cached-mass attention and the token-sparse prefill
    (flashloop_torch/integration.py:179-246, attention.py:278-380), taken from what the
    engine ran."""

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
        self.active_masks: dict[int, torch.Tensor] = {}
        self.mask_nested = False
        self.closed = False

    def observe_prefill(self, out: PrefillOutput) -> None:
        st = out.state
        nl = len(self.engine.layers)
        self.prefill_attention_calls += len(st.prefill_receipts) * nl
        self.active_counts = {str(r.loop): int(r.active_rows) for r in st.prefill_receipts if r.loop >= 3}
        self.active_masks = {2: st.mask_loop3, 3: st.mask_loop4}
        self.mask_nested = bool(torch.all(~st.mask_loop4 | st.mask_loop3).item())

    def observe_decode(self, out: DecodeOutput) -> None:
        rc = out.receipt
        self.source_captures += len(rc.selected_keys_per_layer)
        self.target_replacements += int(rc.sparse_attention_calls)

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
    """Codec audit of the packed cross-loop cache (flashloop_torch/kv_quantization.py:325-392).
    ``forward_calls`` counts routed model forwards (each prefill or decode step),
    ``cache_updates`` the ones that wrote the cache."""

    def __init__(self, engine: FlashLoopEngine) -> None:
        self.engine = engine
        self.forward_calls = 0
        self.cache_updates = 0
        self.closed = False

    def observe_forward(self) -> None:
        self.forward_calls += 1
        self.cache_updates += 1

    def audit(self) -> dict[str, Any]:
        base = {"forward_calls": self.forward_calls, "cache_updates": self.cache_updates, "closed": self.closed}
        if self.engine._state is None:
            return {"status": "PENDING", "quantized_groups": 0, "quantized_tokens": 0, **base}
        st = self.engine.state
        layers = [l for l in st.cache.layers if l is not None]
        first = layers[0]
        b, h = first.batch, first.heads
        # the reference's packed bytes, group by group: loops 3/4 hold the rows their rank
        # maps name (prefill masks, then decode rows), loop 2 every row
        group_bytes = []
        for lay in layers:
            tp = min(lay.packed_host)
            g = tp // 64
            ranks = [lay.rank[s][:, : g * 64].reshape(b, g, 64).ge(0).sum(dim=(0, 2)).cpu().tolist() for s in range(2)]
            for j in range(g):
                group_bytes.append(accounting.codec_group_bytes(b, h, 128, 64, [b * 64, ranks[0][j], ranks[1][j]]))
        total = first.token_count
        codec = accounting.codec_audit(num_layers=len(layers), batch=b, heads=h, channels=128, total_tokens=total,
                                       current_tokens=total, quantized_tokens=min(first.packed_host),
                                       group_bytes=group_bytes,
                                       mask_numel=int(st.mask_loop3.numel()) if st.mask_loop3 is not None else None)
        storage = sum(l.storage_bytes for l in layers)
        reference_storage = sum(
            accounting.reference_layer_storage_bytes(
                batch=1, heads=h, channels=128, packed_tokens=l.packed_host[i], tail_tokens=l.tail_host[i],
                rows_loop3=l.late_rows_host[0][i], rows_loop4=l.late_rows_host[1][i])
            for l in layers for i in range(b))
        dense = sum(l.dense_bf16_bytes for l in layers)
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
            **codec,
            "reference_cache_materialized": False,
            # this build's buffers next to what the reference's packed layer would hold
            "physical_storage_bytes": storage,
            "physical_storage_ratio": storage / dense if dense else None,
            "reference_layout_storage_bytes": reference_storage,
            "reference_layout_storage_ratio": reference_storage / dense if dense else None,
            **base,
        }

    def close(self) -> None:
        self.closed = True


_GENERATE_KW = {"max_new_tokens", "eos_token_id", "attention_mask", "do_sample", "num_beams", "use_cache",
                "pad_token_id", "stop_token_sequences", "return_dict_in_generate", "output_scores"}
_FORWARD_KW = {"attention_mask", "past_key_values", "use_cache", "return_dict", "position_ids", "cache_position"}


def _all_ones(mask) -> bool:
    return mask is None or bool(torch.as_tensor(mask).bool().all())


@contextmanager
def flashloop(model, *, attention_fraction: float = 0.10, fraction_loop3: float = 0.25, fraction_loop4: float = 0.10):
    config = FlashLoopConfig(prefill_fraction_loop3=fraction_loop3, prefill_fraction_loop4=fraction_loop4,
                             decode_key_fraction=attention_fraction)
    engine = FlashLoopEngine(model, config=config)
    joint = TokenSparsePrefillCachedMassIntervention(engine, attention_fraction, fraction_loop3, fraction_loop4)
    kv = CrossLoopKVQuantizationIntervention(engine)

    # every prefill and decode the engine runs (generate's included) is observed
    engine_prefill, engine_decode = engine.prefill, engine.decode

    def prefill(*args, **kwargs):
        out = engine_prefill(*args, **kwargs)
        joint.observe_prefill(out)
        kv.observe_forward()
        return out

    def decode(*args, **kwargs):
        out = engine_decode(*args, **kwargs)
        joint.observe_decode(out)
        kv.observe_forward()
        return out

    engine.prefill, engine.decode = prefill, decode

    def generate(input_ids, max_new_tokens=None, **kwargs):
        unknown = set(kwargs) - _GENERATE_KW
        if unknown:
            raise TypeError(f"flashloop generate: unsupported argument(s) {sorted(unknown)}")
        if max_new_tokens is None:
            raise TypeError("flashloop generate: max_new_tokens is required")
        if kwargs.get("do_sample"):
            raise ValueError("flashloop generate: only greedy decoding (do_sample=False) is implemented")
        if int(kwargs.get("num_beams", 1) or 1) != 1:
            raise ValueError("flashloop generate: beam search is not implemented (num_beams must be 1)")
        if kwargs.get("use_cache") is False:
            raise ValueError("flashloop generate: the packed cache is the decode path (use_cache=False unsupported)")
        if kwargs.get("return_dict_in_generate") or kwargs.get("output_scores"):
            raise ValueError("flashloop generate: returns the token ids only")
        if not _all_ones(kwargs.get("attention_mask")):
            raise ValueError("flashloop generate: padded prompts are not supported at batch one")
        engine.reset()
        return engine.generate(input_ids, max_new_tokens=int(max_new_tokens),
                               eos_token_id=kwargs.get("eos_token_id"),
                               stop_token_sequences=tuple(kwargs.get("stop_token_sequences", ())))

    def forward(input_ids, **kwargs):
        unknown = set(kwargs) - _FORWARD_KW
        if unknown:
            raise TypeError(f"flashloop forward: unsupported argument(s) {sorted(unknown)}")
        if kwargs.get("use_cache") is False:
            raise ValueError("flashloop forward: the packed cache is the path (use_cache=False unsupported)")
        if not _all_ones(kwargs.get("attention_mask")):
            raise ValueError("flashloop forward: padded inputs are not supported at batch one")
        cache = kwargs.get("past_key_values")
        pos = kwargs.get("position_ids", kwargs.get("cache_position"))
        if cache is None:
            if pos is not None and not torch.equal(torch.as_tensor(pos).flatten().cpu(),
                                                   torch.arange(input_ids.shape[1])):
                raise ValueError("flashloop forward: a prefill starts at position 0")
            engine.reset()
            out = engine.prefill(input_ids, all_logits=True)
            return FlashLoopOutput(out.logits, FlashLoopCache(engine, out.state.next_position))
        if not isinstance(cache, FlashLoopCache) or cache.engine is not engine:
            raise TypeError("flashloop forward: past_key_values must be the cache a routed forward returned")
        if engine._state is None or cache.position != engine.state.next_position:
            raise ValueError("flashloop forward: this cache is stale (the engine has moved past it)")
        if input_ids.shape != (1, 1):
            raise ValueError("flashloop forward: decode steps take exactly one token at batch one")
        if pos is not None and int(torch.as_tensor(pos).flatten()[-1]) != cache.position:
            raise ValueError("flashloop forward: position does not follow the cache")
        out = engine.decode(input_ids)
        # a copy: the engine's logits buffer is overwritten by the next step's graph replay,
        # and a caller of an HF-style forward may keep every step's output
        return FlashLoopOutput(out.logits.unsqueeze(1).clone(), FlashLoopCache(engine, out.state.next_position))

    saved = {name: model.__dict__[name] for name in ("generate", "forward") if name in model.__dict__}
    model.generate = generate
    model.forward = forward  # nn.Module.__call__ dispatches to the instance attribute
    try:
        yield {"attention_and_prefill": joint, "kv": kv}
    finally:
        for name in ("generate", "forward"):
            if name in saved:
                setattr(model, name, saved[name])
            else:
                del model.__dict__[name]
        engine.reset()
        kv.close()
        joint.close()
