"""Ragged batched FlashLoop inference: ``B`` sequences of different lengths share one
packed cross-loop cache per layer and decode together.

The reference engine is batch-one (flashloop/engine.py:176-177).  This engine keeps its
per-sequence semantics and batches what batches for free:

* prefill runs the reference's four loops per sequence (token-sparse selection is a
  per-sequence top-k of the hidden delta score, flashloop/selection.py:26-69), then packs
  all sequences of a layer in one ``CrossLoopKVLayer`` with per-sequence prefix and tail
  lengths;
* a decode step is one pass of the model over ``[B, 1]`` tokens: every GEMM runs on the
  whole batch, each (b, h) row of the readers sees its own sequence's length, the loop-2
  selection budget is ``ceil((T_b + 1) * fraction)`` per sequence, and each sequence's
  tail rolls over on its own schedule.  Steps replay a captured HIP graph as in the
  batch-one engine.

Greedy ``generate`` keeps decoding a batch until every sequence has produced its tokens
(or its EOS); a sequence that has stopped is fed its EOS and its later tokens dropped.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .cache import CrossLoopKVCache, CrossLoopKVLayer
from .config import FlashLoopConfig
from .engine import DecodeReceipt, DecodeRunner, FlashLoopEngine, PrefillReceipt
from .model import OuroConfig, OuroForCausalLM


@dataclass(frozen=True)
class BatchState:
    cache: CrossLoopKVCache
    positions: tuple[int, ...]  # next position of every sequence
    mask_loop3: torch.Tensor  # [B, Tmax] bool (False past each sequence's length)
    mask_loop4: torch.Tensor
    prefill_receipts: tuple[tuple[PrefillReceipt, ...], ...]  # per sequence


@dataclass(frozen=True)
class BatchPrefillOutput:
    logits: torch.Tensor  # [B, vocab] f32, at each sequence's last prompt token
    state: BatchState


@dataclass(frozen=True)
class BatchDecodeOutput:
    logits: torch.Tensor  # [B, vocab] f32
    state: BatchState
    receipts: tuple[DecodeReceipt, ...]  # per sequence


class FlashLoopBatchEngine:
    """FlashLoop prefill/decode/generate over a ragged batch (right-padded prompts)."""

    def __init__(self, model: OuroForCausalLM, *, config: FlashLoopConfig | None = None,
                 use_graphs: bool = True) -> None:
        self._one = FlashLoopEngine(model, config=config, use_graphs=False)
        self.model = self._one.model
        self.config = self._one.config
        self._runner = DecodeRunner(self._one, use_graphs)
        self._state: BatchState | None = None

    @classmethod
    def from_random_init(cls, model_config: OuroConfig, *, seed: int = 0, config: FlashLoopConfig | None = None,
                         device="cuda", use_graphs: bool = True) -> "FlashLoopBatchEngine":
        return cls(OuroForCausalLM.random_init(model_config, seed=seed, device=device), config=config,
                   use_graphs=use_graphs)

    @property
    def state(self) -> BatchState:
        if self._state is None:
            raise RuntimeError("engine cache has not been initialized; call prefill() first")
        return self._state

    @property
    def use_graphs(self) -> bool:
        return self._runner.use_graphs

    @use_graphs.setter
    def use_graphs(self, on: bool) -> None:
        self._runner.use_graphs = bool(on)
        self._runner.reset()

    def reset(self) -> None:
        self._state = None
        self._runner.reset()

    # ------------------------------------------------------------------ prefill
    @staticmethod
    def _lengths(input_ids: torch.Tensor, attention_mask: torch.Tensor | None) -> list[int]:
        bsz, t = input_ids.shape
        if attention_mask is None:
            return [t] * bsz
        if tuple(attention_mask.shape) != (bsz, t):
            raise ValueError("attention_mask must have the shape of input_ids")
        m = attention_mask.to(torch.bool).cpu()
        lengths = [int(x) for x in m.sum(dim=1).tolist()]
        for b, n in enumerate(lengths):
            if n <= 0:
                raise ValueError(f"sequence {b} has no tokens")
            if not bool(m[b, :n].all()):
                raise ValueError("prompts must be right-padded (attention_mask 1...1 0...0)")
        return lengths

    @torch.inference_mode()
    def prefill(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None, *,
                decode_capacity: int | None = None) -> BatchPrefillOutput:
        """Prefill ``input_ids`` ``[B, Tmax]`` (right-padded; ``attention_mask`` marks the
        real tokens) into one packed cache per layer."""
        if self._state is not None:
            raise RuntimeError("engine cache is already initialized; call reset()")
        if input_ids.ndim != 2 or input_ids.shape[0] < 1 or input_ids.shape[1] < 1:
            raise ValueError("input_ids must be [B, T] with B, T >= 1")
        lengths = self._lengths(input_ids, attention_mask)
        bsz, tmax = len(lengths), max(lengths)
        one = self._one
        nl = len(one.layers)
        dev = input_ids.device
        runs = [one._prefill_loops(input_ids[b:b + 1, :n]) for b, n in enumerate(lengths)]
        mask3 = torch.zeros(bsz, tmax, dtype=torch.bool, device=dev)
        mask4 = torch.zeros(bsz, tmax, dtype=torch.bool, device=dev)
        for b, (r, n) in enumerate(zip(runs, lengths)):
            mask3[b, :n] = r.mask3[0]
            mask4[b, :n] = r.mask4[0]
        extra = self.config.decode_capacity if decode_capacity is None else int(decode_capacity)
        cache = CrossLoopKVCache(num_layers=nl)
        for li in range(nl):
            keys, values = [], []
            for loop in range(4):
                ref = runs[0].keys[loop][li]
                kb = torch.zeros(bsz, ref.shape[1], tmax, ref.shape[3], dtype=ref.dtype, device=dev)
                vb = torch.zeros_like(kb)
                for b, (r, n) in enumerate(zip(runs, lengths)):
                    kb[b, :, :n] = r.keys[loop][li][0]
                    vb[b, :, :n] = r.values[loop][li][0]
                keys.append(kb)
                values.append(vb)
            cache.set_layer(li, CrossLoopKVLayer.from_prefill(keys, values, mask_loop3=mask3, mask_loop4=mask4,
                                                              lengths=lengths, token_capacity=tmax + extra))
            del keys, values
        logits = torch.cat([r.logits for r in runs], dim=0)
        self._state = BatchState(cache, tuple(lengths), mask3, mask4, tuple(r.receipts for r in runs))
        self._runner.reset()
        return BatchPrefillOutput(logits=logits, state=self._state)

    # ------------------------------------------------------------------ decode
    @torch.inference_mode()
    def decode(self, token_ids: torch.Tensor) -> BatchDecodeOutput:
        """One step for every sequence: ``token_ids`` ``[B, 1]``.  With graphs on, the
        returned logits live in the graph's output buffer until the next step."""
        st = self.state
        bsz = len(st.positions)
        if tuple(token_ids.shape) != (bsz, 1):
            raise ValueError(f"decode requires token_ids of shape ({bsz}, 1)")
        logits = self._runner.step(st.cache, token_ids, st.positions)
        for lc in st.cache.layers:
            lc.commit_append()
        receipts = tuple(self._one._receipt([p]) for p in st.positions)
        self._state = BatchState(st.cache, tuple(p + 1 for p in st.positions), st.mask_loop3, st.mask_loop4,
                                 st.prefill_receipts)
        return BatchDecodeOutput(logits=logits, state=self._state, receipts=receipts)

    # ------------------------------------------------------------------ generate
    @torch.inference_mode()
    def generate(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None, *,
                 max_new_tokens: int, eos_token_id: int | None = None) -> list[torch.Tensor]:
        """Greedy generation; returns each sequence's prompt + completion (1-D)."""
        if int(max_new_tokens) <= 0:
            raise ValueError("max_new_tokens must be positive")
        if eos_token_id is None:
            eos_token_id = getattr(self.model.config, "eos_token_id", None)
        lengths = self._lengths(input_ids, attention_mask)
        out = self.prefill(input_ids, attention_mask, decode_capacity=int(max_new_tokens) + 64)
        logits = out.logits
        bsz = len(lengths)
        done = torch.zeros(bsz, dtype=torch.bool, device=input_ids.device)
        steps = []
        for step in range(int(max_new_tokens)):
            nxt = torch.argmax(logits, dim=-1, keepdim=True)
            if eos_token_id is not None:
                nxt = torch.where(done[:, None], torch.full_like(nxt, int(eos_token_id)), nxt)
                steps.append((nxt.clone(), done.clone()))
                done = done | (nxt[:, 0] == int(eos_token_id))
                if bool(done.all()):
                    break
            else:
                steps.append((nxt.clone(), done.clone()))
            if step + 1 < int(max_new_tokens):
                logits = self.decode(nxt).logits
        result = []
        for b, n in enumerate(lengths):
            toks = [s[0][b] for s in steps if not bool(s[1][b])]
            comp = torch.cat(toks) if toks else input_ids.new_zeros(0)
            result.append(torch.cat([input_ids[b, :n], comp]))
        return result
