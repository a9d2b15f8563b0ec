"""Batch-one looped-decoder inference with the FlashLoop lazy updates on MI355X.

Mirrors ``FlashLoopEngine`` (flashloop/engine.py:112-607): ``from_pretrained``,
``prefill``, ``decode``, ``generate``, ``reset``, ``state``.  The three lazy updates run
on this build's HIP kernels:

* token-sparse prefill loops 3/4 -- row scores (``fl_hidden_delta_score``), nested global
  top-k selection with the forced last token (``fl_select_tokens``) and row gather /
  scatter of hidden states and K/V (``fl_gather_rows`` / ``fl_scatter_rows``);
* the int4 anchor + residual cross-loop KV cache (``fl_pack_kv_groups``);
* decode loops 1-2 dense over the packed cache (``fl_decode_attn_dense``), loop-2 key
  selection (``fl_decode_topk``), loops 3-4 cached-mass sparse attention
  (``fl_decode_attn_sparse_delta[_fused]``).

Model GEMMs, norms and SDPA of the dense prefill loops are torch (hipBLASLt).
"""

from __future__ import annotations

import gc
import math
import weakref
from dataclasses import dataclass, field
from typing import Callable, Sequence

import torch
import torch.nn.functional as F

from . import kernels
from .cache import CrossLoopKVCache, CrossLoopKVLayer
from .config import FlashLoopConfig, validate_ouro_model
from .model import OuroConfig, OuroForCausalLM, apply_rope


@dataclass(frozen=True)
class PrefillReceipt:
    """Row accounting of one prefill loop (flashloop/prefill.py:46-58)."""

    loop: int
    total_rows: int
    active_rows: int


@dataclass(frozen=True)
class EngineState:
    cache: CrossLoopKVCache
    next_position: int
    mask_loop3: torch.Tensor
    mask_loop4: torch.Tensor
    prefill_receipts: tuple[PrefillReceipt, ...]


@dataclass(frozen=True)
class PrefillOutput:
    logits: torch.Tensor
    state: EngineState


@dataclass(frozen=True)
class DecodeReceipt:
    dense_attention_calls: int
    sparse_attention_calls: int
    dense_late_loop_calls: int
    selected_keys_per_layer: tuple[int, ...]


@dataclass(frozen=True)
class DecodeOutput:
    logits: torch.Tensor
    state: EngineState
    receipt: DecodeReceipt


@dataclass
class _LayerSource:
    """Loop-2 state reused by loops 3/4 (flashloop/engine.py:49-56)."""

    projected_output: torch.Tensor
    indices: torch.Tensor
    valid: torch.Tensor
    global_mass: torch.Tensor
    selected_weights: torch.Tensor
    current_value: torch.Tensor
    selected_output: torch.Tensor | None = None
    counts: torch.Tensor | None = None  # selected slots per row (the sparse readers skip the padding)


def _budget(tokens: int, fraction: float) -> int:
    return max(1, math.ceil(tokens * fraction))


@dataclass
class _PrefillLoops:
    keys: list  # [loop][layer] -> [1, H, T, 128] bf16
    values: list
    mask3: torch.Tensor  # [1, T] bool
    mask4: torch.Tensor
    receipts: tuple
    logits: torch.Tensor  # [1, vocab] f32 (or [1, T, vocab] with all_logits)


class DecodeRunner:
    """Runs decode steps of one engine's ``_decode_core``: eagerly, or replayed from a HIP
    graph captured per regime (the per-layer launches of a step become one graph
    launch).  The regime is every host value the captured step depends on -- the cache
    object, the batch, the selection capacity (steps every 64 selected keys) and the
    logits stride; a change recaptures.  Lengths live on the device and kernel grids are
    sized from capacities, so a rollover (which rewrites the cache between steps) does
    not."""

    def __init__(self, engine: "FlashLoopEngine", use_graphs: bool) -> None:
        # a weak back-reference: the engine and its runner form no cycle, so a dropped
        # engine frees its graph at once instead of in some later garbage collection,
        # which may run inside another graph's capture (where destroying a graph aborts)
        self._engine = weakref.ref(engine)
        self.use_graphs = bool(use_graphs)
        self.graph = None
        self.captures = 0  # graphs captured so far
        self.reset()

    @property
    def engine(self) -> "FlashLoopEngine":
        eng = self._engine()
        if eng is None:
            raise RuntimeError("the engine of this decode runner no longer exists")
        return eng

    def _release(self) -> None:
        """Destroy the captured graph and its private memory pool, here and now (never
        inside a capture).  Nothing outside this runner holds a tensor of that pool: the
        step's logits are copied, inside the graph, into ``out``, an ordinary allocation."""
        self.logits = None
        if self.graph is not None:
            self.graph.reset()
        self.graph = None
        self.key = None

    def reset(self) -> None:
        self._release()
        self.tok = self.pos = self.out = None

    def _key(self, cache: CrossLoopKVCache, bsz: int) -> tuple:
        lc = cache.layers[0]
        cap = kernels.decode_capacity(lc.token_count + 1, self.engine.config.effective_decode_key_fraction)
        return (id(cache), bsz, cap, lc.logits_capacity())

    def step(self, cache: CrossLoopKVCache, token_ids: torch.Tensor, positions: Sequence[int]) -> torch.Tensor:
        """Logits ``[B, vocab]`` of one step; the caller then commits the appends
        (``commit_append`` on every layer)."""
        eng = self.engine
        bsz = token_ids.shape[0]
        dev = token_ids.device
        if not self.use_graphs:
            pos_t = torch.tensor([[int(p)] for p in positions], dtype=torch.long, device=dev)
            return eng._decode_core(cache, eng.backbone.embed_tokens(token_ids), pos_t)
        if self.tok is None or self.tok.shape[0] != bsz:
            self._release()
            self.tok = torch.zeros((bsz, 1), dtype=torch.long, device=dev)
            self.pos = torch.zeros((bsz, 1), dtype=torch.long, device=dev)
            self.out = torch.empty((bsz, eng.model.config.vocab_size), dtype=torch.float32, device=dev)
        self.tok.copy_(token_ids)
        if bsz == 1:
            self.pos.fill_(int(positions[0]))
        else:
            self.pos.copy_(torch.tensor([[int(p)] for p in positions], dtype=torch.long), non_blocking=False)
        key = self._key(cache, bsz)
        if self.graph is None or self.key != key:
            self._release()
            self._capture(cache)
            self.key = key
        self.graph.replay()
        return self.out

    def _capture(self, cache: CrossLoopKVCache) -> None:
        """A warm-up run on a side stream first sizes every workspace and library handle;
        its append is then undone on the device (the replay rewrites the same rows)."""
        eng = self.engine
        side = torch.cuda.Stream()  # default priority
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            eng._decode_core(cache, eng.backbone.embed_tokens(self.tok), self.pos)
            for lc in cache.layers:
                lc.tail_tokens -= 1
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        # A graph destroyed while a stream captures aborts the process, so no garbage
        # collection may run during the capture (one triggered by the capture's own
        # allocations could free an unreachable object that owns a graph).
        was_enabled = gc.isenabled()
        gc.disable()
        try:
            with torch.cuda.graph(graph):
                self.logits = eng._decode_core(cache, eng.backbone.embed_tokens(self.tok), self.pos)
                self.out.copy_(self.logits)
        finally:
            if was_enabled:
                gc.enable()
        self.graph = graph
        self.captures += 1


class FlashLoopEngine:
    """FlashLoop inference over an Ouro-shaped looped decoder, batch one."""

    def __init__(self, model: OuroForCausalLM, *, config: FlashLoopConfig | None = None,
                 use_graphs: bool = True) -> None:
        validate_ouro_model(model)
        self.model = model.eval()
        self.config = config or FlashLoopConfig()
        self.backbone = model.model
        self.layers = model.model.layers
        self._state: EngineState | None = None
        self.observer: Callable[[str, dict], None] | None = None
        self._runner = DecodeRunner(self, use_graphs)
        # decode-step model ops on the fused HIP kernels (False: torch modules)
        self.fused_decode = True
        # with fused_decode: each residual/norm chain runs in the prologue of the GEMV that
        # consumes it (False: separate fl_norm_chain launches; same results bit for bit)
        self.fused_chain = True
        self._wcache = None

    @classmethod
    def from_pretrained(cls, model_path: str, *, config: FlashLoopConfig | None = None,
                        torch_dtype: torch.dtype = torch.bfloat16, device="cuda") -> "FlashLoopEngine":
        """Load weights written by ``OuroForCausalLM.save_pretrained`` (flashloop/engine.py:134-150)."""
        return cls(OuroForCausalLM.from_pretrained(model_path, dtype=torch_dtype, device=device), config=config)

    @classmethod
    def from_random_init(cls, model_config: OuroConfig, *, seed: int = 0, config: FlashLoopConfig | None = None,
                         device="cuda") -> "FlashLoopEngine":
        return cls(OuroForCausalLM.random_init(model_config, seed=seed, device=device), config=config)

    @property
    def state(self) -> EngineState:
        if self._state is None:
            raise RuntimeError("engine cache is not initialized")
        return self._state

    @property
    def use_graphs(self) -> bool:
        """Decode steps replay a captured HIP graph (True) or launch eagerly (False)."""
        return self._runner.use_graphs

    @use_graphs.setter
    def use_graphs(self, on: bool) -> None:
        self._runner.use_graphs = bool(on)
        self._runner.reset()

    def reset(self) -> None:
        self._state = None
        self._runner.reset()

    # ------------------------------------------------------------------ prefill
    def _qkv(self, attn, x: torch.Tensor):
        """q, k, v ``[B, heads, S, head_dim]`` of hidden rows ``x`` ``[B, S, hidden]``."""
        bsz, rows = x.shape[0], x.shape[1]
        q = attn.q_proj(x).view(bsz, rows, -1, attn.head_dim).transpose(1, 2)
        k = attn.k_proj(x).view(bsz, rows, -1, attn.head_dim).transpose(1, 2)
        v = attn.v_proj(x).view(bsz, rows, -1, attn.head_dim).transpose(1, 2)
        return q, k, v

    def _dense_loop(self, hidden: torch.Tensor, cos, sin):
        """``dense_prefill_loop`` (flashloop/prefill.py:275-304): every row, causal SDPA."""
        t = hidden.shape[1]
        keys, values = [], []
        h = hidden
        for layer in self.layers:
            a = layer.self_attn
            q, k, v = self._qkv(a, layer.input_layernorm(h))
            q, k = apply_rope(q, k, cos, sin)
            o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
            o = a.o_proj(o.transpose(1, 2).reshape(1, t, -1))
            h = h + layer.input_layernorm_2(o)
            h = h + layer.post_attention_layernorm_2(layer.mlp(layer.post_attention_layernorm(h)))
            keys.append(k.contiguous())
            values.append(v.contiguous())
        return self.backbone.norm(h), keys, values

    def _sparse_loop(self, hidden: torch.Tensor, positions: torch.Tensor, prev_keys, prev_values, cos, sin):
        """``sparse_prefill_loop`` (flashloop/prefill.py:122-272): only the active rows are
        recomputed; their K/V replace the previous loop's rows of a composite cache."""
        t = hidden.shape[1]
        n = positions.numel()
        h = hidden.clone()
        cos_a = cos.index_select(1, positions.long())
        sin_a = sin.index_select(1, positions.long())
        qpos = positions.long()
        allowed = torch.arange(t, device=h.device)[None, :] <= qpos[:, None]  # [n, T]
        keys, values = [], []
        for li, layer in enumerate(self.layers):
            a = layer.self_attn
            active, _ = kernels.gather_rows(h, positions, dim=1)
            q, k, v = self._qkv(a, layer.input_layernorm(active))
            q, k = apply_rope(q, k, cos_a, sin_a)
            full_k = prev_keys[li].clone()
            full_v = prev_values[li].clone()
            kernels.scatter_rows_(full_k, positions, k.contiguous(), dim=2)
            kernels.scatter_rows_(full_v, positions, v.contiguous(), dim=2)
            o = F.scaled_dot_product_attention(q, full_k, full_v, attn_mask=allowed[None, None])
            o = a.o_proj(o.transpose(1, 2).reshape(1, n, -1))
            active = active + layer.input_layernorm_2(o)
            active = active + layer.post_attention_layernorm_2(layer.mlp(layer.post_attention_layernorm(active)))
            kernels.scatter_rows_(h, positions, active.contiguous(), dim=1)
            keys.append(full_k)
            values.append(full_v)
        # final norm on the active rows only (flashloop/prefill.py:254-256)
        act, _ = kernels.gather_rows(h, positions, dim=1)
        kernels.scatter_rows_(h, positions, self.backbone.norm(act).contiguous(), dim=1)
        return h, keys, values

    def _select(self, current, previous, fraction, eligible=None):
        score = kernels.hidden_delta_score(current, previous)
        mask, positions, counts, err = kernels.select_tokens(score, fraction, eligible=eligible)
        n = int(counts[0].item())  # prefill syncs once per loop boundary, as the reference does
        return mask, positions[0, :n].contiguous(), score

    def _prefill_loops(self, input_ids: torch.Tensor, stage: Callable[[str], None] = lambda _n: None,
                       all_logits: bool = False) -> "_PrefillLoops":
        """The four prefill loops of one sequence ``[1, T]`` (flashloop/engine.py:176-333):
        dense loops 1-2, then token-sparse loops 3-4 on the rows selected by the hidden
        delta score.  Returns every layer's K/V of every loop, the masks and the logits."""
        t = int(input_ids.shape[1])
        dev = input_ids.device
        hidden = self.backbone.embed_tokens(input_ids)
        cos, sin = self.backbone.rotary_emb(hidden, torch.arange(t, device=dev)[None])
        stage("inputs_ready")
        h1, k1, v1 = self._dense_loop(hidden, cos, sin)
        stage("loop1_dense")
        h2, k2, v2 = self._dense_loop(h1, cos, sin)
        stage("loop2_dense")
        f3, f4 = self.config.effective_prefill_fractions
        mask3, pos3, _ = self._select(h2, h1, f3)
        h3, k3, v3 = self._sparse_loop(h2, pos3, k2, v2, cos, sin)
        stage("loop3_sparse")
        mask4, pos4, _ = self._select(h3, h2, f4, eligible=mask3)
        h4, k4, v4 = self._sparse_loop(h3, pos4, k3, v3, cos, sin)
        stage("loop4_sparse")
        receipts = (PrefillReceipt(1, t, t), PrefillReceipt(2, t, t), PrefillReceipt(3, t, pos3.numel()),
                    PrefillReceipt(4, t, pos4.numel()))
        logits = self.model.lm_head(h4 if all_logits else h4[:, -1]).float()
        return _PrefillLoops([k1, k2, k3, k4], [v1, v2, v3, v4], mask3, mask4, receipts, logits)

    @torch.inference_mode()
    def prefill(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None, *,
                decode_capacity: int | None = None,
                stage_observer: Callable[[str], None] | None = None, all_logits: bool = False) -> PrefillOutput:
        """``FlashLoopEngine.prefill`` (flashloop/engine.py:161-344).  ``all_logits`` returns
        the logits of every prompt position ``[1, T, vocab]`` instead of the last one."""

        def stage(name: str) -> None:
            if stage_observer is not None:
                stage_observer(name)

        stage("start")
        if self._state is not None:
            raise RuntimeError("engine cache is already initialized; call reset()")
        if input_ids.ndim != 2 or input_ids.shape[0] != 1:
            raise ValueError("the engine supports batch size one")
        t = int(input_ids.shape[1])
        if t <= 0:
            raise ValueError("prefill requires at least one prompt token")
        if attention_mask is not None and (attention_mask.shape != input_ids.shape or not bool(attention_mask.bool().all())):
            raise ValueError("padding is not supported by the batch-one engine")
        loops = self._prefill_loops(input_ids, stage, all_logits=all_logits)
        cap = t + (self.config.decode_capacity if decode_capacity is None else int(decode_capacity))
        cache = CrossLoopKVCache(num_layers=len(self.layers))
        for li in range(len(self.layers)):
            cache.set_layer(li, CrossLoopKVLayer.from_prefill(
                [k[li] for k in loops.keys], [v[li] for v in loops.values],
                mask_loop3=loops.mask3, mask_loop4=loops.mask4, token_capacity=cap))
        stage("physical_cache_finalized")
        self._state = EngineState(cache, t, loops.mask3, loops.mask4, loops.receipts)
        self._runner.reset()  # a new cache: captured pointers are stale
        logits = loops.logits
        stage("logits_ready")
        return PrefillOutput(logits=logits, state=self._state)

    # ------------------------------------------------------------------ decode
    def _decode_core(self, cache: CrossLoopKVCache, h: torch.Tensor, pos_t: torch.Tensor) -> torch.Tensor:
        """One decode step (see ``_decode_core_fused``); the torch-module form runs when the
        fused kernels do not apply (``fused_decode`` off, non-bf16 weights, batch > 8)."""
        if self.fused_decode and h.shape[0] <= 8 and self._fused_weights() is not None:
            return self._decode_core_fused(cache, h, pos_t)
        return self._decode_core_modules(cache, h, pos_t)

    def _fused_weights(self):
        """Per-layer weight tensors of the fused decode path, or None when a weight is not a
        contiguous bf16 device tensor."""
        if self._wcache is None:
            def ok(t):
                return t.dtype == torch.bfloat16 and t.is_cuda and t.is_contiguous()

            layers = []
            for layer in self.layers:
                a, m = layer.self_attn, layer.mlp
                w = dict(q=a.q_proj.weight, k=a.k_proj.weight, v=a.v_proj.weight, o=a.o_proj.weight,
                         gate=m.gate_proj.weight, up=m.up_proj.weight, down=m.down_proj.weight,
                         ln1=layer.input_layernorm.weight, ln2=layer.input_layernorm_2.weight,
                         ln3=layer.post_attention_layernorm.weight, ln4=layer.post_attention_layernorm_2.weight)
                if not all(ok(t) for t in w.values()) or a.num_key_value_heads != a.num_heads:
                    self._wcache = False
                    return None
                layers.append(w)
            extra = dict(norm=self.backbone.norm.weight, lm_head=self.model.lm_head.weight)
            self._wcache = (layers, extra) if all(ok(t) for t in extra.values()) else False
        return self._wcache or None

    def _decode_core_fused(self, cache: CrossLoopKVCache, h: torch.Tensor, pos_t: torch.Tensor) -> torch.Tensor:
        """The step of ``_decode_core_modules`` on the fused decode kernels: per layer and
        loop one q/k/v GEMV with RoPE, the cache readers, one o_proj GEMV (+ the loop-2
        projection for loops 3/4), one residual/norm chain, one SwiGLU GEMV, one down GEMV
        and one chain that also applies the next layer's input norm (and the final norm at
        the end of a loop).  Each op rounds to bf16 where the torch modules do."""
        cfg = self.config
        sparse = cfg.enable_sparse_decode
        fraction = cfg.effective_decode_key_fraction
        eps = float(self.model.config.rms_norm_eps)
        layers_w, extra = self._fused_weights()
        bsz = h.shape[0]
        nl = len(self.layers)
        heads, hd = self.layers[0].self_attn.num_heads, self.layers[0].self_attn.head_dim
        cos, sin = self.backbone.rotary_emb(h, pos_t)
        rope = (cos.reshape(bsz, hd), sin.reshape(bsz, hd))
        hid = h.reshape(bsz, -1)
        chained = self.fused_chain
        # the chain whose output feeds the next GEMV: kwargs of norm_chain (h = hid + n_a(x),
        # optional final norm, z = n_b(h)); it runs inside that GEMV when chained
        pending = dict(w_b=layers_w[0]["ln1"])
        first = True

        def chain_gemv(weights, **gk):
            nonlocal hid, first
            if chained:
                h_new, y = kernels.gemv_chain(hid, weights, eps=eps, want_h=not first, **pending, **gk)
            else:
                h_new, z = kernels.norm_chain(hid, eps=eps, want_h=not first, **pending)
                y = kernels.gemv(h_new if pending.get("w_b") is None else z, weights, **gk)
            if not first:
                hid = h_new
            first = False
            return y

        cur_k = [[None] * 4 for _ in range(nl)]
        cur_v = [[None] * 4 for _ in range(nl)]
        sources: list[_LayerSource | None] = [None] * nl
        for loop in range(4):
            for li, layer in enumerate(self.layers):
                w = layers_w[li]
                a = layer.self_attn
                q, k, v = chain_gemv([w["q"], w["k"], w["v"]], epilogue=kernels.EPI_ROPE, rope=rope, head_dim=hd)
                q, k, v = (t.view(bsz, heads, 1, hd) for t in (q, k, v))
                cur_k[li][loop] = k
                cur_v[li][loop] = v
                lc = cache.layers[li]
                if loop < 2 or not sparse:
                    if loop == 1 and sparse:  # read, merge and loop-2 selection: two launches
                        out, lg, (idx, valid, mass, sw, cnt) = lc.dense_source_attention_select(
                            loop, query=q, current_key=k, current_value=v, scaling=a.scaling, fraction=fraction)
                    else:
                        out, _ = lc.dense_source_attention(loop, query=q, current_key=k, current_value=v,
                                                           scaling=a.scaling, return_logits=False)
                    projected = kernels.gemv(out.reshape(bsz, -1), [w["o"]])
                    if loop == 1 and sparse:
                        sources[li] = _LayerSource(projected, idx, valid, mass, sw, v, counts=cnt)
                else:
                    src = sources[li]
                    if src.selected_output is None:
                        delta, so = lc.cached_mass_sparse_attention_delta_with_source(
                            loop, query=q, current_key=k, current_value=v, indices=src.indices, valid=src.valid,
                            source_weights=src.selected_weights, source_current_value=src.current_value,
                            global_mass=src.global_mass, scaling=a.scaling, counts=src.counts)
                        src.selected_output = so
                    else:
                        delta = lc.cached_mass_sparse_attention_delta(
                            loop, query=q, current_key=k, current_value=v, indices=src.indices, valid=src.valid,
                            source_selected_output=src.selected_output, global_mass=src.global_mass,
                            scaling=a.scaling, counts=src.counts)
                    projected = kernels.gemv(delta.reshape(bsz, -1), [w["o"]], epilogue=kernels.EPI_ADD,
                                             addend=src.projected_output)
                pending = dict(x=projected, w_a=w["ln2"], w_b=w["ln3"])
                act = chain_gemv([w["gate"], w["up"]], epilogue=kernels.EPI_SWIGLU)
                mo = kernels.gemv(act, [w["down"]])
                last = li == nl - 1
                nxt = None if (last and loop == 3) else layers_w[(li + 1) % nl]["ln1"]
                pending = dict(x=mo, w_a=w["ln4"], w_f=extra["norm"] if last else None, w_b=nxt)
        for li in range(nl):
            cache.layers[li].append_rows(cur_k[li], cur_v[li])
        # the last chain (final norm, no input norm) feeds lm_head
        return chain_gemv([extra["lm_head"]], epilogue=kernels.EPI_F32)

    def _decode_core_modules(self, cache: CrossLoopKVCache, h: torch.Tensor, pos_t: torch.Tensor) -> torch.Tensor:
        """One decode step of ``B`` sequences on the device: every layer and loop, then the
        cache appends (device tail lengths, no host index).  ``h``: embedded tokens
        ``[B, 1, hidden]``; ``pos_t``: their positions ``[B, 1]`` on the device.  Returns
        the logits ``[B, vocab]``.  The only host value it reads that changes during decoding
        is the selection capacity (a step every 64 selected keys), so it can be captured."""
        cfg = self.config
        sparse = cfg.enable_sparse_decode
        fraction = cfg.effective_decode_key_fraction
        bsz = h.shape[0]
        cos, sin = self.backbone.rotary_emb(h, pos_t)
        nl = len(self.layers)
        cur_k = [[None] * 4 for _ in range(nl)]
        cur_v = [[None] * 4 for _ in range(nl)]
        sources: list[_LayerSource | None] = [None] * nl
        for loop in range(4):
            for li, layer in enumerate(self.layers):
                a = layer.self_attn
                residual = h
                q, k, v = self._qkv(a, layer.input_layernorm(h))
                q, k = apply_rope(q, k, cos, sin)
                q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
                cur_k[li][loop] = k
                cur_v[li][loop] = v
                lc = cache.layers[li]
                if loop < 2 or not sparse:
                    if loop == 1 and sparse:
                        out, lg, (idx, valid, mass, w, cnt) = lc.dense_source_attention_select(
                            loop, query=q, current_key=k, current_value=v, scaling=a.scaling, fraction=fraction)
                    else:
                        out, _ = lc.dense_source_attention(loop, query=q, current_key=k, current_value=v,
                                                           scaling=a.scaling, return_logits=False)
                    projected = a.o_proj(out.to(q.dtype).transpose(1, 2).reshape(bsz, 1, -1))
                    if loop == 1 and sparse:
                        sources[li] = _LayerSource(projected, idx, valid, mass, w, v, counts=cnt)
                else:
                    src = sources[li]
                    if src.selected_output is None:
                        delta, so = lc.cached_mass_sparse_attention_delta_with_source(
                            loop, query=q, current_key=k, current_value=v, indices=src.indices, valid=src.valid,
                            source_weights=src.selected_weights, source_current_value=src.current_value,
                            global_mass=src.global_mass, scaling=a.scaling, counts=src.counts)
                        src.selected_output = so
                    else:
                        delta = lc.cached_mass_sparse_attention_delta(
                            loop, query=q, current_key=k, current_value=v, indices=src.indices, valid=src.valid,
                            source_selected_output=src.selected_output, global_mass=src.global_mass,
                            scaling=a.scaling, counts=src.counts)
                    projected = src.projected_output + a.o_proj(
                        delta.to(v.dtype).transpose(1, 2).reshape(bsz, 1, -1))
                h = residual + layer.input_layernorm_2(projected)
                h = h + layer.post_attention_layernorm_2(layer.mlp(layer.post_attention_layernorm(h)))
            h = self.backbone.norm(h)
        for li in range(nl):
            cache.layers[li].append_rows(cur_k[li], cur_v[li])
        return self.model.lm_head(h[:, -1]).float()

    def _receipt(self, positions: Sequence[int]) -> DecodeReceipt:
        nl = len(self.layers)
        sparse = self.config.enable_sparse_decode
        fraction = self.config.effective_decode_key_fraction
        # keys selected per layer (of the first sequence; all layers select the same count)
        n = positions[0] + 1
        counts = (min(n, _budget(n, fraction)),) * nl if sparse else ()
        return DecodeReceipt(
            dense_attention_calls=(2 if sparse else 4) * nl,
            sparse_attention_calls=(2 if sparse else 0) * nl,
            dense_late_loop_calls=(0 if sparse else 2) * nl,
            selected_keys_per_layer=counts,
        )

    @torch.inference_mode()
    def decode(self, token_ids: torch.Tensor) -> DecodeOutput:
        """``FlashLoopEngine.decode`` (flashloop/engine.py:373-570).  With ``use_graphs`` the
        step replays a captured HIP graph (recaptured when the selection capacity changes
        its shapes); the returned logits then live in the runner's output buffer and are
        overwritten by the next step."""
        state = self.state
        if token_ids.shape != (1, 1):
            raise ValueError("decode requires exactly one token at batch size one")
        pos = state.next_position
        logits = self._runner.step(state.cache, token_ids, [pos])
        for lc in state.cache.layers:
            lc.commit_append()  # host mirrors; rolls a group out of full tails (outside any graph)
        self._state = EngineState(state.cache, pos + 1, state.mask_loop3, state.mask_loop4, state.prefill_receipts)
        return DecodeOutput(logits=logits, state=self._state, receipt=self._receipt([pos]))

    # ------------------------------------------------------------------ generate
    @torch.inference_mode()
    def generate(self, input_ids: torch.Tensor, *, max_new_tokens: int, eos_token_id: int | None = None,
                 stop_token_sequences: tuple[tuple[int, ...], ...] = ()) -> torch.Tensor:
        """Greedy generation (flashloop/engine.py:572-607).  The host reads each token back
        only when an EOS id or stop sequence has to be checked."""
        if int(max_new_tokens) <= 0:
            raise ValueError("max_new_tokens must be positive")
        if eos_token_id is None:
            eos_token_id = getattr(self.model.config, "eos_token_id", None)
        prefill = self.prefill(input_ids, decode_capacity=int(max_new_tokens) + 64)
        generated = [input_ids]
        logits = prefill.logits
        completion: list[int] = []
        check = eos_token_id is not None or bool(stop_token_sequences)
        for step in range(int(max_new_tokens)):
            nxt = torch.argmax(logits, dim=-1, keepdim=True)
            generated.append(nxt)
            if check:
                completion.append(int(nxt.item()))
                if eos_token_id is not None and completion[-1] == int(eos_token_id):
                    break
                if any(seq and len(completion) >= len(seq) and tuple(completion[-len(seq):]) == seq
                       for seq in stop_token_sequences):
                    break
            if step + 1 < int(max_new_tokens):
                logits = self.decode(nxt).logits
        return torch.cat(generated, dim=1)
