"""Physical anchor-plus-residual cross-loop KV cache of one layer, in HBM.

Mirrors ``CrossLoopKVLayer`` / ``CrossLoopKVCache`` (flashloop/cache.py:315-1950): the
same streams (int4 anchor, int4 loop-2 residual, int4 loop-3/4 residuals at their
active rows through rank maps), the same 64..127-token BF16 tail per loop, the same
rollover of one 64-token group when the tail reaches 128 rows, and the same reader
methods.  Differences, all deliberate:

* batched: ``[B, H]`` sequences, each with its own prefix/tail length (the reference
  is batch-one, flashloop/cache.py:270-271);
* metadata is float32 and loop-3/4 K residuals are grouped per logical 64-token group
  -- the arithmetic of flashloop_torch/kv_quantization.py:455-486, 531-650, so codes
  and reconstructions match the torch reference bit for bit;
* storage is token-major int4 rows (64 bytes per 128 channels) for every stream,
  read by the HIP kernels in libflashloop_amd.so; there is no torch or CPU path.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Sequence

import torch

from . import kernels
from ._lib import GROUP, HEAD_DIM, FlCacheView


def packed_prefix_tokens(tokens: int, group: int = GROUP, residual: int = 64) -> int:
    """Tokens held in packed streams (flashloop/cache.py:385-387)."""
    return max(0, ((int(tokens) - residual) // group) * group)


def _round_up(x: int, m: int) -> int:
    return (int(x) + m - 1) // m * m


@dataclass(frozen=True)
class LayerGeometry:
    batch: int
    heads: int
    token_capacity: int
    tail_capacity: int
    row_capacity: tuple[int, int, int, int]


class CrossLoopKVLayer:
    """One layer's packed recurrent cache for ``batch`` sequences of ``heads`` heads."""

    residual_length = 64
    group_size = GROUP

    def __init__(self, geometry: LayerGeometry, device) -> None:
        g = geometry
        if g.token_capacity % GROUP:
            raise ValueError("token_capacity must be a multiple of 64")
        if g.tail_capacity < self.residual_length + GROUP:
            raise ValueError("tail_capacity must hold 128 rows (residual + one group)")
        if min(g.row_capacity) < 1:
            # the readers read row 0 of a stream in place of an absent row (then mask it)
            raise ValueError("every stream needs a row capacity of at least 1")
        self.geometry = g
        self.device = torch.device(device)
        rows = g.batch * g.heads
        dev = self.device
        # one 128-byte line per token and stream: K codes in bytes 0..63, V codes in 64..127
        self.codes = [torch.zeros(rows, g.row_capacity[s], 2 * (HEAD_DIM // 2), dtype=torch.uint8, device=dev)
                      for s in range(4)]
        self.key_codes = [c[..., : HEAD_DIM // 2] for c in self.codes]
        self.value_codes = [c[..., HEAD_DIM // 2 :] for c in self.codes]
        self.key_meta = [torch.zeros(rows, g.token_capacity // GROUP, HEAD_DIM, 2, dtype=torch.float32, device=dev) for _ in range(4)]
        self.value_meta = [torch.zeros(rows, g.row_capacity[s], 2, 2, dtype=torch.float32, device=dev) for s in range(4)]
        # the V metadata of all four streams again, one 64-byte record per logical token
        # ([half][stream][scale, min]) for the readers of selected tokens
        self.value_meta_token = torch.zeros(rows, g.token_capacity, 2, 4, 2, dtype=torch.float32, device=dev)
        # fp16 copy of the K metadata, streamed by the readers of selected tokens
        self.key_meta_half = [torch.zeros(rows, g.token_capacity // GROUP, HEAD_DIM, 2, dtype=torch.float16, device=dev)
                              for _ in range(4)]
        self.value_meta_half = [torch.zeros(rows, g.row_capacity[s], 2, 2, dtype=torch.float16, device=dev)
                                for s in range(4)]
        self.rank = [torch.full((g.batch, g.token_capacity), -1, dtype=torch.int32, device=dev) for _ in range(2)]
        self.tail_key = [torch.zeros(rows, g.tail_capacity, HEAD_DIM, dtype=torch.bfloat16, device=dev) for _ in range(4)]
        self.tail_value = [torch.zeros(rows, g.tail_capacity, HEAD_DIM, dtype=torch.bfloat16, device=dev) for _ in range(4)]
        # loop-3/4 activity of tail rows (flashloop/cache.py:_tail_active)
        self.tail_active = [torch.zeros(g.batch, g.tail_capacity, dtype=torch.uint8, device=dev) for _ in range(2)]
        self.packed_tokens = torch.zeros(g.batch, dtype=torch.int32, device=dev)
        self.tail_tokens = torch.zeros(g.batch, dtype=torch.int32, device=dev)
        self.late_rows = torch.zeros(2, g.batch, dtype=torch.int32, device=dev)  # rows used in streams 2/3
        # host mirrors (no device sync on the decode path)
        self.packed_host = [0] * g.batch
        self.tail_host = [0] * g.batch
        # host mirror of late_rows, read back lazily: a rollover advances the device counts
        # without a sync and adds GROUP per rolled group to _late_pending, an upper bound
        # of what the mirror is missing (enough for the capacity check)
        self._late_rows_host = [[0] * g.batch, [0] * g.batch]
        self._late_pending = [[0] * g.batch, [0] * g.batch]
        self._late_stale = False
        self._view: FlCacheView | None = None
        self.workspace = kernels.Workspace()

    # ------------------------------------------------------------------ geometry
    @property
    def batch(self) -> int:
        return self.geometry.batch

    @property
    def heads(self) -> int:
        return self.geometry.heads

    @property
    def rows(self) -> int:
        return self.batch * self.heads

    @property
    def late_rows_host(self) -> list[list[int]]:
        """Rows used in streams 2/3 per sequence (host mirror of ``late_rows``)."""
        if self._late_stale:
            self._late_rows_host = [[int(x) for x in r] for r in self.late_rows.tolist()]
            self._late_pending = [[0] * self.batch, [0] * self.batch]
            self._late_stale = False
        return self._late_rows_host

    @late_rows_host.setter
    def late_rows_host(self, rows: list[list[int]]) -> None:
        self._late_rows_host = rows
        self._late_pending = [[0] * self.batch, [0] * self.batch]
        self._late_stale = False

    @property
    def quantized_tokens(self) -> int:
        return max(self.packed_host)

    @property
    def tail_tokens_max(self) -> int:
        return max(self.tail_host)

    @property
    def token_count(self) -> int:
        return max(p + t for p, t in zip(self.packed_host, self.tail_host))

    def view(self) -> FlCacheView:
        if self._view is None:
            g = self.geometry
            v = FlCacheView()
            v.batch, v.heads = g.batch, g.heads
            v.token_capacity, v.tail_capacity = g.token_capacity, g.tail_capacity
            for s in range(4):
                v.row_capacity[s] = g.row_capacity[s]
                v.key_codes[s] = self.key_codes[s].data_ptr()
                v.key_meta[s] = self.key_meta[s].data_ptr()
                v.value_codes[s] = self.value_codes[s].data_ptr()
                v.value_meta[s] = self.value_meta[s].data_ptr()
                v.tail_key[s] = self.tail_key[s].data_ptr()
                v.tail_value[s] = self.tail_value[s].data_ptr()
            v.rank[0], v.rank[1] = self.rank[0].data_ptr(), self.rank[1].data_ptr()
            v.value_meta_token = self.value_meta_token.data_ptr()
            for s in range(4):
                v.key_meta_half[s] = self.key_meta_half[s].data_ptr()
                v.value_meta_half[s] = self.value_meta_half[s].data_ptr()
            v.packed_tokens = self.packed_tokens.data_ptr()
            v.tail_tokens = self.tail_tokens.data_ptr()
            self._view = v
        self._view.max_packed_tokens = self.quantized_tokens
        self._view.max_tail_tokens = self.tail_tokens_max
        return self._view

    # ------------------------------------------------------------------ construction
    @classmethod
    def from_prefill(
        cls,
        keys: Sequence[torch.Tensor],
        values: Sequence[torch.Tensor],
        *,
        mask_loop3: torch.Tensor | None = None,
        mask_loop4: torch.Tensor | None = None,
        lengths: Sequence[int] | None = None,
        token_capacity: int | None = None,
        recon: bool = False,
    ) -> "CrossLoopKVLayer":
        """Pack a prefill's four loop K/V ``[B, H, T, 128]`` bf16 (``CrossLoopKVLayer.from_prefill``,
        flashloop/cache.py:752-817; codec of kv_quantization.py:531-650).

        ``mask_loop3/4``: ``[B, T]`` bool rows recomputed in loops 3/4 (None = all rows);
        ``lengths``: per-sequence token counts for ragged batches (rows beyond are padding);
        ``token_capacity``: packed-prefix capacity (room for decode rollover).
        With ``recon=True`` the reconstructed prefixes R_r are returned as
        ``layer.recon_keys/recon_values`` (bf16 ``[B*H, T, 128]``) for audits.
        """
        if len(keys) != 4 or len(values) != 4:
            raise ValueError("exactly four loop K/V tensors are required")
        b, h, t, c = keys[0].shape
        if c != HEAD_DIM:
            raise ValueError("head_dim must be 128")
        for x in (*keys, *values):
            if tuple(x.shape) != (b, h, t, c) or x.dtype != torch.bfloat16 or not x.is_cuda:
                raise ValueError("loop K/V must be bf16 device tensors of one shape [B, H, T, 128]")
        lengths = [t] * b if lengths is None else [int(x) for x in lengths]
        if len(lengths) != b or any(x <= 0 or x > t for x in lengths):
            raise ValueError("lengths must give 1..T tokens per sequence")
        dev = keys[0].device
        masks = []
        for m in (mask_loop3, mask_loop4):
            if m is None:
                masks.append(torch.ones(b, t, dtype=torch.bool, device=dev))
            else:
                if tuple(m.shape) != (b, t):
                    raise ValueError("prefill masks must have shape [B, T]")
                masks.append(m.to(device=dev, dtype=torch.bool))
        if not bool(torch.all(~masks[1] | masks[0]).item()):
            raise ValueError("Loop-4 overrides must be nested in Loop-3 overrides")
        tp = [packed_prefix_tokens(x) for x in lengths]
        tp_max = max(tp)
        cap = _round_up(max(token_capacity or 0, tp_max, GROUP), GROUP)
        # loop-3/4 compact rows of the packed prefix: rank = running count of active rows
        pos = torch.arange(t, device=dev)
        tp_t = torch.tensor(tp, device=dev)
        prefix = pos[None, :] < tp_t[:, None]
        late_counts = []
        ranks = []
        for m in masks:
            act = m & prefix
            r = torch.cumsum(act.to(torch.int32), dim=1) - 1
            r = torch.where(act, r, torch.full_like(r, -1)).to(torch.int32)
            ranks.append(r)
            late_counts.append([int(x) for x in act.sum(dim=1).tolist()])
        growth = cap - min(tp)  # every future decode token is active in every loop
        row_cap = (cap, cap, max(max(late_counts[0]) + growth, 1), max(max(late_counts[1]) + growth, 1))
        layer = cls(LayerGeometry(b, h, cap, 2 * GROUP, row_cap), dev)
        for s in range(2):
            layer.rank[s][:, : min(t, cap)] = ranks[s][:, : min(t, cap)]
            layer.late_rows_host[s] = late_counts[s]
            layer.late_rows[s] = torch.tensor(late_counts[s], dtype=torch.int32, device=dev)
        layer.packed_host = list(tp)
        layer.tail_host = [x - p for x, p in zip(lengths, tp)]
        layer.packed_tokens.copy_(torch.tensor(tp, dtype=torch.int32))
        layer.tail_tokens.copy_(torch.tensor(layer.tail_host, dtype=torch.int32))
        if tp_max:
            src_k = [x.reshape(b * h, t, c) for x in keys]
            src_v = [x.reshape(b * h, t, c) for x in values]
            mk = [m.to(torch.uint8).contiguous() for m in masks]
            rk = rv = None
            if recon:
                rk = [torch.zeros(b * h, t, c, dtype=torch.bfloat16, device=dev) for _ in range(4)]
                rv = [torch.zeros(b * h, t, c, dtype=torch.bfloat16, device=dev) for _ in range(4)]
            kernels.pack_kv_groups(
                layer.view(), 4, [x.contiguous() for x in src_k], [x.contiguous() for x in src_v],
                src_bh_stride=t, src_row_offset=0,
                dst_group0=torch.zeros(b, dtype=torch.int32, device=dev), n_groups=tp_max // GROUP,
                masks=mk, mask_stride=t, recon_keys=rk, recon_values=rv,
            )
            if recon:
                layer.recon_keys, layer.recon_values = rk, rv
        # BF16 tails (flashloop/cache.py:806-812)
        for bi, (p, n) in enumerate(zip(tp, lengths)):
            rows = slice(bi * h, (bi + 1) * h)
            for r in range(4):
                layer.tail_key[r][rows, : n - p] = keys[r][bi, :, p:n]
                layer.tail_value[r][rows, : n - p] = values[r][bi, :, p:n]
            for s in range(2):
                layer.tail_active[s][bi, : n - p] = masks[s][bi, p:n].to(torch.uint8)
        return layer

    # ------------------------------------------------------------------ readers
    def logits_capacity(self) -> int:
        """Row stride of the logits buffer: the longest possible prefix plus a full tail and
        the current token (a constant of the layer, so a captured decode step keeps its
        buffers across rollovers), rounded up to 64 floats so that every row starts on a
        256-byte boundary."""
        n = self.geometry.token_capacity + self.geometry.tail_capacity + 1
        return (n + 63) // 64 * 64

    def dense_source_attention(self, loop: int, *, query, current_key, current_value, scaling: float,
                               return_logits: bool):
        """``CrossLoopKVLayer.dense_source_attention`` (flashloop/cache.py:1644-1756).

        Returns ``(out f32 [B,H,1,128], logits f32 [B,H,1,C] or None)``: logits row entries
        are valid up to each sequence's own ``T+1`` (C >= max T+1 is the padded stride)."""
        out, logits = kernels.fused_dense_source_attention(
            self.view(), int(loop), query, current_key, current_value, scaling, return_logits=return_logits,
            logits_capacity=self.logits_capacity(), device=self.device, workspace=self.workspace,
        )
        out = out.view(self.batch, self.heads, 1, HEAD_DIM)
        if logits is not None:
            logits = logits.view(self.batch, self.heads, 1, -1)
        return out, logits

    def dense_source_attention_pair(self, *, queries, current_keys, current_values, scaling: float):
        """Loops 1 and 2 of ``dense_source_attention`` (loop 2 with logits) in one reader
        launch (``fl_decode_attn_dense_pair``).  Returns ``(out loop 1, out loop 2, logits)``
        shaped as ``dense_source_attention`` returns them."""
        out0, out1, logits = kernels.fused_dense_pair(
            self.view(), queries, current_keys, current_values, scaling,
            logits_capacity=self.logits_capacity(), device=self.device, workspace=self.workspace)
        shape = (self.batch, self.heads, 1, HEAD_DIM)
        return out0.view(shape), out1.view(shape), logits.view(self.batch, self.heads, 1, -1)

    def dense_source_attention_select(self, loop: int, *, query, current_key, current_value, scaling: float,
                                      fraction: float):
        """``dense_source_attention(loop, ..., return_logits=True)`` followed by
        ``select_decode_keys(logits, fraction)`` (flashloop/engine.py:438-498), with the
        read's merge and the top-k in one launch when the row stride allows it
        (``fl_decode_attn_dense_select``).  Returns ``(out, logits, (indices, valid, mass,
        selected_weights, counts))`` shaped as the two methods return them."""
        cap = kernels.decode_capacity(self.token_count + 1, fraction)
        lcap = self.logits_capacity()
        if not kernels.dense_select_fits(lcap, fraction):
            out, logits = self.dense_source_attention(loop, query=query, current_key=current_key,
                                                      current_value=current_value, scaling=scaling, return_logits=True)
            return out, logits, self.select_decode_keys(logits, fraction)
        out, logits, idx, valid, mass, w, counts = kernels.fused_dense_select(
            self.view(), int(loop), query, current_key, current_value, scaling, fraction, cap,
            logits_capacity=lcap, device=self.device, workspace=self.workspace)
        shape = (self.batch, self.heads, cap)
        return (out.view(self.batch, self.heads, 1, HEAD_DIM), logits.view(self.batch, self.heads, 1, -1),
                (idx.view(shape), valid.view(shape), mass.view(self.batch, self.heads, 1, 1), w.view(shape), counts))

    def key_counts(self) -> torch.Tensor:
        """Keys per sequence including the current token: packed + tail + 1 (device)."""
        return self.packed_tokens + self.tail_tokens + 1

    def select_decode_keys(self, logits: torch.Tensor, fraction: float, validate: bool = False):
        """Loop-2 key selection (flashloop/engine.py:438-498) on the dense reader's logits.
        Returns ``(indices, valid, mass [B,H,1,1], selected_weights, counts)``.
        ``validate=True`` raises ``ValueError`` on NaN/inf logits (a host sync), as
        ``flashloop/selection.py:78-79`` does."""
        cap = kernels.decode_capacity(self.token_count + 1, fraction)
        idx, valid, mass, w, counts = kernels.decode_topk(
            logits.reshape(self.rows, -1), self.key_counts(), fraction, cap, rows_per_count=self.heads,
            validate=validate,
        )
        shape = (self.batch, self.heads, cap)
        return idx.view(shape), valid.view(shape), mass.view(self.batch, self.heads, 1, 1), w.view(shape), counts

    def _reader_counts(self, counts):
        """The selection counts handed to the sparse readers: only for a ragged batch.  With
        equal lengths every row's count is within 16 slots of the capacity, the padded
        partition is already balanced, and the live-tile prefix would only add its latency
        (a few microseconds per launch).  Lengths grow together during decode, so the choice
        holds for a captured step's replays; either choice gives the same results."""
        if counts is None:
            return None
        totals = [p + t for p, t in zip(self.packed_host, self.tail_host)]
        return counts if min(totals) != max(totals) else None

    def pv(self, loop: int, weights, indices, valid, current_value, counts=None):
        """``_selected_value_aggregate`` (flashloop/engine.py:346-371): sum of selected V rows
        of loop ``loop`` weighted by ``weights``; the current token reads ``current_value``.
        ``counts`` (optional, the selection's i32 ``[B*H]`` counts): every valid slot of a row
        lies below its count, so the reader skips the padding past it."""
        out = kernels.fused_cross_loop_pv(self.view(), int(loop), indices, valid, weights, current_value,
                                          device=self.device, workspace=self.workspace,
                                          counts=self._reader_counts(counts))
        return out.view(self.batch, self.heads, 1, HEAD_DIM)

    def cached_mass_sparse_attention_delta(self, loop: int, *, query, current_key, current_value, indices, valid,
                                           source_selected_output, global_mass, scaling: float, counts=None):
        """``CrossLoopKVLayer.cached_mass_sparse_attention_delta`` (flashloop/cache.py:1517-1617);
        ``counts`` as in ``pv``."""
        if int(loop) not in (2, 3):
            raise ValueError("cached-mass sparse attention is only valid for Loop 3/4")
        out = kernels.fused_sparse_attention_delta(
            self.view(), int(loop), query, current_key, current_value, indices, valid, source_selected_output,
            global_mass, scaling, device=self.device, workspace=self.workspace,
            counts=self._reader_counts(counts),
        )
        return out.view(self.batch, self.heads, 1, HEAD_DIM)

    def cached_mass_sparse_attention_delta_with_source(self, loop: int, *, query, current_key, current_value,
                                                       indices, valid, source_weights, source_current_value,
                                                       global_mass, scaling: float, counts=None):
        """Loop-3 form of ``cached_mass_sparse_attention_delta`` that also returns the loop-2
        selected aggregate (``_selected_value_aggregate``, flashloop/engine.py:346-371) from
        the same pass over the selected rows.  Returns ``(delta, source_output)``;
        ``counts`` as in ``pv``."""
        if int(loop) not in (2, 3):
            raise ValueError("cached-mass sparse attention is only valid for Loop 3/4")
        out, src = kernels.fused_sparse_attention_delta_with_source(
            self.view(), int(loop), query, current_key, current_value, indices, valid, source_weights,
            source_current_value, global_mass, scaling, device=self.device, workspace=self.workspace,
            counts=self._reader_counts(counts),
        )
        shape = (self.batch, self.heads, 1, HEAD_DIM)
        return out.view(shape), src.view(shape)

    # ------------------------------------------------------------------ decode append
    def append_decode_token(self, keys: Sequence[torch.Tensor], values: Sequence[torch.Tensor]) -> None:
        """``append_decode_token`` (flashloop/cache.py:1758-1776): write the step's four loop
        K/V rows (``[B,H,1,128]``) into the tails; roll a group out when a tail reaches 128."""
        self.append_rows(keys, values)
        self.commit_append()

    def append_rows(self, keys: Sequence[torch.Tensor], values: Sequence[torch.Tensor]) -> None:
        """Device half of an append: rows go to each sequence's device tail length, which is
        then incremented -- no host index, so the step can be captured in a HIP graph.
        ``commit_append`` must follow (host mirrors, rollover)."""
        if len(keys) != 4 or len(values) != 4:
            raise ValueError("exactly four loop K/V tensors are required")
        if any(t >= self.geometry.tail_capacity for t in self.tail_host):
            raise RuntimeError("tail is full; rollover did not run")
        kernels.append_tail(self.view(), keys, values, self.tail_active, self.tail_tokens)

    def commit_append(self) -> None:
        """Host half of an append: mirrors follow the device lengths; roll full tails."""
        self.tail_host = [x + 1 for x in self.tail_host]
        if any(x >= self.residual_length + GROUP for x in self.tail_host):
            self._roll_groups()

    def _roll_groups(self) -> None:
        """``_roll_one_group`` (flashloop/cache.py:1778-1838) for every sequence whose tail
        holds residual+group rows: pack tail rows [0, 64) as prefix group Tp/64, then shift
        the tail down by 64.  O(group): the prefix is never re-read.  Every step is a device
        op on device counts (no host read-back), unless the loop-3/4 row capacity could be
        exhausted, which is then checked exactly."""
        b, h = self.batch, self.heads
        dev = self.device
        roll = [x >= self.residual_length + GROUP for x in self.tail_host]
        for i in range(b):
            if roll[i] and self.packed_host[i] + GROUP > self.geometry.token_capacity:
                raise RuntimeError("packed prefix capacity exhausted; allocate a larger token_capacity")
        # every capacity check runs before the first device change, so a refused rollover
        # leaves the rank maps and device row counts as they were
        for s in range(2):
            cap = self.geometry.row_capacity[s + 2]
            for i in range(b):
                if roll[i] and self._late_rows_host[s][i] + self._late_pending[s][i] + GROUP > cap:
                    act_n = int(self.tail_active[s][i, :GROUP].sum().item())
                    if self.late_rows_host[s][i] + act_n > cap:  # exact (reads back)
                        raise RuntimeError("loop-3/4 row capacity exhausted")
        # rank maps of the new group's rows (active rows continue the compact numbering)
        for s in range(2):
            for i in range(b):
                if not roll[i]:
                    continue
                act = self.tail_active[s][i, :GROUP].bool()
                r = torch.cumsum(act.to(torch.int32), 0) - 1 + self.late_rows[s, i]
                p = self.packed_host[i]
                self.rank[s][i, p : p + GROUP] = torch.where(act, r, torch.full_like(r, -1))
                self.late_rows[s, i] += act.sum(dtype=torch.int32)
                self._late_pending[s][i] += GROUP
                self._late_stale = True
        dst = torch.full((b,), -1, dtype=torch.int32, device=dev)
        for i in range(b):
            if roll[i]:
                dst[i] = self.packed_host[i] // GROUP
        kernels.pack_kv_groups(
            self.view(), 4, self.tail_key, self.tail_value, src_bh_stride=self.geometry.tail_capacity,
            src_row_offset=0, dst_group0=dst, n_groups=1, masks=self.tail_active,
            mask_stride=self.geometry.tail_capacity,
        )
        for i in range(b):
            if not roll[i]:
                continue
            rows = slice(i * h, (i + 1) * h)
            n = self.tail_host[i] - GROUP
            # rows [GROUP, GROUP + n) -> [0, n): disjoint ranges (no copy first) when n <= GROUP
            def shift(src):
                return src if n <= GROUP else src.clone()
            for tensor in (*self.tail_key, *self.tail_value):
                tensor[rows, :n] = shift(tensor[rows, GROUP : GROUP + n])
            for act in self.tail_active:
                act[i, :n] = shift(act[i, GROUP : GROUP + n])
                act[i, n:] = 0
            self.packed_host[i] += GROUP
            self.tail_host[i] = n
            self.packed_tokens[i] += GROUP
            self.tail_tokens[i] -= GROUP

    # ------------------------------------------------------------------ serialization
    # On-disk format (FORMAT_NAME, FORMAT_VERSION): one safetensors file whose tensors are
    # the device buffers of the layer, byte for byte, under the names below (prefixed
    # "layer{i}." inside a CrossLoopKVCache file), and whose string metadata holds a JSON
    # header with the geometry and the host mirrors of the lengths:
    #   codes.{s}        u8   [B*H, row_capacity[s], 128]  K codes (bytes 0..63) | V codes (64..127)
    #   key_meta.{s}     f32  [B*H, token_capacity/64, 128, 2]  per-channel (scale, min) per group
    #   value_meta.{s}   f32  [B*H, row_capacity[s], 2, 2]  per-token (scale, min) per 64 channels
    #   value_meta_token f32  [B*H, token_capacity, 2, 4, 2]  the same per logical token, [half][stream]
    #   key_meta_half.{s} f16 [B*H, token_capacity/64, 128, 2]  key_meta rounded to fp16 (read by the readers)
    #   value_meta_half.{s} f16 [B*H, row_capacity[s], 2, 2]  value_meta rounded to fp16 (read by the dense readers)
    #   rank.{j}         i32  [B, token_capacity]  logical token -> row of stream 2+j, or -1
    #   tail_key.{r}     bf16 [B*H, tail_capacity, 128]  BF16 tail of loop r (tail_value likewise)
    #   tail_active.{j}  u8   [B, tail_capacity]  loop-3/4 activity of the tail rows
    #   packed_tokens / tail_tokens i32 [B], late_rows i32 [2, B]
    FORMAT_NAME = "flashloop_amd.cross_loop_kv"
    FORMAT_VERSION = 4

    def _named_tensors(self) -> dict[str, torch.Tensor]:
        named = {}
        for s in range(4):
            named[f"codes.{s}"] = self.codes[s]
            named[f"key_meta.{s}"] = self.key_meta[s]
            named[f"value_meta.{s}"] = self.value_meta[s]
            named[f"key_meta_half.{s}"] = self.key_meta_half[s]
            named[f"value_meta_half.{s}"] = self.value_meta_half[s]
            named[f"tail_key.{s}"] = self.tail_key[s]
            named[f"tail_value.{s}"] = self.tail_value[s]
        for j in range(2):
            named[f"rank.{j}"] = self.rank[j]
            named[f"tail_active.{j}"] = self.tail_active[j]
        named["value_meta_token"] = self.value_meta_token
        named["packed_tokens"] = self.packed_tokens
        named["tail_tokens"] = self.tail_tokens
        named["late_rows"] = self.late_rows
        return named

    def _header(self) -> dict:
        g = self.geometry
        return {
            "format": self.FORMAT_NAME, "version": self.FORMAT_VERSION,
            "batch": g.batch, "heads": g.heads, "head_dim": HEAD_DIM, "group_size": GROUP,
            "residual_length": self.residual_length, "token_capacity": g.token_capacity,
            "tail_capacity": g.tail_capacity, "row_capacity": list(g.row_capacity),
            "packed_tokens": list(self.packed_host), "tail_tokens": list(self.tail_host),
            "late_rows": [list(x) for x in self.late_rows_host],
        }

    def state_dict(self) -> tuple[dict[str, torch.Tensor], dict]:
        """(tensors, header) of the layer in the on-disk format above (tensors are the
        live buffers, not copies)."""
        return self._named_tensors(), self._header()

    @classmethod
    def from_state_dict(cls, tensors: dict[str, torch.Tensor], header: dict, device) -> "CrossLoopKVLayer":
        """Rebuild a layer from ``state_dict`` output; every shape and dtype is checked
        against the header before anything is copied."""
        if header.get("format") != cls.FORMAT_NAME:
            raise ValueError(f"not a {cls.FORMAT_NAME} payload")
        if int(header.get("version", -1)) != cls.FORMAT_VERSION:
            raise ValueError(f"unsupported format version {header.get('version')} (expected {cls.FORMAT_VERSION})")
        if int(header["head_dim"]) != HEAD_DIM or int(header["group_size"]) != GROUP \
                or int(header["residual_length"]) != cls.residual_length:
            raise ValueError("head_dim / group_size / residual_length differ from this build's")
        g = LayerGeometry(int(header["batch"]), int(header["heads"]), int(header["token_capacity"]),
                          int(header["tail_capacity"]), tuple(int(x) for x in header["row_capacity"]))
        layer = cls(g, device)
        want = layer._named_tensors()
        if set(tensors) != set(want):
            raise ValueError(f"tensor set differs: missing {sorted(set(want) - set(tensors))}, "
                             f"unexpected {sorted(set(tensors) - set(want))}")
        for name, dst in want.items():
            src = tensors[name]
            if tuple(src.shape) != tuple(dst.shape) or src.dtype != dst.dtype:
                raise ValueError(f"{name}: {tuple(src.shape)} {src.dtype} != {tuple(dst.shape)} {dst.dtype}")
            dst.copy_(src)
        layer.packed_host = [int(x) for x in header["packed_tokens"]]
        layer.tail_host = [int(x) for x in header["tail_tokens"]]
        layer.late_rows_host = [[int(x) for x in r] for r in header["late_rows"]]
        if len(layer.packed_host) != g.batch or len(layer.tail_host) != g.batch:
            raise ValueError("length mirrors do not match the batch")
        if [int(x) for x in layer.packed_tokens.tolist()] != layer.packed_host \
                or [int(x) for x in layer.tail_tokens.tolist()] != layer.tail_host:
            raise ValueError("device lengths disagree with the header")
        return layer

    def save(self, path: str) -> None:
        from safetensors.torch import save_file
        import json

        tensors, header = self.state_dict()
        save_file({k: v.contiguous() for k, v in tensors.items()}, path, metadata={"header": json.dumps(header)})

    @classmethod
    def load(cls, path: str, device="cuda") -> "CrossLoopKVLayer":
        from safetensors import safe_open
        import json

        with safe_open(path, framework="pt", device="cpu") as f:
            header = json.loads(f.metadata()["header"])
            tensors = {k: f.get_tensor(k) for k in f.keys()}
        return cls.from_state_dict(tensors, header, device)

    # ------------------------------------------------------------------ accounting
    @property
    def storage_bytes(self) -> int:
        """Bytes of the used part of every buffer (cf. flashloop/cache.py:1084-1112)."""
        b, h = self.batch, self.heads
        tot = 0
        for i in range(b):
            p = self.packed_host[i]
            rows = [p, p, self.late_rows_host[0][i], self.late_rows_host[1][i]]
            for s in range(4):
                tot += h * rows[s] * (64 + 64 + 16 + 8)  # K/V codes + V meta (f32 and f16)
                tot += h * (p // GROUP) * HEAD_DIM * 8  # K meta
            tot += h * p * 64  # per-token V metadata records
            tot += 4 * h * (p // GROUP) * HEAD_DIM * 4  # fp16 K metadata copies
            tot += 4 * 2 * h * self.tail_host[i] * HEAD_DIM * 2
            tot += 2 * p * 4  # rank maps
        return tot

    @property
    def dense_bf16_bytes(self) -> int:
        return 4 * 2 * self.heads * sum(p + t for p, t in zip(self.packed_host, self.tail_host)) * HEAD_DIM * 2


class CrossLoopKVCache:
    """Layer-indexed owner of physical cross-loop KV storage (flashloop/cache.py:1841-1950)."""

    def __init__(self, *, num_layers: int) -> None:
        if int(num_layers) <= 0:
            raise ValueError("num_layers must be positive")
        self.layers: list[CrossLoopKVLayer | None] = [None] * int(num_layers)

    def set_layer(self, layer_index: int, layer: CrossLoopKVLayer) -> None:
        if layer_index not in range(len(self.layers)):
            raise IndexError("layer index is outside the cache")
        if self.layers[layer_index] is not None:
            raise RuntimeError("physical cache layer is already installed")
        self.layers[layer_index] = layer

    def _require_layer(self, layer_index: int) -> CrossLoopKVLayer:
        if layer_index not in range(len(self.layers)):
            raise IndexError("layer index is outside the cache")
        layer = self.layers[layer_index]
        if layer is None:
            raise RuntimeError("physical cache layer has not been installed")
        return layer

    def dense_source_attention(self, layer_index: int, loop: int, **kwargs):
        return self._require_layer(layer_index).dense_source_attention(loop, **kwargs)

    def cached_mass_sparse_attention_delta(self, layer_index: int, loop: int, **kwargs):
        return self._require_layer(layer_index).cached_mass_sparse_attention_delta(loop, **kwargs)

    def pv(self, layer_index: int, loop: int, weights, indices, valid, current_value, counts=None):
        return self._require_layer(layer_index).pv(loop, weights, indices, valid, current_value, counts=counts)

    @property
    def storage_bytes(self) -> int:
        return sum(layer.storage_bytes for layer in self.layers if layer is not None)

    def save(self, path: str) -> None:
        """Every installed layer in one safetensors file (tensor names ``layer{i}.<name>``,
        per-layer headers in the metadata); see CrossLoopKVLayer for the tensor layout."""
        from safetensors.torch import save_file
        import json

        tensors, headers = {}, {}
        for i, layer in enumerate(self.layers):
            if layer is None:
                continue
            named, header = layer.state_dict()
            tensors.update({f"layer{i}.{k}": v.contiguous() for k, v in named.items()})
            headers[str(i)] = header
        meta = {"format": CrossLoopKVLayer.FORMAT_NAME, "version": CrossLoopKVLayer.FORMAT_VERSION,
                "num_layers": len(self.layers), "layers": headers}
        save_file(tensors, path, metadata={"header": json.dumps(meta)})

    @classmethod
    def load(cls, path: str, device="cuda") -> "CrossLoopKVCache":
        from safetensors import safe_open
        import json

        with safe_open(path, framework="pt", device="cpu") as f:
            meta = json.loads(f.metadata()["header"])
            if meta.get("format") != CrossLoopKVLayer.FORMAT_NAME:
                raise ValueError(f"not a {CrossLoopKVLayer.FORMAT_NAME} file")
            cache = cls(num_layers=int(meta["num_layers"]))
            for key, header in meta["layers"].items():
                i = int(key)
                pre = f"layer{i}."
                tensors = {k[len(pre):]: f.get_tensor(k) for k in f.keys() if k.startswith(pre)}
                cache.set_layer(i, CrossLoopKVLayer.from_state_dict(tensors, header, device))
        return cache


@dataclass
class AttentionStep:
    out0: torch.Tensor
    out1: torch.Tensor
    logits1: torch.Tensor
    indices: torch.Tensor
    valid: torch.Tensor
    mass: torch.Tensor
    selected_weights: torch.Tensor
    counts: torch.Tensor
    selected_output: torch.Tensor
    delta2: torch.Tensor
    delta3: torch.Tensor


def decode_attention_step(layer: CrossLoopKVLayer, queries, keys, values, scaling: float,
                          fraction: float = 0.10, fused_source: bool = True,
                          paired_dense: bool = False) -> AttentionStep:
    """One layer's decode attention over four loops (flashloop/engine.py:422-531, before
    ``o_proj``): dense loops 1-2 (loop 2 with logits), loop-2 key selection and selected
    aggregate, then the cached-mass deltas of loops 3-4.  ``queries/keys/values``: four
    bf16 ``[B,H,1,128]`` (the current token of each loop).

    With ``fused_source`` the loop-2 selected aggregate is formed by the loop-3 reader
    from the rows it reads anyway (it is first consumed there, engine.py:511-528);
    otherwise it is a separate selected-PV pass at loop 2, as in the reference.  With
    ``paired_dense`` the two dense loops share one reader launch; that needs both loops'
    queries at once, which a looped model's decode (every layer of loop 1 before loop 2,
    flashloop/engine.py:393-394) never has."""
    if paired_dense:
        out0, out1, logits = layer.dense_source_attention_pair(
            queries=queries[:2], current_keys=keys[:2], current_values=values[:2], scaling=scaling)
        idx, valid, mass, w, counts = layer.select_decode_keys(logits, fraction)
    else:
        out0, _ = layer.dense_source_attention(0, query=queries[0], current_key=keys[0], current_value=values[0],
                                               scaling=scaling, return_logits=False)
        out1, logits, (idx, valid, mass, w, counts) = layer.dense_source_attention_select(
            1, query=queries[1], current_key=keys[1], current_value=values[1], scaling=scaling, fraction=fraction)
    if fused_source:
        d2, so = layer.cached_mass_sparse_attention_delta_with_source(
            2, query=queries[2], current_key=keys[2], current_value=values[2], indices=idx, valid=valid,
            source_weights=w, source_current_value=values[1], global_mass=mass, scaling=scaling, counts=counts)
    else:
        so = layer.pv(1, w, idx, valid, values[1], counts=counts)
        d2 = layer.cached_mass_sparse_attention_delta(2, query=queries[2], current_key=keys[2],
                                                      current_value=values[2], indices=idx, valid=valid,
                                                      source_selected_output=so, global_mass=mass, scaling=scaling,
                                                      counts=counts)
    d3 = layer.cached_mass_sparse_attention_delta(3, query=queries[3], current_key=keys[3], current_value=values[3],
                                                  indices=idx, valid=valid, source_selected_output=so,
                                                  global_mass=mass, scaling=scaling, counts=counts)
    return AttentionStep(out0, out1, logits, idx, valid, mass, w, counts, so, d2, d3)
