"""Seeded synthetic decode workloads (the input definition of the benchmark configs).

One ``torch.Generator`` per workload, seeded with the config index:
``L1 = bf16(N(0,1))``, ``L_r = bf16(fp32(L_{r-1}) + drift*N(0,1))`` for loops 2..4, for K
and V independently; queries ``bf16(N(0,1))`` per loop; the current token's K/V of
each loop is position ``T`` of the same chain.  ``scaling = 128**-0.5``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

HEAD_DIM = 128
SCALING = HEAD_DIM ** -0.5


def loop_chain(gen: torch.Generator, shape, *, drift: float = 0.1, loops: int = 4, device="cpu"):
    first = torch.randn(shape, generator=gen, device=device).to(torch.bfloat16)
    out = [first]
    for _ in range(1, loops):
        step = torch.randn(shape, generator=gen, device=device)
        out.append((out[-1].float() + drift * step).to(torch.bfloat16))
    return out


@dataclass
class DecodeWorkload:
    keys: list  # 4 x bf16 [B, H, T+extra, 128]: positions < T_b are the cache, T_b is current
    values: list
    queries: list  # 4 x bf16 [B, H, 1, 128]
    lengths: list  # per sequence cached tokens T_b
    scaling: float = SCALING

    def current(self, loop: int):
        """(k_cur, v_cur) ``[B, H, 1, 128]`` of one loop: position T_b of each sequence."""
        b = len(self.lengths)
        idx = torch.tensor(self.lengths, device=self.keys[0].device)
        ar = torch.arange(b, device=self.keys[0].device)
        k = self.keys[loop][ar, :, idx].unsqueeze(2)
        v = self.values[loop][ar, :, idx].unsqueeze(2)
        return k.contiguous(), v.contiguous()

    def cache(self, loop: int):
        """Cached K/V ``[B, H, Tmax, 128]`` (rows >= T_b are padding)."""
        t = max(self.lengths)
        return self.keys[loop][:, :, :t].contiguous(), self.values[loop][:, :, :t].contiguous()


def decode_workload(batch: int, heads: int, tokens: int, *, seed: int, lengths=None, device="cpu",
                    drift: float = 0.1, extra: int = 1) -> DecodeWorkload:
    """Workload of ``batch`` sequences with ``tokens`` cached keys (or per-sequence
    ``lengths``) plus ``extra`` future positions (the first is the current token)."""
    gen = torch.Generator(device=device).manual_seed(int(seed))
    lengths = [int(tokens)] * batch if lengths is None else [int(x) for x in lengths]
    t = max(lengths) + extra
    shape = (batch, heads, t, HEAD_DIM)
    keys = loop_chain(gen, shape, drift=drift, device=device)
    values = loop_chain(gen, shape, drift=drift, device=device)
    queries = [torch.randn((batch, heads, 1, HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
               for _ in range(4)]
    return DecodeWorkload(keys, values, queries, lengths)


def ragged_lengths(batch: int, low: int, high: int, *, seed: int) -> list[int]:
    """Per-sequence context lengths drawn uniformly from [low, high] (seeded)."""
    gen = torch.Generator().manual_seed(int(seed))
    return [int(x) for x in torch.randint(low, high + 1, (batch,), generator=gen).tolist()]
