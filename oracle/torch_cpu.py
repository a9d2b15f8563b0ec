"""flashloop_torch's decode attention step of one layer, on torch-CPU.

Test infrastructure: the CPU baseline that ``bench.py`` times next to the HIP step
(and ``tests/test_oracle_torch_cpu.py`` checks against ``oracle/attention.py``).  It
restates the work a decode step of one layer costs in the reference's torch path, in
the reference's dtypes:

* every loop r: the cache update appends the current token to the materialised bf16
  K_r/V_r cache (flashloop_torch keeps the codec's reconstructions as the cache,
  ``flashloop_torch/kv_quantization.py:198-244``), then the HF eager attention
  computes the dense output: ``bf16(q.K^T) * scaling``, fp32 softmax cast to bf16,
  ``P.V`` in bf16;
* loop 2: the hook captures the source state, its top-k mask over the fp32 weights and
  the selected mass (``flashloop_torch/attention.py:297-317``,
  ``flashloop_torch/attention_utils.py:139-148, 196-213``);
* loops 3-4: the dense output is replaced by ``mass_scaled_sparse_output`` with the
  cached source mass (``flashloop_torch/attention.py:326-380``,
  ``attention_utils.py:151-166, 216-248``); the o_proj that follows is not part of the
  step (the HIP step ends before it too), so the delta before o_proj is returned.
"""

from __future__ import annotations

import math

import torch


def _subset_softmax(logits: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    p = torch.softmax(logits.float().masked_fill(~mask, -torch.inf), dim=-1)
    return p.masked_fill(~mask, 0)


def decode_layer_step(q, k_cur, v_cur, keys, values, scaling: float, fraction: float = 0.10):
    """``q``/``k_cur``/``v_cur``: 4 bf16 tensors ``[R, 1, C]`` (per loop); ``keys``/``values``:
    4 bf16 tensors ``[R, T, C]`` (the materialised cache of each loop).  Returns
    ``(out0, out1, delta2, delta3, mask, mass)``: the loop-1/2 attention outputs, the
    loop-3/4 mass-scaled deltas (fp32, before o_proj), the selection mask and mass."""
    outs = []
    src = None
    for r in range(4):
        kc = torch.cat([keys[r], k_cur[r]], dim=1)  # the cache update of the step
        vc = torch.cat([values[r], v_cur[r]], dim=1)
        logits = torch.matmul(q[r], kc.transpose(1, 2)) * scaling  # bf16 [R, 1, T+1]
        weights = torch.softmax(logits, dim=-1, dtype=torch.float32).to(q[r].dtype)
        out = torch.matmul(weights, vc)
        if r < 2:
            outs.append(out.float())
        if r == 1:
            keys_n = logits.shape[-1]
            k = min(keys_n, max(1, math.ceil(keys_n * fraction)))
            idx = torch.topk(weights.float(), k, dim=-1).indices
            mask = torch.zeros_like(logits, dtype=torch.bool).scatter_(-1, idx, True)
            mass = (torch.softmax(logits.float(), dim=-1) * mask).sum(dim=-1, keepdim=True)
            src = (logits, vc, mask, mass)
        elif r >= 2:
            s_logits, s_values, mask, mass = src
            target = torch.matmul(_subset_softmax(logits, mask), vc.float())
            source = torch.matmul(_subset_softmax(s_logits, mask), s_values.float())
            outs.append(target * mass - source * mass)
    return outs[0], outs[1], outs[2], outs[3], src[2], src[3]
