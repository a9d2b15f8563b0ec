"""The torch-CPU step that bench.py times as its CPU baseline computes the same decode
step as the float64 oracle (within the bf16 arithmetic the reference's torch path uses:
bf16 logits and bf16 probabilities)."""

import numpy as np
import torch

from oracle import attention as OA
from oracle import torch_cpu
from flashloop_amd.synthetic import SCALING, decode_workload


def test_torch_cpu_step_matches_oracle_step():
    R, T = 6, 700
    w = decode_workload(1, R, T, seed=17)
    keys = [w.keys[r][0, :, :T] for r in range(4)]
    values = [w.values[r][0, :, :T] for r in range(4)]
    cur = [w.current(r) for r in range(4)]
    q = [w.queries[r][0] for r in range(4)]
    kc = [c[0][0] for c in cur]
    vc = [c[1][0] for c in cur]
    o0, o1, d2, d3, mask, mass = torch_cpu.decode_layer_step(q, kc, vc, keys, values, SCALING, 0.10)
    f = lambda t: t.float().numpy().reshape(R, -1)  # noqa: E731
    ref = OA.decode_layer_step([f(x) for x in q], [f(x) for x in kc], [f(x) for x in vc],
                               [k.float().numpy() for k in keys], [v.float().numpy() for v in values], SCALING, 0.10)
    for got, want in ((o0, ref.out0), (o1, ref.out1), (d2, ref.delta2), (d3, ref.delta3)):
        err = np.abs(f(got) - want)
        assert err.max() < 3e-2 and err.mean() < 4e-3
    # the selection ranks bf16 weights: nearly the oracle's set, its mass within bf16 rounding
    sel = mask.reshape(R, -1).numpy()
    for r in range(R):
        k = int(ref.selection.count[r])
        assert sel[r].sum() == k
        overlap = len(set(np.nonzero(sel[r])[0]) & set(ref.selection.indices[r, :k])) / k
        assert overlap > 0.9
    assert np.allclose(mass.reshape(R).numpy(), ref.selection.mass, rtol=3e-2)
