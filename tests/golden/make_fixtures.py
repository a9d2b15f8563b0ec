"""Write the golden fixture tests/golden/decode_small.npz from the numpy oracle.

Run from the repository root: ``python tests/golden/make_fixtures.py``.  The fixture is
data only (inputs as bf16 bit patterns, and the oracle's codes, metadata,
reconstructions, selection and attention outputs); loading it never executes code
(``numpy.load`` with ``allow_pickle=False``).  The reference package is not imported:
it has no fixtures of its own for this path and its algorithm is restated in
``oracle/``.
"""

from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from flashloop_amd.synthetic import SCALING, decode_workload  # noqa: E402
from oracle import attention as OA  # noqa: E402
from oracle import codec  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "decode_small.npz")
B, H, T, SEED, FRACTION = 1, 1, 200, 0, 0.10


def bits(t):
    return t.contiguous().view(dtype=__import__("torch").int16).numpy().astype(np.uint16)


def build() -> dict:
    w = decode_workload(B, H, T, seed=SEED)
    rng = np.random.default_rng(SEED)
    m3 = rng.random((B, T)) < 0.3
    m4 = m3 & (rng.random((B, T)) < 0.5)
    m3[:, -1] = m4[:, -1] = True
    keys = [w.keys[r].float().numpy() for r in range(4)]  # [B,H,T+1,128]
    vals = [w.values[r].float().numpy() for r in range(4)]
    chain, tp = codec.compress_prefix([k[:, :, :T] for k in keys], [v[:, :, :T] for v in vals], (m3, m4))
    K, V = codec.materialize_loop_cache([k[:, :, :T] for k in keys], [v[:, :, :T] for v in vals], chain, tp)
    R = B * H
    q = [w.queries[r].float().numpy().reshape(R, 128) for r in range(4)]
    kc = [keys[r][:, :, T].reshape(R, 128) for r in range(4)]
    vc = [vals[r][:, :, T].reshape(R, 128) for r in range(4)]
    step = OA.decode_layer_step(q, kc, vc, [K[r].reshape(R, T, 128) for r in range(4)],
                                [V[r].reshape(R, T, 128) for r in range(4)], SCALING, FRACTION)
    f = dict(
        seed=np.int64(SEED), batch=np.int64(B), heads=np.int64(H), tokens=np.int64(T), fraction=np.float64(FRACTION),
        packed_tokens=np.int64(tp),
        keys=np.stack([bits(w.keys[r]) for r in range(4)]),
        values=np.stack([bits(w.values[r]) for r in range(4)]),
        queries=np.stack([bits(w.queries[r]) for r in range(4)]),
        mask_loop3=m3, mask_loop4=m4,
        k_codes=np.stack([s.k_codes for s in chain.streams]),
        k_scale=np.stack([s.k_scale for s in chain.streams]),
        k_min=np.stack([s.k_min for s in chain.streams]),
        v_codes=np.stack([s.v_codes for s in chain.streams]),
        v_scale=np.stack([s.v_scale for s in chain.streams]),
        v_min=np.stack([s.v_min for s in chain.streams]),
        recon_keys=np.stack(chain.recon_keys).astype(np.float32).view(np.uint32).__rshift__(16).astype(np.uint16),
        recon_values=np.stack(chain.recon_values).astype(np.float32).view(np.uint32).__rshift__(16).astype(np.uint16),
        out0=step.out0, out1=step.out1, logits1=np.asarray(step.logits1),
        sel_indices=step.selection.indices, sel_valid=step.selection.valid, sel_mass=step.selection.mass,
        sel_count=step.selection.count, selected_output=step.selected_output,
        delta2=step.delta2, delta3=step.delta3,
    )
    return f


def main() -> None:
    np.savez_compressed(OUT, **build())
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
