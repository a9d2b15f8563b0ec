"""Golden fixture tests/golden/decode_small.npz (written by tests/golden/make_fixtures.py).

CPU: the oracle still reproduces the fixture (regression of the checker itself).
GPU: the HIP path reproduces the fixture's codes, metadata and reconstructions bit for
bit, its selection bit for bit on its own logits, and its outputs within tolerance.
"""

import os

import numpy as np
import pytest

from oracle import attention as OA
from oracle import codec

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "decode_small.npz")


def _load():
    return dict(np.load(FIX, allow_pickle=False))


def _f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def test_oracle_reproduces_fixture():
    f = _load()
    T = int(f["tokens"])
    keys = [_f32(f["keys"][r])[:, :, :T] for r in range(4)]
    vals = [_f32(f["values"][r])[:, :, :T] for r in range(4)]
    chain, tp = codec.compress_prefix(keys, vals, (f["mask_loop3"], f["mask_loop4"]))
    assert tp == int(f["packed_tokens"])
    for s in range(4):
        st = chain.streams[s]
        assert np.array_equal(st.k_codes, f["k_codes"][s]) and np.array_equal(st.v_codes, f["v_codes"][s])
        assert np.array_equal(st.k_scale, f["k_scale"][s]) and np.array_equal(st.k_min, f["k_min"][s])
        assert np.array_equal(st.v_scale, f["v_scale"][s]) and np.array_equal(st.v_min, f["v_min"][s])
        assert np.array_equal(chain.recon_keys[s], _f32(f["recon_keys"][s]))
    sel = OA.decode_topk(f["logits1"], float(f["fraction"]))
    assert np.array_equal(sel.indices, f["sel_indices"])


@pytest.mark.gpu
def test_hip_path_reproduces_fixture():
    import torch

    from flashloop_amd import CrossLoopKVLayer, decode_attention_step
    from flashloop_amd.synthetic import SCALING

    print("case: golden decode_small", flush=True)
    f = _load()
    T, B, H = int(f["tokens"]), int(f["batch"]), int(f["heads"])
    R = B * H
    dev = "cuda"

    def bf(x):
        return torch.from_numpy(x.astype(np.int16)).view(torch.bfloat16)

    ks = [bf(f["keys"][r][:, :, :T]).contiguous().to(dev) for r in range(4)]
    vs = [bf(f["values"][r][:, :, :T]).contiguous().to(dev) for r in range(4)]
    layer = CrossLoopKVLayer.from_prefill(ks, vs, mask_loop3=torch.from_numpy(f["mask_loop3"]).to(dev),
                                          mask_loop4=torch.from_numpy(f["mask_loop4"]).to(dev), recon=True)
    tp = int(f["packed_tokens"])
    for s in range(4):
        kc = layer.key_codes[s].cpu().numpy()
        got = np.empty(kc.shape[:-1] + (128,), np.uint8)
        got[..., 0::2], got[..., 1::2] = kc & 0xF, kc >> 4
        act = f["mask_loop3"][0, :tp] if s == 2 else (f["mask_loop4"][0, :tp] if s == 3 else np.ones(tp, bool))
        rows = np.nonzero(act)[0] if s < 2 else layer.rank[s - 2][0].cpu().numpy()[np.nonzero(act)[0]]
        assert np.array_equal(got[:, rows], f["k_codes"][s].reshape(R, tp, 128)[:, np.nonzero(act)[0]])
        km = layer.key_meta[s].cpu().numpy()[:, : tp // 64]
        assert np.array_equal(km[..., 0], f["k_scale"][s].reshape(R, tp // 64, 128))
        assert np.array_equal(km[..., 1], f["k_min"][s].reshape(R, tp // 64, 128))
        rk = layer.recon_keys[s].cpu().view(torch.int16).numpy().astype(np.uint16)[:, :tp]
        assert np.array_equal(rk, f["recon_keys"][s].reshape(R, tp, 128))
    cur_k = [bf(f["keys"][r][:, :, T:T + 1]).contiguous().to(dev) for r in range(4)]
    cur_v = [bf(f["values"][r][:, :, T:T + 1]).contiguous().to(dev) for r in range(4)]
    qs = [bf(f["queries"][r]).contiguous().to(dev) for r in range(4)]
    step = decode_attention_step(layer, qs, cur_k, cur_v, SCALING, float(f["fraction"]))
    torch.cuda.synchronize()
    for name in ("out0", "out1", "delta2", "delta3"):
        got = getattr(step, name).float().cpu().numpy().reshape(R, 128)
        err = np.abs(got - f[name])
        assert err.max() <= 2e-2 and err.mean() <= 1e-3, name
    lg = step.logits1.float().cpu().numpy().reshape(R, -1)[:, : T + 1]
    sel = OA.decode_topk(lg, float(f["fraction"]), kpad=step.indices.shape[-1])
    assert np.array_equal(step.indices.cpu().numpy().reshape(R, -1), sel.indices)
