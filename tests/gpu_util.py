"""Helpers shared by the GPU parity tests (host-side conversions only)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import codec


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def unpack_codes(codes: torch.Tensor) -> np.ndarray:
    """u8 ``[..., 64]`` rows (channel 2j low nibble, 2j+1 high) -> ``[..., 128]``."""
    c = codes.cpu().numpy()
    out = np.empty(c.shape[:-1] + (128,), np.uint8)
    out[..., 0::2] = c & 0xF
    out[..., 1::2] = c >> 4
    return out


def oracle_prefix(keys, values, m3=None, m4=None):
    """Oracle chain over the packed prefix of [B,H,T,128] bf16 torch tensors."""
    nk = [np32(k) for k in keys]
    nv = [np32(v) for v in values]
    masks = None if m3 is None else (np.asarray(m3, bool), np.asarray(m4, bool))
    chain, tp = codec.compress_prefix(nk, nv, masks)
    return nk, nv, chain, tp


def assert_layer_matches_chain(layer, chain, tp, batch, heads):
    """Bit-exact codes, K/V metadata of all four streams against the oracle chain."""
    bh = batch * heads
    G = tp // 64
    for s in range(4):
        sc = chain.streams[s]
        kc = unpack_codes(layer.key_codes[s])
        vc = unpack_codes(layer.value_codes[s])
        kmeta = layer.key_meta[s].cpu().numpy()
        vmeta = layer.value_meta[s].cpu().numpy()
        ks = sc.k_scale.reshape(bh, G, 128)
        km = sc.k_min.reshape(bh, G, 128)
        assert np.array_equal(kmeta[:, :G, :, 0], ks), f"stream {s}: K scale mismatch"
        assert np.array_equal(kmeta[:, :G, :, 1], km), f"stream {s}: K min mismatch"
        okc = sc.k_codes.reshape(batch, heads, tp, 128)
        ovc = sc.v_codes.reshape(batch, heads, tp, 128)
        ovs = sc.v_scale.reshape(batch, heads, tp, 2)
        ovm = sc.v_min.reshape(batch, heads, tp, 2)
        for b in range(batch):
            act = sc.active[b, :tp]
            t_idx = np.nonzero(act)[0]
            if s < 2:
                rows = t_idx
            else:
                rank = layer.rank[s - 2][b].cpu().numpy()
                rows = rank[t_idx]
                assert np.all(rows >= 0), "active row without a rank"
                assert np.all(rank[:tp][~act] == -1)
            for h in range(heads):
                r = b * heads + h
                assert np.array_equal(kc[r, rows], okc[b, h, t_idx]), f"stream {s}: K codes mismatch (b={b}, h={h})"
                assert np.array_equal(vc[r, rows], ovc[b, h, t_idx]), f"stream {s}: V codes mismatch (b={b}, h={h})"
                assert np.array_equal(vmeta[r, rows, :, 0], ovs[b, h, t_idx]), f"stream {s}: V scale mismatch"
                assert np.array_equal(vmeta[r, rows, :, 1], ovm[b, h, t_idx]), f"stream {s}: V min mismatch"


def materialized(nk, nv, chain, tp):
    """Per-loop K_r/V_r the reference attends to: reconstructed prefix + raw tail."""
    return codec.materialize_loop_cache(nk, nv, chain, tp)


def flat_rows(x: np.ndarray, lengths=None):
    """[B,H,T,C] -> list over (b,h) of [T_b, C] arrays."""
    b, h = x.shape[:2]
    out = []
    for i in range(b):
        t = x.shape[2] if lengths is None else lengths[i]
        for j in range(h):
            out.append(x[i, j, :t])
    return out


def assert_close(got: np.ndarray, want: np.ndarray, max_abs: float = 2e-2, mean_abs: float = 1e-3, what: str = ""):
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    print(f"[parity] {what}: max abs {err.max():.3e} mean abs {err.mean():.3e}", flush=True)
    assert err.max() <= max_abs, f"{what}: max abs err {err.max():.3e} > {max_abs}"
    assert err.mean() <= mean_abs, f"{what}: mean abs err {err.mean():.3e} > {mean_abs}"
    return float(err.max()), float(err.mean())
