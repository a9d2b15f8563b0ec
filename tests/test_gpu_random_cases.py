"""Seeded random cases of the decode path against the oracle: whole decode steps, decode
appends across rollovers, the decode top-k on adversarial score rows, and the pack
kernel on adversarial value distributions.  Each case draws
its shape, lengths, masks and retention from its seed (printed first), then holds the
results to the same bars as the fixed-shape parity tests."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import codec

from flashloop_amd import CrossLoopKVLayer, kernels
from flashloop_amd.synthetic import DecodeWorkload, decode_workload

import test_gpu_parity as P
from gpu_util import assert_layer_matches_chain, np32, oracle_prefix

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("seed", range(16))
def test_random_decode_step(seed):
    """1-6 sequences x 1-6 heads, 1-3000 tokens each (equal or ragged), loop-3/4 streams
    masked or full, retention 2%-100%: packed streams bit-exact (equal lengths) and the
    step against the oracle."""
    rng = np.random.default_rng(1000 + seed)
    B, H = int(rng.integers(1, 7)), int(rng.integers(1, 7))
    ragged = B > 1 and rng.random() < 0.4
    lengths = [int(x) for x in rng.integers(1, 3000, size=B)] if ragged else [int(rng.integers(1, 3000))] * B
    frac = float(rng.choice([0.02, 0.05, 0.1, 0.1, 0.25, 0.5, 0.9, 1.0]))
    masked = bool(rng.random() < 0.5)
    tm = max(lengths)
    print(f"case: random decode step seed={seed} B{B} H{H} lengths={lengths} frac={frac} masked={masked}",
          flush=True)
    w = decode_workload(B, H, tm, seed=seed, lengths=lengths if ragged else None)
    m3 = m4 = None
    if masked:
        m3, m4 = P._masks(B, tm, seed, p3=float(rng.uniform(0.05, 0.6)), p4=float(rng.uniform(0.05, 0.6)))
    layer = P._build(w, m3, m4)
    if not ragged and tm >= 64:
        _, _, chain, tp = oracle_prefix([w.cache(r)[0] for r in range(4)], [w.cache(r)[1] for r in range(4)], m3, m4)
        assert tp == layer.quantized_tokens
        assert_layer_matches_chain(layer, chain, tp, B, H)
    P._step_vs_oracle(w, layer, m3, m4, frac=frac)


@pytest.mark.parametrize("seed", range(10))
def test_random_appends_across_rollovers(seed):
    """A prefill of 1-700 tokens per sequence (1-3 sequences, equal or ragged, masked or
    not), then 1-199 decode appends: the packed streams equal the oracle's encode of every
    grown sequence (equal lengths), and the next decode step matches the oracle."""
    rng = np.random.default_rng(2000 + seed)
    B, H = int(rng.integers(1, 4)), int(rng.integers(1, 5))
    ragged = B > 1 and rng.random() < 0.5
    L = [int(x) for x in rng.integers(1, 700, size=B)] if ragged else [int(rng.integers(1, 700))] * B
    steps = int(rng.integers(1, 200))
    masked = bool(rng.random() < 0.6)
    frac = float(rng.choice([0.05, 0.1, 0.3, 1.0]))
    print(f"case: random appends seed={seed} B{B} H{H} L={L} steps={steps} masked={masked} frac={frac}",
          flush=True)
    lm = max(L)
    w = decode_workload(B, H, lm, seed=seed, lengths=L, extra=steps + 1)
    tot = [x + steps for x in L]
    tt = max(tot) + 1
    kw, m3, m4 = {}, None, None
    if masked:
        m3p, m4p = P._masks(B, lm, seed, p3=float(rng.uniform(0.05, 0.7)), p4=float(rng.uniform(0.05, 0.7)))
        kw = dict(mask_loop3=torch.from_numpy(m3p).to(DEV), mask_loop4=torch.from_numpy(m4p).to(DEV))
        # decode tokens are active in loops 3/4: the masks of the grown sequences
        m3, m4 = np.ones((B, tt), bool), np.ones((B, tt), bool)
        for b in range(B):
            m3[b, : L[b]] = m3p[b, : L[b]]
            m4[b, : L[b]] = m4p[b, : L[b]]
    ks = [w.keys[r][:, :, :lm].contiguous().to(DEV) for r in range(4)]
    vs = [w.values[r][:, :, :lm].contiguous().to(DEV) for r in range(4)]
    layer = CrossLoopKVLayer.from_prefill(ks, vs, lengths=L, token_capacity=(tt + 127) // 64 * 64 + 64, **kw)
    ar = torch.arange(B)
    for s in range(steps):
        pos = torch.tensor([x + s for x in L])
        layer.append_decode_token([w.keys[r][ar, :, pos].unsqueeze(2).contiguous().to(DEV) for r in range(4)],
                                  [w.values[r][ar, :, pos].unsqueeze(2).contiguous().to(DEV) for r in range(4)])
    torch.cuda.synchronize()
    if not ragged:
        total = tot[0]
        assert layer.quantized_tokens == codec.packed_prefix_tokens(total)
        nk = [np32(w.keys[r][:, :, :total]) for r in range(4)]
        nv = [np32(w.values[r][:, :, :total]) for r in range(4)]
        chain, tp = codec.compress_prefix(nk, nv, None if m3 is None else (m3[:, :total], m4[:, :total]))
        assert_layer_matches_chain(layer, chain, tp, B, H)
    grown = DecodeWorkload(w.keys, w.values, w.queries, tot)
    cut = max(tot)
    P._step_vs_oracle(grown, layer, None if m3 is None else m3[:, :cut], None if m4 is None else m4[:, :cut],
                      frac=frac)


@pytest.mark.parametrize("seed", range(24))
def test_random_topk_rows(seed):
    """1-8 rows of 1-70,000 keys in one padded buffer (values past a row's count are
    never read), drawn normal, tied, all-equal, peaked (x64), -inf-riddled, NaN/inf-carrying
    or +-0; retention 0.1%-100%: indices, validity, counts and non-finite counts equal
    the oracle's, mass and weights within 2e-6 / 2e-5 relative."""
    rng = np.random.default_rng(3000 + seed)
    rows = int(rng.integers(1, 9))
    long_rows = rng.random() < 0.25
    lens = [int(x) for x in rng.integers(1, 70000 if long_rows else 36000, size=rows)]
    frac = float(rng.choice([0.001, 0.01, 0.1, 0.25, 0.5, 1.0, float(rng.uniform(0.001, 1.0))]))
    kind = ["normal", "ties", "equal", "peaked", "neginf", "nonfinite", "zeros"][seed % 7]
    print(f"case: random topk seed={seed} rows={rows} lens={lens} frac={frac:.4f} kind={kind}", flush=True)
    stride = max(lens) + int(rng.integers(0, 70))
    lg = np.full((rows, stride), 12345.0, np.float32)
    row_list = []
    for r, n in enumerate(lens):
        if kind == "normal":
            x = rng.standard_normal(n).astype(np.float32) * float(rng.choice([0.1, 1.0, 4.0]))
        elif kind == "ties":
            x = (rng.integers(-30, 30, size=n) / 4.0).astype(np.float32)
        elif kind == "equal":
            x = np.full(n, float(rng.standard_normal()), np.float32)
        elif kind == "peaked":
            x = (rng.standard_normal(n) * 64.0).astype(np.float32)
        elif kind == "neginf":
            x = rng.standard_normal(n).astype(np.float32)
            x[rng.random(n) < 0.3] = -np.inf
        elif kind == "zeros":
            x = np.where(rng.random(n) < 0.5, np.float32(0.0), np.float32(-0.0)).astype(np.float32)
            x[rng.random(n) < 0.1] = 1.0
        else:
            x = rng.standard_normal(n).astype(np.float32)
            u = rng.random(n)
            x[u < 0.001] = np.nan
            x[u > 0.999] = np.inf
        lg[r, :n] = x
        row_list.append(x)
    sel = OA.decode_topk(row_list, frac)
    cap = sel.indices.shape[1]
    nk = torch.tensor(lens, dtype=torch.int32, device=DEV)
    nf = torch.full((rows,), -1, dtype=torch.int32, device=DEV)
    idx, valid, mass, wts, counts = kernels.decode_topk(torch.from_numpy(lg).to(DEV), nk, frac, cap, nonfinite=nf)
    torch.cuda.synchronize()
    assert np.array_equal(idx.cpu().numpy(), sel.indices), "indices differ"
    assert np.array_equal(valid.cpu().numpy().astype(bool), sel.valid), "validity differs"
    assert np.array_equal(counts.cpu().numpy(), sel.count), "counts differ"
    gm, gw = mass.cpu().numpy(), wts.cpu().numpy()
    assert np.array_equal(np.isnan(gm), np.isnan(sel.mass)), "rows without finite weights differ"
    fin = np.isfinite(sel.mass)
    assert np.allclose(gm[fin], sel.mass[fin], rtol=2e-6, atol=1e-7), "mass differs"
    fw = np.isfinite(sel.selected_weights)
    assert np.allclose(gw[fw], sel.selected_weights[fw], rtol=2e-5, atol=1e-8), "weights differ"
    assert nf.cpu().tolist() == [int(np.sum(np.isnan(x) | np.isinf(x))) for x in row_list], "non-finite counts"


def _draw(shape, kind, g):
    if kind == "cauchy":
        x = torch.tan(math.pi * (torch.rand(shape, generator=g) - 0.5)).clamp(-3e38, 3e38)  # standard Cauchy
    elif kind == "uniform":
        x = torch.rand(shape, generator=g) * 2 - 1
    elif kind == "scaled":  # per-head magnitudes from 1e-30 to 1e30
        x = torch.randn(shape, generator=g) * (10.0 ** torch.randint(-30, 30, (shape[0], shape[1], 1, 1),
                                                                        generator=g).float())
    elif kind == "constant":  # near-constant channels: tiny spans
        x = torch.randn(shape[:-1] + (1,), generator=g).expand(shape).clone()
        x[..., ::7] += 1e-3
    elif kind == "sparse":  # 95% zeros, signed (-0.0 from negative draws)
        x = torch.randn(shape, generator=g) * (torch.rand(shape, generator=g) < 0.05)
    elif kind == "quantized":  # half-integers: exact ties in the quotient
        x = torch.randint(-8, 8, shape, generator=g).float() * 0.5
    else:
        x = torch.randn(shape, generator=g)
    return x


@pytest.mark.parametrize("seed", range(14))
def test_random_pack(seed):
    """The pack kernel on 1-2 sequences x 1-3 heads x 64-700 tokens drawn Cauchy, uniform,
    scaled by 10^+-30, near-constant, 95%-sparse (signed zeros), half-integer or normal,
    with per-loop drift 0-10x, masked or not: codes, fp32 and fp16 metadata and the bf16
    reconstructions equal the oracle's bit for bit (bit patterns, so zero signs count)."""
    rng = np.random.default_rng(4000 + seed)
    B, H, T = int(rng.integers(1, 3)), int(rng.integers(1, 4)), int(rng.integers(64, 700))
    kind = ["cauchy", "uniform", "scaled", "constant", "sparse", "quantized", "normal"][seed % 7]
    drift = float(rng.choice([0.0, 1e-3, 0.1, 1.0, 10.0]))
    masked = bool(rng.random() < 0.5)
    print(f"case: random pack seed={seed} B{B} H{H} T{T} kind={kind} drift={drift} masked={masked}", flush=True)
    g = torch.Generator().manual_seed(5000 + seed)
    shape = (B, H, T, 128)
    k, v = _draw(shape, kind, g), _draw(shape, kind, g)
    ks, vs = [], []
    for r in range(4):
        ks.append(k.bfloat16())
        vs.append(v.bfloat16())
        k = k.float() + drift * _draw(shape, kind, g)
        v = v.float() + drift * _draw(shape, kind, g)
    m3 = m4 = None
    kw = {}
    if masked:
        m3, m4 = P._masks(B, T, seed, p3=float(rng.uniform(0.1, 0.9)), p4=float(rng.uniform(0.1, 0.9)))
        kw = dict(mask_loop3=torch.from_numpy(m3).to(DEV), mask_loop4=torch.from_numpy(m4).to(DEV))
    layer = CrossLoopKVLayer.from_prefill([x.to(DEV) for x in ks], [x.to(DEV) for x in vs], recon=True, **kw)
    torch.cuda.synchronize()
    _, _, chain, tp = oracle_prefix(ks, vs, m3, m4)
    assert tp == layer.quantized_tokens
    assert_layer_matches_chain(layer, chain, tp, B, H)
    for r in range(4 if tp else 0):  # (below 128 tokens nothing is packed)
        gk = np32(layer.recon_keys[r]).reshape(B, H, T, 128)[:, :, :tp]
        gv = np32(layer.recon_values[r]).reshape(B, H, T, 128)[:, :, :tp]
        assert np.array_equal(gk.view(np.uint32), chain.recon_keys[r].view(np.uint32)), f"R_{r} keys differ"
        assert np.array_equal(gv.view(np.uint32), chain.recon_values[r].view(np.uint32)), f"R_{r} values differ"
    P._assert_half_copies(layer, chain, tp, B, H)
