"""Ragged batched engine: B sequences of different lengths in one packed cache per layer,
decoded together, against batch-one engines run on each sequence alone."""

import pytest
import torch

pytestmark = pytest.mark.gpu

from flashloop_amd.batch_engine import FlashLoopBatchEngine  # noqa: E402
from flashloop_amd.engine import FlashLoopEngine  # noqa: E402
from flashloop_amd.model import OuroConfig, OuroForCausalLM  # noqa: E402

TINY = OuroConfig(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                  num_attention_heads=2, num_key_value_heads=2)
LENGTHS = [150, 262, 200]
STEPS = 80  # tails of 86/70/72 rows roll over at different steps


def _batch(seed=11):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, TINY.vocab_size, (len(LENGTHS), max(LENGTHS) + STEPS), generator=g).cuda()
    mask = torch.zeros(len(LENGTHS), max(LENGTHS), dtype=torch.long, device="cuda")
    for b, n in enumerate(LENGTHS):
        mask[b, :n] = 1
    return ids, mask


def _cos(a, b):
    return float(torch.nn.functional.cosine_similarity(a.flatten().double(), b.flatten().double(), dim=0))


def test_batched_decode_tracks_single_sequences():
    model = OuroForCausalLM.random_init(TINY, seed=9, device="cuda")
    ids, mask = _batch()
    tmax = max(LENGTHS)
    prompts = ids[:, :tmax] * mask  # padding ids are arbitrary
    eng = FlashLoopBatchEngine(model, use_graphs=False)
    out = eng.prefill(prompts, mask, decode_capacity=STEPS + 64)
    singles = [FlashLoopEngine(model, use_graphs=False) for _ in LENGTHS]
    ref = [s.prefill(ids[b:b + 1, :n], decode_capacity=STEPS + 64) for b, (s, n) in enumerate(zip(singles, LENGTHS))]
    for b in range(len(LENGTHS)):
        # prefill logits come from the same per-sequence loops
        assert torch.equal(out.logits[b:b + 1], ref[b].logits)
        assert torch.equal(out.state.mask_loop3[b, :LENGTHS[b]], ref[b].state.mask_loop3[0])
    for i in range(STEPS):
        tok = torch.stack([ids[b, n + i] for b, n in enumerate(LENGTHS)])[:, None]
        d = eng.decode(tok)
        for b, s in enumerate(singles):
            r = s.decode(tok[b:b + 1]).logits
            got = d.logits[b:b + 1]
            assert torch.isfinite(got).all()
            assert _cos(got, r) > 0.999, f"step {i} seq {b}"
            assert (got - r).abs().max().item() < 5e-2 * max(1.0, r.abs().max().item()), f"step {i} seq {b}"
    # every sequence's cache rolled over on its own schedule
    for li, lay in enumerate(eng.state.cache.layers):
        for b, s in enumerate(singles):
            one = s.state.cache.layers[li]
            assert lay.packed_host[b] == one.packed_host[0] and lay.tail_host[b] == one.tail_host[0]
    assert eng.state.positions == tuple(n + STEPS for n in LENGTHS)


def test_batched_graph_matches_eager():
    model = OuroForCausalLM.random_init(TINY, seed=10, device="cuda")
    ids, mask = _batch(seed=12)
    tmax = max(LENGTHS)
    eager = FlashLoopBatchEngine(model, use_graphs=False)
    graphed = FlashLoopBatchEngine(model, use_graphs=True)
    eager.prefill(ids[:, :tmax], mask, decode_capacity=STEPS + 64)
    graphed.prefill(ids[:, :tmax], mask, decode_capacity=STEPS + 64)
    for i in range(STEPS):
        tok = torch.stack([ids[b, n + i] for b, n in enumerate(LENGTHS)])[:, None]
        a = eager.decode(tok).logits
        g = graphed.decode(tok).logits
        assert torch.equal(a, g), f"step {i}"


def test_batched_generate_shapes():
    model = OuroForCausalLM.random_init(TINY, seed=13, device="cuda")
    ids, mask = _batch(seed=14)
    eng = FlashLoopBatchEngine(model)
    out = eng.generate(ids[:, :max(LENGTHS)], mask, max_new_tokens=20)
    assert [int(x.numel()) for x in out] == [n + 20 for n in LENGTHS]
    for b, n in enumerate(LENGTHS):
        assert torch.equal(out[b][:n], ids[b, :n])
