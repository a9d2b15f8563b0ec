"""Host-side checks of the Ouro-shaped model, the settings mirror and the hook objects."""

import pytest
import torch

from flashloop_amd.config import FlashLoopConfig, validate_ouro_model
from flashloop_amd.model import OuroConfig, OuroForCausalLM

TINY = OuroConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                  num_attention_heads=2, num_key_value_heads=2)


def test_config_validation():
    FlashLoopConfig()
    with pytest.raises(ValueError):
        FlashLoopConfig(prefill_fraction_loop3=0.1, prefill_fraction_loop4=0.2)
    with pytest.raises(ValueError):
        FlashLoopConfig(decode_key_fraction=0.0)
    with pytest.raises(ValueError):
        FlashLoopConfig(kv_bits=8)
    assert FlashLoopConfig(enable_token_sparse_prefill=False).effective_prefill_fractions == (1.0, 1.0)
    assert FlashLoopConfig(enable_sparse_decode=False).effective_decode_key_fraction == 1.0


def test_shape_contract():
    validate_ouro_model(OuroForCausalLM(TINY))
    with pytest.raises(ValueError):
        validate_ouro_model(OuroForCausalLM(OuroConfig(**{**TINY.__dict__, "total_ut_steps": 3})))
    with pytest.raises(ValueError):
        validate_ouro_model(OuroForCausalLM(OuroConfig(**{**TINY.__dict__, "num_key_value_heads": 1})))


def test_random_init_deterministic_and_save_load(tmp_path):
    a = OuroForCausalLM.random_init(TINY, seed=3)
    b = OuroForCausalLM.random_init(TINY, seed=3)
    ids = torch.randint(0, TINY.vocab_size, (1, 17), generator=torch.Generator().manual_seed(0))
    la = a.dense_forward(ids)
    assert torch.equal(la, b.dense_forward(ids))
    a.save_pretrained(str(tmp_path))
    c = OuroForCausalLM.from_pretrained(str(tmp_path))
    assert torch.equal(la, c.dense_forward(ids))
    out = a.generate(ids, max_new_tokens=2)
    assert out.shape == (1, 19) and torch.equal(out[:, :17], ids)


def test_dense_forward_is_causal():
    """Last-position logits do not depend on tokens after it: appending a token and
    reading position -2 through a shorter prompt gives the same logits."""
    m = OuroForCausalLM.random_init(TINY, seed=1)
    ids = torch.randint(0, TINY.vocab_size, (1, 12), generator=torch.Generator().manual_seed(1))
    full = m.dense_forward(ids[:, :11])
    again = m.dense_forward(ids[:, :11].clone())
    assert torch.equal(full, again)


def test_batch_engine_lengths_validation():
    import pytest as _pt
    import torch as _t

    from flashloop_amd.batch_engine import FlashLoopBatchEngine

    ids = _t.zeros(3, 5, dtype=_t.long)
    assert FlashLoopBatchEngine._lengths(ids, None) == [5, 5, 5]
    m = _t.tensor([[1, 1, 1, 0, 0], [1, 1, 1, 1, 1], [1, 0, 0, 0, 0]])
    assert FlashLoopBatchEngine._lengths(ids, m) == [3, 5, 1]
    with _pt.raises(ValueError, match="right-padded"):
        FlashLoopBatchEngine._lengths(ids, _t.tensor([[0, 1, 1, 1, 1]] * 3))
    with _pt.raises(ValueError, match="no tokens"):
        FlashLoopBatchEngine._lengths(ids, _t.zeros(3, 5))
