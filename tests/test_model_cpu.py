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


def _hf_dir(tmp_path, model, *, shards=2, extra=True, tied=False):
    """A Hugging Face-style Ouro checkpoint directory written the way HF writes one:
    config.json with keys this build ignores, weights sharded per an index file, plus
    tensors (early-exit gate) this model has no parameter for."""
    import json

    from safetensors.torch import save_file

    cfg = dict(model.config.__dict__)
    del cfg["head_dim"]  # HF Ouro configs may leave it implicit (hidden / heads)
    cfg.update(model_type="ouro", architectures=["OuroForCausalLM"], torch_dtype="bfloat16",
               max_position_embeddings=65536, hidden_act="silu", layer_types=["full_attention"] * 2,
               sliding_window=None, tie_word_embeddings=tied, auto_map={"AutoConfig": "x.OuroConfig"},
               eos_token_id=[2])
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    sd = {k: v.contiguous() for k, v in model.state_dict().items()}
    if tied:
        del sd["lm_head.weight"]
    if extra:
        sd["model.early_exit_gate.weight"] = torch.zeros(1, model.config.hidden_size)
    names = sorted(sd)
    weight_map = {}
    for i in range(shards):
        part = names[i::shards]
        fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        save_file({k: sd[k] for k in part}, str(tmp_path / fname))
        weight_map.update({k: fname for k in part})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))


def test_from_pretrained_reads_hf_sharded_checkpoints(tmp_path):
    a = OuroForCausalLM.random_init(TINY, seed=5)
    _hf_dir(tmp_path, a)
    b = OuroForCausalLM.from_pretrained(str(tmp_path))
    assert b.config.head_dim == 128 and b.config.eos_token_id == 2
    assert b.unused_checkpoint_keys == ["model.early_exit_gate.weight"]
    for (ka, va), (kb, vb) in zip(a.state_dict().items(), b.state_dict().items()):
        assert ka == kb and torch.equal(va, vb)


def test_from_pretrained_ties_and_refusals(tmp_path):
    import json

    a = OuroForCausalLM.random_init(TINY, seed=6)
    d1 = tmp_path / "tied"
    d1.mkdir()
    _hf_dir(d1, a, shards=1, tied=True)
    b = OuroForCausalLM.from_pretrained(str(d1))
    assert torch.equal(b.lm_head.weight, a.model.embed_tokens.weight)
    # a variant the engine does not implement, and a checkpoint missing a parameter
    cfg = json.loads((d1 / "config.json").read_text())
    for bad in ({"model_type": "llama"}, {"sliding_window": 4096}, {"layer_types": ["sliding_attention"] * 2}):
        (d1 / "config.json").write_text(json.dumps({**cfg, **bad}))
        with pytest.raises(ValueError):
            OuroForCausalLM.from_pretrained(str(d1))
    (d1 / "config.json").write_text(json.dumps({**cfg, "tie_word_embeddings": False}))
    with pytest.raises(KeyError):
        OuroForCausalLM.from_pretrained(str(d1))


def test_flashloop_hooks_refuse_what_they_cannot_honour():
    from flashloop_amd.hooks import flashloop

    model = OuroForCausalLM.random_init(TINY, seed=7)
    ids = torch.randint(0, TINY.vocab_size, (1, 9), generator=torch.Generator().manual_seed(1))
    dense = model(ids).logits
    with flashloop(model):
        with pytest.raises(TypeError):
            model.generate(ids, max_new_tokens=2, temperature=0.7)
        with pytest.raises(ValueError):
            model.generate(ids, max_new_tokens=2, do_sample=True)
        with pytest.raises(ValueError):
            model.generate(ids, max_new_tokens=2, num_beams=4)
        with pytest.raises(ValueError):
            model.generate(ids, max_new_tokens=2, attention_mask=torch.tensor([[0] + [1] * 8]))
        with pytest.raises(TypeError):
            model(ids, output_attentions=True)
        with pytest.raises(TypeError):
            model(ids[:, :1], past_key_values=object())
    # restored on exit: the dense model again
    assert "forward" not in model.__dict__ and "generate" not in model.__dict__
    assert torch.equal(model(ids).logits, dense)
