"""On-disk format of the packed cross-loop cache: save -> load round trips every buffer
and length mirror bit for bit; version, tensor-set and shape mismatches are rejected."""

import json

import pytest
import torch

from flashloop_amd.cache import CrossLoopKVCache, CrossLoopKVLayer, LayerGeometry


def _random_layer(seed=0, batch=2, heads=3):
    g = torch.Generator().manual_seed(seed)
    geo = LayerGeometry(batch, heads, 256, 128, (256, 256, 96, 80))
    layer = CrossLoopKVLayer(geo, "cpu")
    for name, t in layer._named_tensors().items():
        if t.dtype == torch.uint8:
            t.copy_(torch.randint(0, 256, t.shape, generator=g, dtype=torch.uint8))
        elif t.dtype == torch.int32:
            t.copy_(torch.randint(-1, 200, t.shape, generator=g, dtype=torch.int32))
        else:
            t.copy_(torch.randn(t.shape, generator=g).to(t.dtype))
    layer.packed_host = [192, 128][:batch]
    layer.tail_host = [70, 100][:batch]
    layer.late_rows_host = [[40, 30][:batch], [20, 10][:batch]]
    layer.packed_tokens.copy_(torch.tensor(layer.packed_host, dtype=torch.int32))
    layer.tail_tokens.copy_(torch.tensor(layer.tail_host, dtype=torch.int32))
    layer.late_rows.copy_(torch.tensor(layer.late_rows_host, dtype=torch.int32))
    return layer


def _assert_same(a, b):
    ta, tb = a._named_tensors(), b._named_tensors()
    assert set(ta) == set(tb)
    for k in ta:
        assert ta[k].dtype == tb[k].dtype and torch.equal(ta[k].view(torch.uint8), tb[k].view(torch.uint8)), k
    assert a.packed_host == b.packed_host and a.tail_host == b.tail_host and a.late_rows_host == b.late_rows_host
    assert a.geometry == b.geometry


def test_layer_round_trip(tmp_path):
    layer = _random_layer()
    path = str(tmp_path / "layer.safetensors")
    layer.save(path)
    back = CrossLoopKVLayer.load(path, device="cpu")
    _assert_same(layer, back)
    # the codes stay one 128-byte line per token: key/value views share it
    assert back.key_codes[0].data_ptr() == back.codes[0].data_ptr()
    assert back.value_codes[0].data_ptr() == back.codes[0].data_ptr() + 64


def test_cache_round_trip(tmp_path):
    cache = CrossLoopKVCache(num_layers=3)
    cache.set_layer(0, _random_layer(1))
    cache.set_layer(2, _random_layer(2, batch=1, heads=2))
    path = str(tmp_path / "cache.safetensors")
    cache.save(path)
    back = CrossLoopKVCache.load(path, device="cpu")
    assert len(back.layers) == 3 and back.layers[1] is None
    _assert_same(cache.layers[0], back.layers[0])
    _assert_same(cache.layers[2], back.layers[2])
    assert back.storage_bytes == cache.storage_bytes


def test_rejects_bad_payloads():
    layer = _random_layer()
    tensors, header = layer.state_dict()
    bad = dict(header, version=99)
    with pytest.raises(ValueError, match="version"):
        CrossLoopKVLayer.from_state_dict(tensors, bad, "cpu")
    with pytest.raises(ValueError, match="not a"):
        CrossLoopKVLayer.from_state_dict(tensors, dict(header, format="other"), "cpu")
    missing = {k: v for k, v in tensors.items() if k != "rank.1"}
    with pytest.raises(ValueError, match="missing"):
        CrossLoopKVLayer.from_state_dict(missing, header, "cpu")
    wrong = dict(tensors)
    wrong["codes.0"] = wrong["codes.0"][:, :-1]
    with pytest.raises(ValueError, match="codes.0"):
        CrossLoopKVLayer.from_state_dict(wrong, header, "cpu")
    with pytest.raises(ValueError, match="disagree"):
        CrossLoopKVLayer.from_state_dict(tensors, dict(header, tail_tokens=[1, 2]), "cpu")
    json.dumps(header)  # the header is plain JSON
