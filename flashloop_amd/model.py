"""An Ouro-shaped looped decoder (random init or local weights) for the FlashLoop engine.

The reference drives Ouro-1.4B/2.6B loaded through Hugging Face remote code
(`flashloop/engine.py:134-150`, shape contract `flashloop/config.py:92-134`); that code
is not available offline, so this module provides a model with the same module
structure and arithmetic the engine touches (`flashloop/engine.py:396-537`): token
embedding, `layers[i].{input_layernorm, self_attn.{q,k,v,o}_proj, input_layernorm_2,
post_attention_layernorm, mlp.{gate,up,down}_proj, post_attention_layernorm_2}`, a final
`norm` applied after every loop, rotary embeddings (theta 1e4) and `lm_head`; all
`total_ut_steps` loops reuse the same layers.  Weights are bf16 ~ N(0, 0.02) unless
loaded with `from_pretrained` from a directory written by `save_pretrained`
(`config.json` + `model.safetensors`).
"""

from __future__ import annotations

import json
import os
from dataclasses import asdict, dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class OuroConfig:
    vocab_size: int = 49152
    hidden_size: int = 2048
    intermediate_size: int = 5632
    num_hidden_layers: int = 24
    num_attention_heads: int = 16
    num_key_value_heads: int = 16
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    total_ut_steps: int = 4
    eos_token_id: int | None = None
    init_std: float = 0.02

    @classmethod
    def from_hf_config(cls, raw: dict) -> "OuroConfig":
        """The fields this model uses from a Hugging Face Ouro ``config.json``; every other
        key is ignored.  ``head_dim`` defaults to hidden/heads.  Variants the engine does not
        implement are refused here (flashloop/config.py:92-134): another ``model_type``,
        sliding-window attention, non-full attention layers."""
        mt = raw.get("model_type")
        if mt is not None and mt != "ouro":
            raise ValueError(f"config.json: model_type {mt!r} is not an Ouro checkpoint")
        if raw.get("sliding_window") is not None and raw.get("use_sliding_window", True):
            raise ValueError("config.json: sliding-window attention is not supported")
        lt = raw.get("layer_types")
        if lt is not None and set(lt) != {"full_attention"}:
            raise ValueError("config.json: every layer must use full attention")
        hidden = int(raw["hidden_size"])
        heads = int(raw["num_attention_heads"])
        kw = dict(
            vocab_size=int(raw["vocab_size"]),
            hidden_size=hidden,
            intermediate_size=int(raw["intermediate_size"]),
            num_hidden_layers=int(raw["num_hidden_layers"]),
            num_attention_heads=heads,
            num_key_value_heads=int(raw.get("num_key_value_heads", heads)),
            head_dim=int(raw.get("head_dim") or hidden // heads),
            rms_norm_eps=float(raw.get("rms_norm_eps", 1e-6)),
            rope_theta=float(raw.get("rope_theta", 10000.0)),
            total_ut_steps=int(raw.get("total_ut_steps", 4)),
        )
        eos = raw.get("eos_token_id")
        if isinstance(eos, list):
            eos = eos[0] if eos else None
        kw["eos_token_id"] = None if eos is None else int(eos)
        if "init_std" in raw:
            kw["init_std"] = float(raw["init_std"])
        return cls(**kw)


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = x.float()
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.eps)
        return (self.weight.float() * h).to(x.dtype)


@dataclass
class DenseOutput:
    logits: torch.Tensor
    past_key_values: None = None


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, theta: float) -> None:
        super().__init__()
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        self.register_buffer("inv_freq", inv, persistent=False)

    def forward(self, x: torch.Tensor, positions: torch.Tensor):
        freqs = positions[..., None].float() * self.inv_freq.to(positions.device)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    a, b = x.chunk(2, dim=-1)
    return torch.cat((-b, a), dim=-1)


def apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """``_apply_rope`` (flashloop/engine.py:64-75): cos/sin ``[1, T, D]`` → broadcast over heads."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


class Attention(nn.Module):
    def __init__(self, cfg: OuroConfig) -> None:
        super().__init__()
        h, d = cfg.hidden_size, cfg.head_dim
        self.head_dim = d
        self.num_heads = cfg.num_attention_heads
        self.num_key_value_heads = cfg.num_key_value_heads
        self.num_key_value_groups = self.num_heads // self.num_key_value_heads
        self.scaling = d ** -0.5
        self.q_proj = nn.Linear(h, self.num_heads * d, bias=False)
        self.k_proj = nn.Linear(h, self.num_key_value_heads * d, bias=False)
        self.v_proj = nn.Linear(h, self.num_key_value_heads * d, bias=False)
        self.o_proj = nn.Linear(self.num_heads * d, h, bias=False)


class MLP(nn.Module):
    def __init__(self, cfg: OuroConfig) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.up_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    """Sandwich-norm block: ``h + n2(attn(n1(h)))`` then ``h + n4(mlp(n3(h)))``
    (flashloop/engine.py:533-537)."""

    def __init__(self, cfg: OuroConfig) -> None:
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.self_attn = Attention(cfg)
        self.input_layernorm_2 = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.mlp = MLP(cfg)
        self.post_attention_layernorm_2 = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)


class Backbone(nn.Module):
    def __init__(self, cfg: OuroConfig) -> None:
        super().__init__()
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(cfg) for _ in range(cfg.num_hidden_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(cfg.head_dim, cfg.rope_theta)


class OuroForCausalLM(nn.Module):
    def __init__(self, cfg: OuroConfig) -> None:
        super().__init__()
        self.config = cfg
        self.model = Backbone(cfg)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)

    @classmethod
    def random_init(cls, cfg: OuroConfig, *, seed: int = 0, dtype=torch.bfloat16, device="cpu") -> "OuroForCausalLM":
        """N(0, init_std) weights (norm weights 1), generated on ``device`` from ``seed``."""
        model = cls(cfg)
        gen = torch.Generator(device=device).manual_seed(int(seed))
        model = model.to(device=device, dtype=dtype)
        with torch.no_grad():
            for name, p in model.named_parameters():
                if name.endswith("norm.weight") or "layernorm" in name:
                    p.fill_(1.0)
                else:
                    p.copy_(torch.randn(p.shape, generator=gen, device=device, dtype=torch.float32).mul_(cfg.init_std))
        return model.eval()

    def save_pretrained(self, path: str) -> None:
        """``config.json`` (Hugging Face field names, ``model_type: ouro``) and
        ``model.safetensors`` with the Hugging Face parameter names."""
        from safetensors.torch import save_file

        os.makedirs(path, exist_ok=True)
        cfg = asdict(self.config)
        cfg.update(model_type="ouro", architectures=["OuroForCausalLM"], tie_word_embeddings=False,
                   layer_types=["full_attention"] * self.config.num_hidden_layers, sliding_window=None)
        with open(os.path.join(path, "config.json"), "w") as f:
            json.dump(cfg, f, indent=1)
        save_file({k: v.contiguous() for k, v in self.state_dict().items()}, os.path.join(path, "model.safetensors"))

    @classmethod
    def from_pretrained(cls, path: str, *, dtype=torch.bfloat16, device="cpu") -> "OuroForCausalLM":
        """Load a Hugging Face-style Ouro checkpoint directory (the layout
        ``flashloop/engine.py:134-150`` loads through ``AutoModelForCausalLM``): a
        ``config.json`` (``OuroConfig.from_hf_config``) and the weights in
        ``model.safetensors`` or sharded per ``model.safetensors.index.json``.  Only
        safetensors are read (no code runs).  Parameters are matched by their Hugging Face
        names; checkpoint tensors this model has no parameter for (e.g. early-exit gates)
        are listed in ``unused_checkpoint_keys``; a missing parameter is an error, except
        ``lm_head.weight`` with ``tie_word_embeddings``."""
        from safetensors import safe_open

        with open(os.path.join(path, "config.json")) as f:
            raw = json.load(f)
        cfg = OuroConfig.from_hf_config(raw)
        index = os.path.join(path, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                weight_map = json.load(f)["weight_map"]
            files: dict[str, list[str]] = {}
            for name, fname in weight_map.items():
                files.setdefault(fname, []).append(name)
        elif os.path.exists(os.path.join(path, "model.safetensors")):
            files = {"model.safetensors": None}
        else:
            raise FileNotFoundError(f"{path}: neither model.safetensors nor model.safetensors.index.json")
        model = cls(cfg)
        wanted = model.state_dict()
        loaded: dict[str, torch.Tensor] = {}
        unused = []
        for fname, names in files.items():
            with safe_open(os.path.join(path, fname), framework="pt") as f:
                for name in (names if names is not None else f.keys()):
                    if name in wanted:
                        loaded[name] = f.get_tensor(name)
                    else:
                        unused.append(name)
        if "lm_head.weight" not in loaded and raw.get("tie_word_embeddings") and "model.embed_tokens.weight" in loaded:
            loaded["lm_head.weight"] = loaded["model.embed_tokens.weight"]
        missing = sorted(set(wanted) - set(loaded))
        if missing:
            raise KeyError(f"{path}: checkpoint lacks {len(missing)} parameter(s), e.g. {missing[:3]}")
        for name, t in loaded.items():
            if tuple(t.shape) != tuple(wanted[name].shape):
                raise ValueError(f"{path}: {name} has shape {tuple(t.shape)}, the config implies {tuple(wanted[name].shape)}")
        model.load_state_dict({k: v.to(torch.float32) for k, v in loaded.items()})
        model.unused_checkpoint_keys = sorted(unused)
        return model.to(device=device, dtype=dtype).eval()

    # ------------------------------------------------------------------ dense reference
    @torch.inference_mode()
    def dense_forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        """All loops dense, no cache compression: logits of the last position (the
        looped model without FlashLoop's lazy updates)."""
        return self.lm_head(self._dense_hidden(input_ids)[:, -1]).float()

    @torch.inference_mode()
    def forward(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None, **kwargs):
        """Logits ``[1, T, vocab]`` of every position with every loop dense and no cache
        (the model without FlashLoop).  Inside ``flashloop_amd.hooks.flashloop(model)``
        calls are routed through ``FlashLoopEngine`` instead."""
        if kwargs.get("past_key_values") is not None:
            raise ValueError("the dense model keeps no cache; use flashloop(model) or FlashLoopEngine to decode")
        if attention_mask is not None and not bool(attention_mask.bool().all()):
            raise ValueError("padded inputs are not supported")
        return DenseOutput(self.lm_head(self._dense_hidden(input_ids)).float())

    def _dense_hidden(self, input_ids: torch.Tensor) -> torch.Tensor:
        bb = self.model
        h = bb.embed_tokens(input_ids)
        t = input_ids.shape[1]
        cos, sin = bb.rotary_emb(h, torch.arange(t, device=input_ids.device)[None])
        for _ in range(self.config.total_ut_steps):
            for layer in bb.layers:
                a = layer.self_attn
                x = layer.input_layernorm(h)
                q = a.q_proj(x).view(1, t, -1, a.head_dim).transpose(1, 2)
                k = a.k_proj(x).view(1, t, -1, a.head_dim).transpose(1, 2)
                v = a.v_proj(x).view(1, t, -1, a.head_dim).transpose(1, 2)
                q, k = apply_rope(q, k, cos, sin)
                o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
                o = a.o_proj(o.transpose(1, 2).reshape(1, t, -1))
                h = h + layer.input_layernorm_2(o)
                h = h + layer.post_attention_layernorm_2(layer.mlp(layer.post_attention_layernorm(h)))
            h = bb.norm(h)
        return h

    @torch.inference_mode()
    def generate(self, input_ids: torch.Tensor, *, max_new_tokens: int, eos_token_id: int | None = None) -> torch.Tensor:
        """Greedy generation with every loop dense and no cache (the looped model without
        FlashLoop).  Inside ``flashloop_amd.hooks.flashloop(model)`` this method is routed
        through ``FlashLoopEngine`` instead."""
        ids = input_ids
        for _ in range(int(max_new_tokens)):
            nxt = torch.argmax(self.dense_forward(ids), dim=-1, keepdim=True)
            ids = torch.cat([ids, nxt], dim=1)
            if eos_token_id is not None and int(nxt.item()) == int(eos_token_id):
                break
        return ids
