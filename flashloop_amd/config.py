"""Validated FlashLoop settings (mirror of ``FlashLoopConfig``, flashloop/config.py:14-77)."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class FlashLoopConfig:
    prefill_fraction_loop3: float = 0.25
    prefill_fraction_loop4: float = 0.10
    decode_key_fraction: float = 0.10
    kv_bits: int = 4
    group_size: int = 64
    residual_length: int = 64
    enable_token_sparse_prefill: bool = True
    enable_sparse_decode: bool = True
    quantize_cross_loop_kv: bool = True
    decode_capacity: int = 4096  # packed-prefix room reserved for decode tokens

    def __post_init__(self) -> None:
        if not 0.0 < self.prefill_fraction_loop4 <= self.prefill_fraction_loop3 <= 1.0:
            raise ValueError("prefill fractions require 0 < loop4 <= loop3 <= 1")
        if not 0.0 < self.decode_key_fraction <= 1.0:
            raise ValueError("decode_key_fraction must be in (0, 1]")
        if self.kv_bits != 4:
            raise ValueError("the production FlashLoop codec is fixed to 4 bits")
        if self.group_size != 64:
            raise ValueError("the production FlashLoop codec uses group_size=64")
        if self.residual_length != 64:
            raise ValueError("the production FlashLoop cache uses residual_length=64")
        if not self.quantize_cross_loop_kv:
            raise ValueError("this build implements the quantized cross-loop cache only")
        for name in ("enable_token_sparse_prefill", "enable_sparse_decode"):
            if not isinstance(getattr(self, name), bool):
                raise TypeError(f"{name} must be bool")
        if self.decode_capacity < 0:
            raise ValueError("decode_capacity must be non-negative")

    @property
    def effective_prefill_fractions(self) -> tuple[float, float]:
        if not self.enable_token_sparse_prefill:
            return (1.0, 1.0)
        return (self.prefill_fraction_loop3, self.prefill_fraction_loop4)

    @property
    def effective_decode_key_fraction(self) -> float:
        return self.decode_key_fraction if self.enable_sparse_decode else 1.0


def validate_ouro_model(model) -> None:
    """Shape contract of the engine (flashloop/config.py:92-134): 4 loops, MHA, head_dim 128."""
    cfg = model.config
    if int(getattr(cfg, "total_ut_steps", 0)) != 4:
        raise ValueError("FlashLoop requires exactly four recurrent loops")
    if int(cfg.head_dim) != 128:
        raise ValueError("FlashLoop kernels require head_dim 128")
    if int(cfg.num_attention_heads) != int(cfg.num_key_value_heads):
        raise ValueError("FlashLoop kernels require multi-head attention (no grouped KV)")
