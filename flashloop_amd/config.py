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
            raise ValueError(f"token retention must satisfy 0 < loop-4 fraction ({self.prefill_fraction_loop4}) <= loop-3 fraction ({self.prefill_fraction_loop3}) <= 1")
        if not 0.0 < self.decode_key_fraction <= 1.0:
            raise ValueError(f"decode key retention {self.decode_key_fraction} lies outside (0, 1]")
        if self.kv_bits != 4:
            raise ValueError(f"kv_bits={self.kv_bits}: the int4 residual codec has no other width")
        if self.group_size != 64:
            raise ValueError(f"group_size={self.group_size}: codes are grouped by 64 tokens / 64 channels only")
        if self.residual_length != 64:
            raise ValueError(f"residual_length={self.residual_length}: the BF16 tail keeps exactly 64 tokens")
        if not self.quantize_cross_loop_kv:
            raise ValueError("quantize_cross_loop_kv=False (a BF16 cross-loop cache) is not part of this build")
        for name in ("enable_token_sparse_prefill", "enable_sparse_decode"):
            if not isinstance(getattr(self, name), bool):
                raise TypeError(f"{name} takes True or False, got {getattr(self, name)!r}")
        if self.decode_capacity < 0:
            raise ValueError(f"decode_capacity={self.decode_capacity} is negative")

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
        raise ValueError(f"total_ut_steps={getattr(cfg, 'total_ut_steps', None)}: the cross-loop cache holds four loops")
    if int(cfg.head_dim) != 128:
        raise ValueError(f"head_dim={cfg.head_dim}: the HIP kernels are built for 128 channels per head")
    if int(cfg.num_attention_heads) != int(cfg.num_key_value_heads):
        raise ValueError("grouped KV heads are not supported: the readers take one K/V head per query head")
