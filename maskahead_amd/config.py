"""Cache quantization settings (the reference's ``maskahead.config.QuantizationConfig``,
config.py:34-86): same fields, defaults and validation.  The kernels of this package are
built for 4-bit packed or 16-bit K/V with key token groups and value channel groups of
32 and float16 scale/zero; other valid settings raise KernelUnavailableError where a
kernel would need them (``require_built``)."""

from __future__ import annotations

from dataclasses import dataclass

from ._native import KernelUnavailableError


def _validate_bits(name: str, bits: int) -> None:
    """config.py:28-30: packed widths 2 and 4, or 16 (unquantized)."""
    if bits not in (2, 4, 16):
        raise ValueError(f"{name} must be 2, 4, or 16; got {bits}")


@dataclass(slots=True)
class QuantizationConfig:
    k_bits: int = 4
    v_bits: int = 4
    key_token_group: int = 32
    value_channel_group: int = 32
    residual_tokens: int = 32
    param_dtype: str = "float16"
    key_mode: str = "channel"
    key_bias: str = "none"
    rotation: str = "none"

    def validate(self, *, head_dim: int | None = None) -> None:
        """config.py:61-86."""
        _validate_bits("k_bits", self.k_bits)
        _validate_bits("v_bits", self.v_bits)
        if self.rotation not in ("none", "hadamard"):
            raise ValueError(f"unknown rotation: {self.rotation}")
        if self.rotation != "none" and head_dim is not None and head_dim & (head_dim - 1):
            raise ValueError("hadamard rotation needs a power-of-two head_dim")
        if self.key_bias not in ("none", "mean"):
            raise ValueError(f"unknown key_bias: {self.key_bias}")
        if self.key_mode not in ("channel", "token"):
            raise ValueError(f"unknown key_mode: {self.key_mode}")
        if self.key_token_group <= 0 or self.key_token_group % 8 != 0:
            raise ValueError("key_token_group must be a positive multiple of 8")
        if self.value_channel_group <= 0 or self.value_channel_group % 8 != 0:
            raise ValueError("value_channel_group must be a positive multiple of 8")
        if self.residual_tokens < 0:
            raise ValueError("residual_tokens must be non-negative")
        if head_dim is not None and head_dim % self.value_channel_group:
            raise ValueError(
                f"head_dim={head_dim} must be divisible by value_channel_group={self.value_channel_group}")
        if self.k_bits < 16 and self.key_token_group % (8 // self.k_bits):
            raise ValueError("key_token_group is incompatible with packed key bit width")
        if self.v_bits < 16 and self.value_channel_group % (8 // self.v_bits):
            raise ValueError("value_channel_group is incompatible with packed value bit width")

    @property
    def packed(self) -> bool:
        return self.k_bits < 16 or self.v_bits < 16

    def require_built(self) -> None:
        """Raise KernelUnavailableError for a valid setting this library has no kernel for."""
        if self.packed:
            if (self.k_bits, self.v_bits) != (4, 4):
                raise KernelUnavailableError(
                    f"k_bits={self.k_bits}, v_bits={self.v_bits}: only 4-bit packed K and V (or 16-bit) are built")
            if self.key_token_group != 32 or self.value_channel_group != 32:
                raise KernelUnavailableError("only key_token_group = value_channel_group = 32 is built")
            if self.param_dtype != "float16":
                raise KernelUnavailableError("only float16 scale/zero (param_dtype) is built")
            if self.key_mode != "channel":
                raise KernelUnavailableError("quant.key_mode='token' is not built")
        if self.key_bias != "none" or self.rotation != "none":
            raise KernelUnavailableError("key_bias / rotation transforms are not built")
