"""Per-role precision presets: the counterpart of the reference's `Dtype` (sa3jax/dtypes.py:23-58) in torch dtypes.

Each field is the dtype of one role: `compute` is the attention inputs' and outputs' dtype (the kernels' `qkv` and
`out`), `norm` and `rope` are the fp32 islands of the norms and rotary embedding, `weight` is storage. The three
presets are the reference's: BF16 (the default), FP16, and FP32_PARITY (fp32 everywhere, the parity path). The
attention kernels read the compute dtype from their inputs; under BF16 and FP16 their matrix-core operands are
bf16, as in the reference's fused kernels (dense_attention.py:75-77, 83, 90; band_attention.py:85, 94, 101).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Dtype:
    """Storage and compute dtypes per role (sa3jax/dtypes.py:23-37)."""

    weight: torch.dtype = torch.bfloat16
    compute: torch.dtype = torch.bfloat16
    norm: torch.dtype = torch.float32
    rope: torch.dtype = torch.float32
    t: torch.dtype = torch.float32
    audio: torch.dtype = torch.float32
    text: torch.dtype = torch.bfloat16

    @property
    def name(self) -> str:
        """The compute dtype's name, as the reference's `Dtype.name` (`jnp.dtype(compute).name`)."""
        return str(self.compute).removeprefix("torch.")


BF16 = Dtype()
FP32_PARITY = Dtype(weight=torch.float32, compute=torch.float32, norm=torch.float32, rope=torch.float32,
                    t=torch.float32, audio=torch.float32, text=torch.float32)
FP16 = Dtype(weight=torch.float16, compute=torch.float16, norm=torch.float32, rope=torch.float32, t=torch.float32,
             audio=torch.float32, text=torch.float16)
