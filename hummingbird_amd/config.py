"""Hot-path configuration: the reference's DiTConfig / SameConfig fields the two attention kernels read
(sa3jax/config.py:36-78, 81-141), with `"hip"` added to both `attention` literals.

`attention="hip"` selects the MI355X kernels (`dense_attention` / `band_attention` of this package). The other
values keep the reference's meaning: `"xla"` is the plain chain (here restated in torch, any device), and
`"fused"` / `"pallas"` name the TPU kernels, which do not exist on this platform and therefore run the plain
chain exactly as the reference does off-TPU (sa3jax/config.py:54-56, 112-114).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Literal


@dataclass(frozen=True)
class DiTConfig:
    """DiT self-attention fields (sa3jax/config.py:36-78)."""

    embed_dim: int = 1024
    num_heads: int = 16
    differential: bool = False
    qk_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    num_memory_tokens: int = 64
    attention: Literal["xla", "fused", "hip"] = "xla"
    fused_min_tokens: int = 800  # the TPU kernel's floor; the "hip" kernel has none

    @property
    def head_dim(self) -> int:
        return self.embed_dim // self.num_heads

    @property
    def rope_dim(self) -> int:
        """`RotaryEmbedding(max(head_dim // 2, 32))`: partial rotary (sa3jax/config.py:67-70)."""
        return max(self.head_dim // 2, 32)


@dataclass(frozen=True)
class SameConfig:
    """SAME-L attention fields (sa3jax/config.py:81-141)."""

    channels: int = 128
    c_mults: tuple[int, ...] = (6,)
    stride: int = 16
    transformer_depth: int = 6
    dim_heads: int = 64
    ff_mult: int = 3
    differential: bool = True
    dyt: bool = True
    sinusoidal_blocks: int = 0
    sliding_window: tuple[int, int] | None = None
    attention: Literal["xla", "pallas", "hip"] = "xla"

    @property
    def dim(self) -> int:
        return self.channels * self.c_mults[0]

    @property
    def num_heads(self) -> int:
        return self.dim // self.dim_heads

    @property
    def ff_inner(self) -> int:
        return self.dim * self.ff_mult

    def sinusoidal(self, index: int) -> bool:
        """Block `index` gates its GLU with sin(pi x) instead of SiLU: `sinusoidal_blocks` counts from the end
        (sa3jax/same_l.py:172-179)."""
        return index >= self.transformer_depth - self.sinusoidal_blocks + 1

    @property
    def sub_chunk_size(self) -> int:
        """One latent plus `stride` new-token positions: the band half-width w (sa3jax/config.py:129-132)."""
        return self.stride + 1


# The `medium` preset's attention geometry (sa3jax/config.py:171-185) with the MI355X kernels selected.
MEDIUM_DIT = DiTConfig(embed_dim=1536, num_heads=24, differential=True, attention="hip")
MEDIUM_SAME_L = SameConfig(channels=256, transformer_depth=12, sliding_window=(1, 1), sinusoidal_blocks=8,
                           attention="hip")
