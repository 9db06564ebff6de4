"""Configuration: the reference's DiTConfig (sa3jax/config.py:36-78) and the SameConfig fields the band kernel
reads (sa3jax/config.py:81-141), with `"hip"` added to both `attention` literals; the sampler's constants
(sa3jax/config.py:158-165, sa3jax/pipeline.py:43-45).

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
    """The DiT's fields (sa3jax/config.py:36-78): the self-attention geometry the kernels read, and the model
    fields `dit.dit_forward` and the sampler read (channels, depth, conditioning widths, feed-forward width,
    norm eps, timestep features)."""

    io_channels: int = 256
    embed_dim: int = 1024
    depth: int = 20
    num_heads: int = 16
    cond_token_dim: int = 768
    global_cond_dim: int = 768
    local_add_cond_dim: int = 257
    num_memory_tokens: int = 64
    ff_mult: float = 4.0
    differential: bool = False
    norm_eps: float = 1e-5
    qk_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    fourier_dim: int = 256
    attention: Literal["xla", "fused", "hip"] = "xla"
    fused_min_tokens: int = 800  # the TPU kernel's floor; the "hip" kernel has none

    @property
    def head_dim(self) -> int:
        return self.embed_dim // self.num_heads

    @property
    def rope_dim(self) -> int:
        """`RotaryEmbedding(max(head_dim // 2, 32))`: partial rotary (sa3jax/config.py:67-70)."""
        return max(self.head_dim // 2, 32)

    @property
    def ff_inner(self) -> int:
        return int(self.embed_dim * self.ff_mult)

    @property
    def adaln_dim(self) -> int:
        """Scale, shift and gate of the self-attention and the feed-forward: 6 * embed_dim."""
        return 6 * self.embed_dim


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
MEDIUM_DIT = DiTConfig(embed_dim=1536, depth=24, num_heads=24, differential=True, attention="hip")
MEDIUM_SAME_L = SameConfig(channels=256, transformer_depth=12, sliding_window=(1, 1), sinusoidal_blocks=8,
                           attention="hip")

# The sampler (sa3jax/config.py:163-164; the LogSNR shift of sa3jax/pipeline.py:43-45).
SAMPLER_STEPS = 8
SIGMA_MAX = 1.0
ANCHOR_LOGSNR = -6.2
LOGSNR_END = 2.0
