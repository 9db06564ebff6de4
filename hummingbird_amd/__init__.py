"""hummingbird_amd: MI355X-native (gfx950) kernels for Stable Audio 3's two differential attentions.

* `hummingbird_amd.dense_attention.dense_attention` / `.tables` -- DiT self-attention
  (reference: sa3jax/dense_attention.py)
* `hummingbird_amd.band_attention.band_attention` / `.rope_tables` -- SAME-L band attention
  (reference: sa3jax/band_attention.py)
* `hummingbird_amd.config.DiTConfig` / `SameConfig` with `attention="hip"`, and the call sites
  `hummingbird_amd.dit.self_attention` and `hummingbird_amd.same_l.attention`
  (reference: sa3jax/dit.py:185-200, sa3jax/same_l.py:151-169)

The kernels live in `libhummingbird_amd.so` (C ABI: include/hummingbird_amd.h), built with
`python -m hummingbird_amd._build`. As in the reference package, the operators are reached through their
modules (`from hummingbird_amd.dense_attention import dense_attention`).
"""
__version__ = "0.1.0"
