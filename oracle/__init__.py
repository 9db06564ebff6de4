"""CPU oracle for the two differential-attention kernels. TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the arithmetic of the reference's XLA attention paths
(kelechi-c/hummingbird `sa3jax`), with each function citing the reference file:line it follows:

* `oracle.dense` -- DiT self-attention: RMSNorm -> RoPE -> V-mask -> two softmax attentions -> subtract
  (sa3jax/dit.py:45-57, 82-119, 122-176, 185-200), plus the fused-kernel cast profile
  (sa3jax/dense_attention.py:43-101).
* `oracle.band` -- SAME-L sliding-window attention: DyT -> RoPE -> two band attentions -> subtract
  (sa3jax/same_l.py:58-69, 84-169), plus the fused-kernel cast profile (sa3jax/band_attention.py:43-120).
* `oracle.cross` -- DiT cross-attention: q/q_diff RMSNorm, the context's k/k_diff RMSNorm, two softmax
  attentions over the context, subtract (sa3jax/dit.py:203-215, 274-284, 131-176), built from `oracle.dense`.
* `oracle.block` -- the SAME-L decoder block (sa3jax/same_l.py:58-69, 151-192): DyT, to_qkv, band attention,
  to_out, residual; DyT, glu_proj, the GLU gate, proj_out, residual; built from `oracle.band`.
* `oracle.dit` -- the DiT denoiser around the self- and cross-attention (sa3jax/dit.py:31-79, 218-361) and the
  pingpong sampler with its LogSNR-shift schedule (sa3jax/sampling.py:65-118), built from `oracle.dense` and
  `oracle.cross`.
* `oracle.bf16` -- round-to-nearest-even bfloat16 emulation for the cast points.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg may import this package,
and only as the reference results that outputs are compared against or as the timed CPU baseline. The product
(`hummingbird_amd`) never imports it.

How each function is pinned (the checks live in tests/test_oracle.py):

* bf16 rounding: against torch's `.to(torch.bfloat16)` (a library routine) on random values, ties and
  extremes.
* RMSNorm: unit RMS of the output at w=1, eps=0; scale invariance; eps limit.
* RoPE tables / rotate-half: against an independent complex-number rotation of the pairs
  (x[d] + i x[d+half]) * exp(i * theta); norm preservation; inv_freq=0 is the identity; the relative-position
  property of the rotated dot product.
* SDPA and the whole dense chain (fp32 profile): against torch.nn.functional.scaled_dot_product_attention in
  float64 on the CPU (a library routine), plus q=0 -> mean of V, L=1 -> V, key permutation invariance.
* Differential subtraction: q_d=q, k_d=k gives exactly 0 at lambda=1; linearity in lambda.
* Band: the grouped three-window restatement (same_l.py:103-148) against brute-force masked attention on the
  CPU via torch SDPA with an explicit boolean mask; w >= S-1 equals dense unmasked attention; translation
  equivariance away from the edges.
* DyT: against torch.tanh; alpha=0 and gamma=0 special cases.
* Cross-attention (tests/test_cross.py): against torch's SDPA in float64 over the context (sections sliced by
  index); bit-identical to the dense chain without RoPE and mask when the context has as many tokens as there
  are queries; one context token gives (1 - lambda) v, q = 0 gives (1 - lambda) mean(v); exact cancellation of
  identical branches and linearity in lambda.
* SAME-L block (tests/test_block.py): the GLU against torch's SiLU and sine in float64; its bf16 cast points on
  a known case; the block with both branches off is the identity; the FF branch alone against a torch float64
  composition; the attention branch alone against torch's SDPA under an explicit band mask.

* DiT denoiser and sampler (tests/test_sampler.py): the schedule against the values the reference documents for
  the shipped sampler (t[1] is 0.99609375 in bf16 and 0.994140625 in half) and its special cases; the pingpong
  step against closed forms with stub denoisers; the timestep features at their end-point frequencies; the 1x1
  convolution against a brute-force sum; the depth-0 denoiser against its linear maps composed in float64; the
  adaLN block on known cases (cancelling branches give the identity, the local constant on the latent tokens
  only, the sigmoid(1 - gate) gate, the x (1 + scale) + shift modulation through an exactly-identity
  feed-forward).

Parity unpinned: the bit-level behaviour of XLA itself (where it rounds einsum outputs, its exp/cos/sin/tanh
ulps and reduction order) cannot be pinned here because jax is not installed; the oracle fixes the cast
points the reference's source states, and the tolerance contract (bf16: max-abs <= 2e-2 and cosine >=
0.9999; fp32: <= 1e-5 relative) absorbs the remaining ulp-level differences.
"""
from oracle import band, bf16, block, cross, dense, dit  # noqa: F401
