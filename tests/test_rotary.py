"""The head reordering that lets the HIP kernels (which pair 8-dim groups) take any rotary half-width
(hummingbird_amd.rotary), checked on the CPU against the oracle's rotate-half RoPE (sa3jax/dit.py:90-98):
RoPE of the reordered head with the widened tables is the reordered RoPE of the head, bit for bit, and dot
products are unchanged."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import rotary
from oracle.dense import rope, rope_tables

CASES = [(64, h) for h in (1, 3, 5, 12, 17, 20, 30, 31)] + [(128, h) for h in (9, 36, 45, 63)]


@pytest.mark.parametrize("head_dim,half", CASES)
def test_reordered_rope_is_the_reordered_reference(head_dim, half):
    rng = np.random.default_rng(head_dim + half)
    ha = rotary.aligned_half(half)
    assert ha % 8 == 0 and half <= ha < half + 8 and 2 * ha <= head_dim
    order = np.array(rotary.head_order(head_dim, half))
    assert sorted(order) == list(range(head_dim))                    # a permutation
    inv = (10000.0 ** (-np.arange(half) / half)).astype(np.float32)
    x, y = rng.standard_normal((2, 40, head_dim)).astype(np.float32)
    cos, sin = rope_tables(40, inv)
    ref_x, ref_y = rope(x, cos, sin, "fp32"), rope(y, cos, sin, "fp32")
    # the kernels' tables: (L, half) padded to (L, ha) by pad_tables; the oracle duplicates them over both halves
    c, s = rotary.pad_tables(torch.from_numpy(cos[:, :half].copy()), torch.from_numpy(sin[:, :half].copy()), half)
    assert c.shape == (40, ha) and torch.all(c[:, half:] == 1) and torch.all(s[:, half:] == 0)
    c2 = np.concatenate([c.numpy(), c.numpy()], axis=1)
    s2 = np.concatenate([s.numpy(), s.numpy()], axis=1)
    got_x, got_y = rope(x[:, order], c2, s2, "fp32"), rope(y[:, order], c2, s2, "fp32")
    assert np.array_equal(got_x, ref_x[:, order])
    np.testing.assert_allclose((got_x.astype(np.float64) * got_y).sum(-1), (ref_x.astype(np.float64) * ref_y).sum(-1),
                               rtol=1e-12, atol=1e-12)


def test_reorder_sections_moves_only_the_marked_heads():
    H, D, half = 3, 64, 12
    order = rotary.head_order(D, half)
    x = torch.arange(2 * 5 * H * D, dtype=torch.float32).reshape(2, 5 * H * D)
    got = rotary.reorder_sections(x, H, D, half, (True, True, False, True, True))
    for sec in range(5):
        for h in range(H):
            base = (sec * H + h) * D
            want = x[:, base + torch.tensor(order)] if sec != 2 else x[:, base:base + D]
            assert torch.equal(got[:, base:base + D], want), (sec, h)
    w = torch.arange(D, dtype=torch.float32)
    assert torch.equal(rotary.reorder_dims(w, D, half), w[torch.tensor(order)])
    with pytest.raises(ValueError):
        rotary.head_order(64, 33)
