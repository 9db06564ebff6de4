"""Values derived from a caller's tensors (fp32 copies of bf16 biases, packed DyT vectors, RoPE tables), kept while
those tensors live and are unchanged, so that a loop that passes the same parameters on every call (a decoder's
blocks, a sampler's steps) converts them once instead of once per call.

An entry is keyed by the identities of its source tensors plus a key of plain values, and holds the sources'
versions: an in-place edit of a source bumps its version, and the next lookup rebuilds the value. An entry is dropped
when any of its sources is garbage-collected (`weakref.finalize`), so an identity is never matched to a new tensor
that reuses the address, and callers that build fresh tensors per call do not pile entries up.
"""
from __future__ import annotations

import weakref
from typing import Callable

import torch

_CACHE: dict = {}
_CACHE_MAX = 256


def derived(sources: tuple[torch.Tensor, ...], key: tuple, make: Callable[[], object]):
    """`make()`, or the value it returned for the same live, unedited `sources` and the same `key`. Tensors made
    under `torch.inference_mode` keep no version counter, so values derived from them are not kept."""
    if any(s.is_inference() for s in sources):
        return make()
    full = (tuple(id(s) for s in sources), key)
    versions = tuple(s._version for s in sources)
    hit = _CACHE.get(full)
    alive = hit is not None and all(r() is s for r, s in zip(hit[0], sources))
    if alive and hit[1] == versions:
        return hit[2]
    value = make()
    if not alive:  # a new entry: drop it when the first of its sources dies
        if len(_CACHE) >= _CACHE_MAX:
            _CACHE.clear()
        for s in sources:
            weakref.finalize(s, _CACHE.pop, full, None)
    _CACHE[full] = (tuple(weakref.ref(s) for s in sources), versions, value)
    return value


def f32_vector(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    """`t` as a contiguous fp32 vector on `device` (the C ABI's per-channel vectors), converted once per tensor."""
    if t.dtype == torch.float32 and t.device == device and t.is_contiguous():
        return t.reshape(-1)
    return derived((t,), ("f32", device), lambda: t.to(device=device, dtype=torch.float32).contiguous().reshape(-1))
