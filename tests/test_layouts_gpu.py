"""GPU checks of the C ABI's layout and stream contract:

* padded rows: inputs that are column slices of wider tensors (row stride > the packed width) give results
  bit-identical to contiguous inputs, for the dense, band and cross-attention entry points;
* a batch stride that is not N * row stride is rejected by the Python operators with ValueError;
* HIP graph capture: the dense, band and cross-attention calls captured into one graph and replayed three times,
  with eager work and synchronisations between the replays, match the eager results bit for bit on every replay
  (nothing in these entry points records a memset or allocates).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from hummingbird_amd import band_attention as ba
from hummingbird_amd import cross_attention as xattn
from hummingbird_amd import dense_attention as da
from hummingbird_amd import workloads

pytestmark = pytest.mark.gpu
DEV = "cuda"


def announce(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def dev(a, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t.to(dtype) if dtype is not None else t


def padded(x: torch.Tensor, extra: int) -> torch.Tensor:
    """The same values as a column slice of a tensor `extra` columns wider (row stride = width + extra)."""
    wide = torch.full((*x.shape[:-1], x.shape[-1] + extra), float("nan"), dtype=x.dtype, device=x.device)
    wide[..., : x.shape[-1]] = x
    return wide[..., : x.shape[-1]]


def dense_call(inp, qkv):
    freq, valid = dev(inp["inv_freq"]), dev(inp["valid"])
    cos, sin, mask = da.tables(qkv.shape[1], freq, valid, inp["head_dim"], qkv.dtype)
    return da.dense_attention(qkv, dev(inp["q_weight"]), dev(inp["k_weight"]), cos, sin, mask, inp["heads"],
                              inp["head_dim"], inp["half"], inp["eps"], lam=dev(inp["lam"]))


def band_call(inp, qkv, window):
    norm = lambda n: {k: torch.as_tensor(np.asarray(v)).to(DEV) for k, v in n.items()}  # noqa: E731
    return ba.band_attention(qkv, norm(inp["q_norm"]), norm(inp["k_norm"]), dev(inp["inv_freq"]), inp["heads"],
                             inp["head_dim"], window, lam=dev(inp["lam"]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_padded_rows_match_contiguous(dtype):
    announce(f"padded rows {dtype}")
    code = "bf16" if dtype == torch.bfloat16 else "fp32"
    inp = workloads.dense_inputs(2, 300, 3, 64, seed=21, dtype=code, ragged=True)
    qkv = dev(inp["qkv"], dtype)
    assert torch.equal(dense_call(inp, qkv), dense_call(inp, padded(qkv, 64)))
    for w in (64, 200):  # the streaming kernel and the tiled pair (bf16); the fp32 kernel
        binp = workloads.band_inputs(1, 500, 2, 64, w, seed=22 + w, dtype=code)
        bqkv = dev(binp["qkv"], dtype)
        assert torch.equal(band_call(binp, bqkv, w), band_call(binp, padded(bqkv, 8), w)), w
    cinp = workloads.cross_inputs(2, 200, 77, 2, 64, seed=23, dtype=code)
    q, kv = dev(cinp["q"], dtype), dev(cinp["kv"], dtype)
    outs = []
    for qq, kk in ((q, kv), (padded(q, 32), padded(kv, 8))):
        ctx = xattn.prepare_cross_kv(kk, dev(cinp["k_weight"]), 2, 64, cinp["eps"])
        outs.append(xattn.cross_attention(qq, ctx, dev(cinp["q_weight"]), cinp["eps"], lam=dev(cinp["lam"])))
    assert torch.equal(outs[0], outs[1])


def test_batch_stride_must_follow_rows():
    announce("batch stride check")
    inp = workloads.dense_inputs(2, 64, 2, 64, seed=24)
    qkv = dev(inp["qkv"], torch.bfloat16)
    gap = torch.zeros((2, 65, qkv.shape[-1]), dtype=qkv.dtype, device=DEV)
    gap[:, :64] = qkv
    with pytest.raises(ValueError):
        dense_call(inp, gap[:, :64])  # stride(0) = 65 rows, not 64


def test_graph_replays_match_eager():
    """One HIP graph holding a dense, a band and a cross-attention call on preallocated buffers."""
    announce("graph capture: dense + band + cross")
    dinp = workloads.dense_inputs(2, 400, 4, 64, seed=25)
    binp = workloads.band_inputs(1, 3000, 2, 64, 128, seed=26)
    cinp = workloads.cross_inputs(2, 400, 257, 4, 64, seed=27)
    qkv, bqkv = dev(dinp["qkv"], torch.bfloat16), dev(binp["qkv"], torch.bfloat16)
    q, kv = dev(cinp["q"], torch.bfloat16), dev(cinp["kv"], torch.bfloat16)
    ctx = xattn.prepare_cross_kv(kv, dev(cinp["k_weight"]), 4, 64, cinp["eps"])
    # tables, weights and workspaces are made outside the graph; the calls inside allocate only their outputs
    freq, valid = dev(dinp["inv_freq"]), dev(dinp["valid"])
    cos, sin, mask = da.tables(400, freq, valid, 64, torch.bfloat16)
    qw, kw, lam = dev(dinp["q_weight"]), dev(dinp["k_weight"]), dev(dinp["lam"])
    ws = torch.empty(da.workspace_bytes(torch.bfloat16, 2, 400, 4, 64), dtype=torch.uint8, device=DEV)
    norm = lambda n: {k: torch.as_tensor(np.asarray(v)).to(DEV) for k, v in n.items()}  # noqa: E731
    qn, kn, bfreq, blam = norm(binp["q_norm"]), norm(binp["k_norm"]), dev(binp["inv_freq"]), dev(binp["lam"])
    cqw, clam = dev(cinp["q_weight"]), dev(cinp["lam"])

    def calls():
        a = da.dense_attention(qkv, qw, kw, cos, sin, mask, 4, 64, 32, 1e-6, lam=lam, workspace=ws)
        b = ba.band_attention(bqkv, qn, kn, bfreq, 2, 64, 128, lam=blam)
        c = xattn.cross_attention(q, ctx, cqw, cinp["eps"], lam=clam)
        return a, b, c

    eager = [t.clone() for t in calls()]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        calls()  # warm-up on the capture stream (table caches, library load)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = calls()
    for replay in range(3):
        noise = torch.randn(1 << 20, device=DEV).sum()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        for name, got, ref in zip(("dense", "band", "cross"), outs, eager):
            assert torch.equal(got, ref), f"replay {replay}: {name} differs from the eager call"
