"""The no-allocation entry point hb_dense_diffattn_noalloc on the GPU, through the C ABI.

It runs the kernels of hb_dense_diffattn with their workspace in the library's own device array instead of a
caller's buffer, so its output must be bit-identical to hb_dense_diffattn's on the same inputs. Two calls in a row
on one GPU, the second with a smaller input (the array keeps the first call's contents), then an fp32 call, then a
shape too large for the array, which is rejected before anything runs.
"""
from __future__ import annotations

import pytest
import torch

from hummingbird_amd import _lib
from hummingbird_amd import dense_attention as da
from hummingbird_amd import workloads
from oracle import dense as odense
from tests.util import assert_bf16_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(B, L, H, D, half, dtype, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    qkv = torch.randn((B, L, 5 * H * D), device=DEV, generator=gen).to(dtype)
    qw = 1 + 0.02 * torch.randn(D, device=DEV, generator=gen)
    kw = 1 + 0.02 * torch.randn(D, device=DEV, generator=gen)
    lam = 0.2 + 0.6 * torch.rand(H, device=DEV, generator=gen)
    valid = torch.ones((B, L), device=DEV)
    valid[:, L - min(16, L // 4):] = 0
    cos, sin, mask = da.tables(L, torch.from_numpy(workloads.inv_freq(half)).to(DEV), valid, D, dtype)
    return dict(B=B, L=L, H=H, D=D, half=half, dtype=dtype, qkv=qkv, qw=qw, kw=kw, lam=lam, cos=cos, sin=sin,
                mask=mask)


def args(c, out):
    code = da.dtype_code(c["dtype"])
    H, D = c["H"], c["D"]
    return (torch.cuda.current_stream().cuda_stream, c["qkv"].data_ptr(), code, 5 * H * D, c["qw"].data_ptr(),
            c["kw"].data_ptr(), c["cos"].data_ptr() if c["half"] else None, c["sin"].data_ptr() if c["half"] else None,
            c["half"], c["mask"].data_ptr(), c["lam"].data_ptr(), out.data_ptr(), c["B"], c["L"], H, D, 1e-6)


def run_both(lib, c):
    """(no-allocation output, workspace output) for case c."""
    shape = (c["B"], c["L"], c["H"] * c["D"])
    a = torch.full(shape, float("nan"), dtype=c["dtype"], device=DEV)
    b = torch.full(shape, float("nan"), dtype=c["dtype"], device=DEV)
    _lib.check(lib.hb_dense_diffattn_noalloc(*args(c, a)), "noalloc")
    need = int(lib.hb_dense_workspace_size(da.dtype_code(c["dtype"]), c["B"], c["L"], c["H"], c["D"]))
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    _lib.check(lib.hb_dense_diffattn(*args(c, b), ws.data_ptr(), need), "workspace")
    torch.cuda.synchronize()
    return a, b


def test_noalloc_matches_workspace_entry_point():
    lib = _lib.load()
    assert lib.hb_dense_noalloc_max_bytes() == 64 << 20
    seq = [(2, 2584, 24, 64, 32, torch.bfloat16, 1),   # the 120 s clip: 49.5 MB of the 64 MiB array
           (1, 300, 2, 64, 16, torch.bfloat16, 2),     # smaller, over what the first call left
           (2, 150, 3, 128, 64, torch.float32, 3)]     # fp32 path (another kernel pair on the same array)
    for B, L, H, D, half, dtype, seed in seq:
        print(f"\n[case] noalloc B={B} L={L} H={H} D={D} half={half} {dtype}", flush=True)
        c = case(B, L, H, D, half, dtype, seed)
        a, b = run_both(lib, c)
        assert not torch.isnan(a.float()).any()
        assert torch.equal(a.view(torch.int16) if dtype == torch.bfloat16 else a.view(torch.int32),
                           b.view(torch.int16) if dtype == torch.bfloat16 else b.view(torch.int32))
        if (B, L) == (1, 300):  # and against the oracle (the parity contract)
            host = lambda t: t.float().cpu().numpy()  # noqa: E731
            ref = odense.dense_xla(host(c["qkv"]), host(c["qw"]), host(c["kw"]), workloads.inv_freq(half),
                                   host(c["mask"]), H, D, 1e-6, host(c["lam"]), "bf16")
            assert_bf16_parity(host(a), ref, "noalloc vs oracle")


def test_noalloc_rejects_shapes_beyond_the_array():
    lib = _lib.load()
    print("\n[case] noalloc too large", flush=True)
    # every buffer is sized for the rejected shape (L = 6000: 92 MB of qkv), so that a regression of the size
    # check would show up as a wrong status code rather than as kernels reading past short buffers
    c = case(2, 6000, 24, 64, 32, torch.bfloat16, 4)
    need = int(lib.hb_dense_workspace_size(0, 2, 6000, 24, 64))
    assert need > lib.hb_dense_noalloc_max_bytes()
    out = torch.empty((2, 6000, 24 * 64), dtype=torch.bfloat16, device=DEV)
    a = list(args(c, out))
    assert lib.hb_dense_diffattn_noalloc(*a) == 8  # HB_ERR_WORKSPACE, before anything is launched
    assert b"no-allocation scratch" in lib.hb_last_error()
    with pytest.raises(ValueError):
        _lib.check(lib.hb_dense_diffattn_noalloc(*a), "noalloc")
