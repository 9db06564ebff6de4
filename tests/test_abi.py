"""The C ABI on the CPU: the shared library loads, exports every entry point include/hummingbird_amd.h
declares, and its host-side validators reject what the reference rejects at trace time. No kernel is
launched here (no GPU in this environment)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from hummingbird_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hummingbird_amd.h"


def _gpu_visible() -> bool:
    try:
        import torch
        return torch.cuda.device_count() > 0  # counts devices without initialising them
    except Exception:  # noqa: BLE001
        return False


# Tests whose valid-but-fake layouts pass every host check and reach a kernel launch: that launch fails without a
# GPU, which is what they expect; with a GPU it would run a kernel on fake addresses, so they are CPU-only.
cpu_only_launch = pytest.mark.skipif(_gpu_visible(), reason="reaches a kernel launch with fake addresses")


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(hb_[a-z0-9_]+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libhummingbird_amd.so is not built: run `python -m hummingbird_amd._build`")
    return _lib.load()


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for required in ("hb_dense_diffattn", "hb_band_diffattn", "hb_rope_tables", "hb_dense_prep", "hb_dense_attend",
                     "hb_dense_workspace_size", "hb_band_workspace_size", "hb_dense_validate", "hb_band_validate",
                     "hb_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(raw, n)]
    assert not missing, f"declared in the header but not exported: {missing}"


def test_python_prototypes_cover_the_header(lib):
    assert declared_functions() == set(_lib.SIGNATURES)


def test_version_and_status_names(lib):
    assert b"gfx950" in lib.hb_version()
    assert lib.hb_status_name(0) == b"HB_OK"
    assert lib.hb_status_name(2) == b"HB_ERR_SHAPE"
    assert lib.hb_status_name(999) == b"HB_ERR_UNKNOWN"


DENSE_OK = dict(dtype=0, row_stride=5 * 24 * 64, B=2, L=2584, H=24, D=64, half=32, eps=1e-6)


def dense_validate(lib, **kw):
    a = dict(DENSE_OK, **kw)
    return lib.hb_dense_validate(a["dtype"], a["row_stride"], a["B"], a["L"], a["H"], a["D"], a["half"], a["eps"])


@pytest.mark.parametrize("kw,status", [
    ({}, 0),
    ({"D": 128, "H": 12, "row_stride": 5 * 12 * 128, "half": 64}, 0),
    ({"D": 96}, 4),                       # head_dim (reference: dense_attention.py:119-120)
    ({"half": 33}, 5), ({"half": -1}, 5),
    ({"dtype": 7}, 3), ({"dtype": 2}, 0),  # HB_F16: the reference's FP16 preset (dtypes.py:50-58)
    ({"row_stride": 100}, 7), ({"row_stride": 5 * 24 * 64 + 4}, 7),
    ({"L": 0}, 2), ({"B": 0}, 2), ({"H": 0}, 2),
    ({"eps": -1.0}, 10), ({"eps": float("nan")}, 10),
])
def test_dense_validate(lib, kw, status):
    assert dense_validate(lib, **kw) == status
    if status:
        assert lib.hb_last_error()  # a message is recorded


@pytest.mark.parametrize("kw,status", [
    ({}, 0), ({"window": 0}, 0), ({"window": -1}, 6), ({"D": 32}, 4), ({"half": 40}, 5),
])
def test_band_validate(lib, kw, status):
    a = {**dict(dtype=0, row_stride=5 * 8 * 64, B=1, S=82688, H=8, D=64, half=32, window=128), **kw}
    assert lib.hb_band_validate(a["dtype"], a["row_stride"], a["B"], a["S"], a["H"], a["D"], a["half"],
                                a["window"]) == status


def _expected_status(dtype, row_stride, B, N, H, D, half, last):
    """The validators' contract (include/hummingbird_amd.h) restated check by check, in the order the status
    codes take precedence: dtype, head_dim, shape, half, row stride, extent, then the entry point's own last check
    (`last`: the status it returns, or 0)."""
    if dtype not in (0, 1, 2):
        return 3
    if D not in (64, 128):
        return 4
    if B < 1 or N < 1 or H < 1 or B > 65535 or H > 65535 or N > 1 << 28 or B * N * H * D > 1 << 40:
        return 2
    if half < 0 or 2 * half > D:
        return 5
    if row_stride < 5 * H * D or row_stride % 8:
        return 7
    if (B * N - 1) * row_stride + 5 * H * D >= 1 << 48:
        return 7
    return last


_EXTREME = st.sampled_from([0, -1, 65535, 65536, 1 << 28, (1 << 28) + 1, (1 << 31) - 1, -(1 << 31)])
_DIM = st.one_of(st.integers(1, 64), st.integers(1, 64), st.integers(1, 1 << 20), _EXTREME)


@settings(max_examples=400, deadline=None, suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(dtype=st.sampled_from([0, 0, 1, 2, 2, -1, 3]), D=st.sampled_from([64, 64, 128, 128, 96]), B=_DIM, N=_DIM,
       H=_DIM, half=st.one_of(st.sampled_from([0, 8, 16, 32, 64]), st.integers(-1, 70)),
       stride_mult=st.one_of(st.integers(1, 4), st.integers(-1, 1 << 24)),
       stride_pad=st.sampled_from([0, 0, 0, 8, 16, 4, -8]),
       eps=st.sampled_from([0.0, 1e-6, 1e-6, -1e-6, float("inf"), float("nan")]), window=st.integers(-3, 4096))
def test_validators_follow_the_contract(lib, dtype, D, B, N, H, half, stride_mult, stride_pad, eps, window):
    """hb_dense_validate and hb_band_validate against the header's rules on random arguments, including extreme
    strides and shapes (these paths run only host code)."""
    h = max(H, 1)
    row_stride = stride_mult * 5 * h * D + stride_pad
    if not -(1 << 62) < row_stride < 1 << 62:
        return
    eps_ok = eps >= 0.0 and eps != float("inf") and eps == eps
    assert lib.hb_dense_validate(dtype, row_stride, B, N, H, D, half, eps) == \
        _expected_status(dtype, row_stride, B, N, H, D, half, 0 if eps_ok else 10)
    assert lib.hb_band_validate(dtype, row_stride, B, N, H, D, half, window) == \
        _expected_status(dtype, row_stride, B, N, H, D, half, 0 if window >= 0 else 6)


def test_workspace_size(lib):
    # three (B, H, Lp, D) regions (k, k_diff, v prepared) with L padded to the 128-query block
    assert lib.hb_dense_workspace_size(0, 2, 2584, 24, 64) == 3 * 2 * 24 * 2688 * 64 * 2
    assert lib.hb_dense_workspace_size(2, 2, 2584, 24, 64) == 3 * 2 * 24 * 2688 * 64 * 2  # half: bf16 operands
    assert lib.hb_dense_workspace_size(1, 1, 1, 1, 64) == 3 * 128 * 64 * 4
    assert lib.hb_dense_workspace_size(0, 1, 1, 1, 96) == 0


def test_null_pointers_are_rejected_before_any_launch(lib):
    # every pointer NULL: the launcher must return HB_ERR_NULL without touching the GPU
    st = lib.hb_dense_diffattn(None, None, 0, 5 * 64, None, None, None, None, 0, None, None, None, 1, 8, 1, 64,
                               1e-6, None, 0)
    assert st == 1
    st = lib.hb_band_diffattn(None, None, 0, 5 * 64, None, None, None, None, 0, 4, None, None, 1, 8, 1, 64, None, 0)
    assert st == 1
    assert lib.hb_rope_tables(None, None, 4, 10, None, None) == 1
    assert lib.hb_rope_tables(None, None, 0, 10, None, None) == 0  # nothing to build


def test_errors_map_to_python_exceptions(lib):
    with pytest.raises(ValueError, match="HB_ERR_HEAD_DIM"):
        _lib.check(dense_validate(lib, D=96), "dense")
    with pytest.raises(TypeError):
        _lib.check(dense_validate(lib, dtype=7), "dense")


def test_workspace_and_alignment_errors_before_any_launch(lib):
    """Too small or misaligned workspaces and misaligned inputs are rejected with their status codes before any
    GPU call (fake, never dereferenced addresses; the checks read only the pointer values)."""
    B, L, H, D = 1, 200, 2, 64
    need = lib.hb_dense_workspace_size(0, B, L, H, D)
    qkv, w, tab, ws = 0x10000, 0x20000, 0x30000, 0x40000  # 256-byte aligned stand-ins
    args = lambda qkv=qkv, ws=ws, wsb=need, cos=tab: (None, qkv, 0, 5 * H * D, w, w, cos, cos, 32, None, None,  # noqa: E731
                                                      0x50000, B, L, H, D, 1e-6, ws, wsb)
    assert lib.hb_dense_diffattn(*args(wsb=need - 1)) == 8                  # HB_ERR_WORKSPACE: too small
    assert "workspace" in lib.hb_last_error().decode()
    assert lib.hb_dense_diffattn(*args(ws=ws + 16)) == 8                    # HB_ERR_WORKSPACE: not 256-aligned
    assert lib.hb_dense_diffattn(*args(qkv=qkv + 2)) == 7                   # HB_ERR_STRIDE: qkv not 16-aligned
    assert lib.hb_dense_diffattn(*args(cos=tab + 4)) == 7                   # HB_ERR_STRIDE: tables not 16-aligned
    st = lib.hb_band_diffattn(None, qkv + 2, 0, 5 * H * D, w, w, tab, tab, 32, 16, None, 0x50000, B, L, H, D, None, 0)
    assert st == 7
    # bf16 with a window beyond the streaming kernel needs a workspace: missing or short ones are rejected
    need = lib.hb_band_workspace_size(0, B, L, H, D, 32, 200)
    assert need == 3 * B * H * 256 * D * 2
    assert lib.hb_band_workspace_size(0, B, L, H, D, 32, 128) == 0
    # fp32: the optional workspace of the prepared keys, three fp32 (B, H, round_up(S, 128), D) regions
    assert lib.hb_band_workspace_size(1, B, L, H, D, 32, 200) == 3 * B * H * 256 * D * 4
    band = lambda ws, wsb: lib.hb_band_diffattn(None, qkv, 0, 5 * H * D, w, w, tab, tab, 32, 200, None, 0x50000,  # noqa: E731
                                                B, L, H, D, ws, wsb)
    assert band(None, 0) == 8 and band(ws, need - 1) == 8 and band(ws + 64, need) == 8


def test_noalloc_rejects_before_touching_the_gpu(lib):
    """hb_dense_diffattn_noalloc checks the shape and the size of its workspace against its fixed device array
    before it looks the array up or reads a pointer."""
    assert lib.hb_dense_noalloc_max_bytes() == 64 << 20
    fake = 0x100000  # never dereferenced: every call below fails on the host first
    call = lambda L, D=64, qkv=fake: lib.hb_dense_diffattn_noalloc(  # noqa: E731
        None, qkv, 0, 5 * 24 * D, fake, fake, fake, fake, 32, None, None, fake, 2, L, 24, D, 1e-6)
    assert call(6000) == 8       # HB_ERR_WORKSPACE: 3 * 2 * 24 * 6016 * 64 * 2 B > 64 MiB
    assert b"no-allocation" in lib.hb_last_error()
    assert call(100, D=96) == 4  # HB_ERR_HEAD_DIM
    assert call(100, qkv=None) == 1  # HB_ERR_NULL


def test_projection_entry_points_reject_before_any_launch(lib):
    """hb_dit_qkv_proj, hb_dense_attend_qq and hb_proj validate dtype, shapes, strides, alignment and the workspace
    on the host (no kernel is launched here)."""
    fake = 0x100000
    B, L, H, D, E = 2, 100, 4, 64, 256
    need = lib.hb_dense_workspace_size(0, B, L, H, D)

    def qkv(**kw):
        a = dict(h=fake, dtype=0, hs=E, w=fake, wstride=E, E=E, kw=fake, cos=fake, sin=fake, half=32, qq=fake, B=B,
                 L=L, H=H, D=D, eps=1e-6, ws=fake, wsb=need)
        a.update(kw)
        return lib.hb_dit_qkv_proj(None, a["h"], a["dtype"], a["hs"], a["w"], a["wstride"], a["E"], a["kw"], a["cos"],
                                   a["sin"], a["half"], None, a["qq"], a["B"], a["L"], a["H"], a["D"], a["eps"],
                                   a["ws"], a["wsb"])
    assert qkv(dtype=1) == 3            # fp32 is not taken by the fused projection
    assert qkv(D=128) == 4
    assert qkv(H=6) == 2                # heads must be a multiple of 4
    assert qkv(E=100) == 2              # model width a multiple of 64
    assert qkv(half=40) == 5
    assert qkv(hs=E - 8) == 7           # row stride below the width
    assert qkv(h=fake + 8) == 7         # misaligned input
    assert qkv(wsb=need - 1) == 8
    assert qkv(h=None) == 1
    proj = lambda **kw: lib.hb_proj(None, kw.get("x", fake), kw.get("dtype", 0), kw.get("xs", 128), fake,  # noqa: E731
                                    128, fake, kw.get("os", 256), kw.get("N", 10), kw.get("K", 128), kw.get("F", 256))
    assert proj(F=200) == 2 and proj(K=100) == 2 and proj(N=0) == 2 and proj(dtype=1) == 3 and proj(os=100) == 7
    attend = lambda **kw: lib.hb_dense_attend_qq(None, fake, kw.get("dtype", 0), kw.get("rs", 2 * H * D), fake,  # noqa: E731
                                                 fake, fake, fake, 32, None, fake, B, L, H, D, 1e-6,
                                                 kw.get("ws", fake), kw.get("wsb", need))
    assert attend(rs=2 * H * D - 8) == 7 and attend(dtype=1) == 3 and attend(wsb=need - 1) == 8


def test_same_l_projection_entry_points_reject_before_any_launch(lib):
    """hb_proj_glu and hb_proj_residual validate dtype, shapes, strides, alignment, the dyt / out_y pairing and which
    buffers may alias on the host (fake, never dereferenced addresses; no kernel is launched)."""
    x, w, o, h, y, v = 0x100000, 0x400000, 0x800000, 0xC00000, 0x1000000, 0x1400000

    def glu(**kw):
        a = dict(x=x, dtype=0, xs=128, w=w, ws=128, bias=None, sine=1, out=o, os=256, N=10, K=128, F=256)
        a.update(kw)
        return lib.hb_proj_glu(None, a["x"], a["dtype"], a["xs"], a["w"], a["ws"], a["bias"], a["sine"], a["out"],
                               a["os"], a["N"], a["K"], a["F"])
    assert glu(dtype=1) == 3 and glu(dtype=5) == 3       # fp32 is not taken by the fused GEMMs
    assert glu(F=200) == 2 and glu(F=64) == 2 and glu(K=100) == 2 and glu(K=0) == 2 and glu(N=0) == 2
    assert glu(N=(1 << 24) + 1) == 2
    assert glu(x=None) == 1 and glu(w=None) == 1 and glu(out=None) == 1
    assert glu(xs=120) == 7 and glu(x=x + 8) == 7 and glu(ws=100) == 7  # strides and alignment of the operands
    assert glu(os=200) == 7 and glu(out=o + 4) == 7                     # out row stride below F, misaligned out
    assert glu(out=x) == 7 and glu(out=w + 512) == 7                    # out over x, over W (2F rows of it)
    assert glu(out=w + 2 * 256 * 128 * 2 - 16) == 7                    # the last 16 bytes of W
    assert glu(bias=o + 64) == 7                                        # the bias (2F floats) inside out

    def res(**kw):
        a = dict(x=x, dtype=0, xs=128, w=w, ws=128, bias=None, h=h, hs=256, dyt=None, oh=o, oy=None, os=256, N=10,
                 K=128, F=256)
        a.update(kw)
        return lib.hb_proj_residual(None, a["x"], a["dtype"], a["xs"], a["w"], a["ws"], a["bias"], a["h"], a["hs"],
                                    a["dyt"], a["oh"], a["oy"], a["os"], a["N"], a["K"], a["F"])
    assert res(dtype=1) == 3
    assert res(F=128) == 2 and res(K=96) == 2 and res(N=0) == 2
    assert res(h=None) == 1 and res(oh=None) == 1 and res(x=None) == 1
    assert res(dyt=v) == 1 and res(oy=y) == 1                             # dyt and out_y come together
    assert res(hs=200) == 7 and res(h=h + 4) == 7 and res(os=128) == 7    # strides and alignment
    assert res(oh=x) == 7 and res(oh=w) == 7                              # out_h over the GEMM operands
    assert res(oh=h, os=512) == 7                                         # h itself under another row stride
    assert res(oh=h + 8) == 7                                             # partly over h
    assert res(dyt=v, oy=h) == 7 and res(dyt=v, oy=o) == 7 and res(dyt=v, oy=x) == 7
    assert res(dyt=o + 64, oy=y) == 7 and res(bias=o + 64) == 7           # the vectors inside an output


def test_dit_block_entry_points_reject_before_any_launch(lib):
    """hb_rms_modulate and hb_gated_residual validate dtype, shapes, strides, alignment and their optional
    operands on the host (fake, never dereferenced addresses)."""
    fake = 0x100000
    rms = lambda **kw: lib.hb_rms_modulate(  # noqa: E731
        None, kw.get("x", fake), kw.get("dtype", 0), kw.get("xs", 64), kw.get("w", fake), kw.get("eps", 1e-5),
        kw.get("scale", None), kw.get("shift", None), kw.get("ms", 384), kw.get("L", 10), fake, 64, kw.get("N", 20),
        kw.get("C", 64))
    assert rms(dtype=5) == 3 and rms(C=60) == 2 and rms(N=0) == 2 and rms(L=0) == 2
    assert rms(xs=56) == 7 and rms(x=fake + 8) == 7 and rms(w=None) == 1 and rms(eps=-1.0) == 10
    assert rms(scale=fake) == 1                      # scale without shift
    assert rms(scale=fake, shift=fake, N=25) == 2    # rows not a whole number of batches
    assert rms(scale=fake, shift=fake, ms=40) == 7   # batch stride below C
    res = lambda **kw: lib.hb_gated_residual(  # noqa: E731
        None, fake, kw.get("dtype", 0), 64, kw.get("x", fake), kw.get("xs", 64), kw.get("xb", None),
        kw.get("gate", None), kw.get("gs", 64), kw.get("local", None), kw.get("memory", 0), 10, fake, 64, 20, 64)
    assert res(dtype=9) == 3 and res(x=None) == 1 and res(xs=8) == 7 and res(xb=fake + 4) == 7
    assert res(gate=fake, gs=32) == 7 and res(local=fake + 2) == 7 and res(memory=-1) == 2


def test_attention_outputs_that_overlap_their_inputs_are_refused(lib):
    """The attention and projection entry points refuse an output or workspace whose bytes meet a buffer the same
    call reads (HB_ERR_STRIDE), after every other check and before any launch (fake, never dereferenced, otherwise
    valid addresses)."""
    B, L, H, D = 1, 200, 2, 64
    HD = H * D
    qkv, w, tab = 0x100000, 0x400000, 0x500000
    qkv_bytes = L * 5 * HD * 2                                           # 256000 bytes from qkv
    need = lib.hb_dense_workspace_size(0, B, L, H, D)
    ws, out = 0x1000000, 0x2000000                                       # far from everything

    def dense(o=out, wsp=ws):
        return lib.hb_dense_diffattn(None, qkv, 0, 5 * HD, w, w, tab, tab, 32, None, None, o, B, L, H, D, 1e-6, wsp,
                                     need)
    assert dense(o=qkv + qkv_bytes - 16) == 7                            # out's first row in qkv's last bytes
    assert dense(wsp=qkv + 256 * (qkv_bytes // 256 - 1)) == 7            # workspace over qkv (256-byte aligned)
    assert dense(o=ws + need - 8) == 7                                   # out over the workspace's end
    assert "overlaps" in lib.hb_last_error().decode()
    band = lambda o: lib.hb_band_diffattn(None, qkv, 0, 5 * HD, w, w, tab, tab, 32, 16, None, o, B, L, H, D, None, 0)  # noqa: E731
    assert band(qkv + 5 * HD * 2 * 7) == 7                               # out inside qkv's rows
    tneed = lib.hb_band_workspace_size(0, B, L, H, D, 32, 200)
    tiled = lambda wsp: lib.hb_band_diffattn(None, qkv, 0, 5 * HD, w, w, tab, tab, 32, 200, None, out, B, L, H, D,  # noqa: E731
                                             wsp, tneed)
    assert tiled(out - 256 * 4) == 7 and tiled(qkv) == 7                 # the tiled path's workspace over out / qkv
    cneed = lib.hb_cross_workspace_size(0, B, 257, H, D)
    assert lib.hb_cross_prep(None, qkv, 0, 3 * HD, w, B, 257, H, D, 1e-6, qkv + 256 * 8, cneed) == 7
    assert lib.hb_cross_attend(None, qkv, 0, 2 * HD, w, w, None, qkv + 64, B, L, 257, H, D, 1e-6, ws, cneed) == 7
    assert lib.hb_proj(None, qkv, 0, 256, w, 256, qkv + 1024, 256, 64, 256, 256) == 7   # out over x


def test_row_outputs_that_overlap_their_inputs_are_refused(lib):
    """Every row-wise entry point refuses an output that shares an element with a row input or with the other
    output, before any launch (HB_ERR_STRIDE; fake, never dereferenced addresses): partial overlaps within a row and
    across rows, and in place where the kernel's operands are restrict-qualified. Only hb_residual_dyt may update h
    in place (its test on the GPU); interleaved column slices of one buffer are accepted (GPU test)."""
    a, b, c = 0x100000, 0x200000, 0x300000
    N, C = 20, 64                                    # bf16 rows of 128 bytes at a row stride of 64 elements
    dyt = lambda x, out: lib.hb_dyt(None, x, 0, C, c + 0x80000, out, C, N, C)  # noqa: E731
    assert dyt(a, a) == 7 and dyt(a, a + 16) == 7 and dyt(a, a + 128 * (N - 1)) == 7 and dyt(a + 16, a) == 7
    F = 64                                           # glu: proj rows hold 2F, out rows F
    glu = lambda proj, ps, out, os_: lib.hb_glu(None, proj, 0, ps, None, 0, out, os_, N, F)  # noqa: E731
    assert glu(a, 2 * F, a + 2 * F, 2 * F) == 7      # out over the gate half of proj's rows
    assert glu(a, 2 * F, a + 2 * 2 * F * (N - 1), F) == 7  # out starts on proj's last row
    rd = lambda h, x, oh, oy, os_=C: lib.hb_residual_dyt(None, h, 0, C, x, C, None, c + 0x80000 if oy else None,  # noqa: E731
                                                         oh, oy, os_, N, C)
    assert rd(a, b, a + 16, None) == 7               # out_h part of h, not h itself
    assert rd(a, b, b + 128 * 3, None) == 7          # out_h over rows of x
    assert rd(a, b, a, a + 128 * (N - 1)) == 7       # out_y over h's (and out_h's) last row
    assert rd(a, b, c, c + 64) == 7                  # out_y inside out_h's first row
    assert rd(a, b, c, b + 32) == 7                  # out_y over x
    rms = lambda x, out: lib.hb_rms_modulate(None, x, 0, C, c + 0x80000, 1e-5, None, None, C, N, out, C, N, C)  # noqa: E731
    assert rms(a, a) == 7 and rms(a, a + 128 * 5 + 48) == 7
    res = lambda h, x, out: lib.hb_gated_residual(None, h, 0, C, x, C, None, None, C, None, 0, N, out, C, N, C)  # noqa: E731
    assert res(a, b, a) == 7 and res(a, b, b + 16) == 7
    rr = lambda oh, oy: lib.hb_residual_rms(None, a, 0, C, b, C, None, None, C, None, 0, c + 0x80000, 1e-5,  # noqa: E731
                                            None, None, C, N, oh, oy, C, N, C)
    assert rr(a, c) == 7 and rr(c, c) == 7 and rr(c, b + 128 * 2) == 7 and rr(c, c + 128 * (N - 1)) == 7
    assert "overlaps" in lib.hb_last_error().decode()



@cpu_only_launch
def test_row_overlap_check_matches_brute_force(lib):
    """The row-overlap test behind every row-wise entry point, against a byte-by-byte intersection of the rows on
    random layouts (hb_dyt, bf16 rows of 8 elements; fake, never dereferenced addresses). Equal row strides are
    decided exactly, so interleaved rows that share no byte pass the check (and reach the launch, which fails here
    without a GPU); unequal strides are refused whenever the two address ranges meet."""
    import random

    rng = random.Random(11)
    C, esize, base = 8, 2, 0x100000
    for _ in range(400):
        N = rng.randint(1, 6)
        xs, os_ = rng.choice([8, 16, 24, 32]), rng.choice([8, 16, 24, 32])
        if rng.random() < 0.6:
            os_ = xs
        x = base + 16 * rng.randint(0, 24)
        out = base + 16 * rng.randint(0, 24)
        rows = lambda p, s: {p + i * s * esize + k for i in range(N) for k in range(C * esize)}  # noqa: E731
        shared = bool(rows(x, xs) & rows(out, os_))
        st = lib.hb_dyt(None, x, 0, xs, base + 0x80000, out, os_, N, C)
        if shared:
            assert st == 7, (N, xs, os_, x - base, out - base)
        elif xs == os_:
            assert st != 7, (N, xs, os_, x - base, out - base, lib.hb_last_error().decode())
        else:
            x_end, o_end = x + ((N - 1) * xs + C) * esize, out + ((N - 1) * os_ + C) * esize
            assert (st == 7) == (x < o_end and out < x_end), (N, xs, os_, x - base, out - base)

def test_residual_rms_rejects_before_any_launch(lib):
    fake = 0x100000
    call = lambda **kw: lib.hb_residual_rms(  # noqa: E731
        None, fake, kw.get("dtype", 0), kw.get("C", 64), fake, kw.get("C", 64), None, kw.get("gate", None), 384,
        None, 0, kw.get("w", fake), 1e-5, kw.get("scale", None), kw.get("shift", None), 384, 10,
        kw.get("oh", fake), fake, kw.get("C", 64), kw.get("N", 20), kw.get("C", 64))
    assert call(C=4096) == 2                  # the row must fit in registers
    assert call(dtype=1, C=2304) == 2         # fp32 rows up to 2048 as well
    assert call(w=None) == 1 and call(scale=fake) == 1 and call(oh=None) == 1
    assert call(gate=fake, N=25) == 2         # not a whole number of batches
    assert call(dtype=4) == 3


def test_residual_dyt_rejects_before_any_launch(lib):
    """hb_residual_dyt checks dtype, shapes, strides, alignment, the dyt / out_y pairing and which buffers may alias
    on the host (fake, never dereferenced addresses)."""
    fake, other, third = 0x100000, 0x200000, 0x300000
    call = lambda **kw: lib.hb_residual_dyt(  # noqa: E731
        None, kw.get("h", fake), kw.get("dtype", 0), kw.get("hs", 64), kw.get("x", other), kw.get("xs", 64),
        kw.get("bias", None), kw.get("dyt", None), kw.get("oh", fake), kw.get("oy", None), kw.get("os", 64),
        kw.get("N", 20), kw.get("C", 64))
    assert call(dtype=7) == 3 and call(C=60) == 2 and call(N=0) == 2
    assert call(h=None) == 1 and call(x=None) == 1 and call(oh=None) == 1
    assert call(xs=56) == 7 and call(x=other + 8) == 7 and call(dtype=1, C=62) == 2
    assert call(dyt=third) == 1 and call(oy=third) == 1              # dyt and out_y come together
    assert call(dyt=third, oy=third + 8) == 7                         # out_y 16-byte aligned
    assert call(dyt=third, oy=other) == 7                             # out_y aliases x
    assert call(oh=other) == 7                                        # out_h aliases x
    assert call(os=128) == 7                                          # out_h is h with another row stride


def test_strides_whose_extent_overflows_are_refused(lib):
    """A row stride so large that the buffer's rows would span 2^48 elements or more is refused with HB_ERR_STRIDE
    by every entry point that takes one, before the overlap checks compute any byte extent (which would overflow
    int64 for such strides; the host-sanitizer build of test_sanitized_host.py traps that arithmetic)."""
    fake, big = 0x100000, 1 << 61
    H, D = 4, 64
    HD = H * D
    assert dense_validate(lib, row_stride=big) == 7
    assert "2^48" in lib.hb_last_error().decode()
    assert lib.hb_band_validate(0, big, 1, 1000, 8, 64, 32, 128) == 7
    assert lib.hb_cross_validate(0, big, 3 * HD, 2, 100, 257, H, D, 1e-6) == 7
    assert lib.hb_cross_validate(0, 2 * HD, big, 2, 100, 257, H, D, 1e-6) == 7
    need = lib.hb_dense_workspace_size(0, 2, 100, H, D)
    assert lib.hb_dense_diffattn(None, fake, 0, big, fake, fake, fake, fake, 32, None, None, 0x8000000, 2, 100, H, D,
                                 1e-6, 0x9000000, need) == 7
    assert lib.hb_band_diffattn(None, fake, 0, big, fake, fake, fake, fake, 32, 16, None, 0x8000000, 1, 100, H, D,
                                None, 0) == 7
    assert lib.hb_dense_attend_qq(None, fake, 0, big, fake, fake, fake, fake, 32, None, 0x8000000, 2, 100, H, D, 1e-6,
                                  0x9000000, need) == 7
    assert lib.hb_proj(None, fake, 0, big, 0x4000000, 128, 0x8000000, 256, 10, 128, 256) == 7           # x
    assert lib.hb_proj(None, fake, 0, 128, 0x4000000, 128, 0x8000000, big, 10, 128, 256) == 7           # out
    assert lib.hb_dit_qkv_proj(None, fake, 0, big, 0x4000000, 256, 256, fake, fake, fake, 32, None, 0x8000000, 2, 100,
                               H, D, 1e-6, 0x9000000, need) == 7
    N, C = 20, 64
    a, b, c = 0x1000000, 0x2000000, 0x3000000
    assert lib.hb_dyt(None, a, 0, big, c, b, C, N, C) == 7
    assert lib.hb_dyt(None, a, 0, C, c, b, big, N, C) == 7
    assert lib.hb_glu(None, a, 0, big, None, 0, b, C, N, C) == 7
    assert lib.hb_residual_dyt(None, a, 0, C, b, big, None, None, c, None, C, N, C) == 7
    assert lib.hb_rms_modulate(None, a, 0, big, c, 1e-5, None, None, C, N, b, C, N, C) == 7
    assert lib.hb_rms_modulate(None, a, 0, C, c, 1e-5, c + 0x10000, c + 0x20000, big, 10, b, C, N, C) == 7  # scale rows
    assert lib.hb_gated_residual(None, a, 0, C, b, C, None, c, big, None, 0, 10, c + 0x80000, C, N, C) == 7  # gate rows
    assert lib.hb_residual_rms(None, a, 0, C, b, C, None, None, C, None, 0, c, 1e-5, None, None, C, N,
                               c + 0x80000, c + 0x90000, big, N, C) == 7


@cpu_only_launch
def test_row_outputs_that_overlap_the_vectors_they_read_are_refused(lib):
    """The row-wise entry points also refuse an output that shares a byte with the per-batch adaLN rows (scale,
    shift, gate), the per-channel vectors (bias, local, the fp32 norm weight) or the DyT parameters the same call
    reads: workgroups read those while others write their rows (HB_ERR_STRIDE; fake, never dereferenced addresses)."""
    N, C, L = 20, 64, 10                      # bf16 rows of 128 bytes, two batches of 10 rows
    a, b, out = 0x1000000, 0x2000000, 0x3000000
    vec = 0x5000000                           # a vector region far from everything
    ob = ((N - 1) * C + C) * 2                # bytes of the output rows
    rms = lambda w, scale, shift, o=out: lib.hb_rms_modulate(None, a, 0, C, w, 1e-5, scale, shift, 3 * C, L, o, C,  # noqa: E731
                                                             N, C)
    assert rms(vec, vec + 0x1000, vec + 0x2000) in (0, 9)                      # disjoint: reaches the launch
    assert rms(vec, vec + 0x1000, vec + 0x2000, o=vec + 0x1000 - 128) == 7     # out's last row over scale
    assert rms(vec, vec + 0x1000, vec + 0x2000, o=vec + 0x2000 + 256) == 7     # out inside shift's second batch row
    assert rms(out + 64, None, None) == 7                                      # fp32 weight inside out's first row
    assert "overlaps" in lib.hb_last_error().decode()
    res = lambda xb, gate, local, o=out: lib.hb_gated_residual(None, a, 0, C, b, C, xb, gate, 2 * C, local, 0, L,  # noqa: E731
                                                               o, C, N, C)
    assert res(out + ob - 16, None, None) == 7                                 # x_bias in out's last row
    assert res(None, out + 128 * 3, None) == 7                                 # gate rows inside out
    assert res(None, None, out) == 7                                           # local at out's start
    rr = lambda w, gate, scale, shift, oh, oy: lib.hb_residual_rms(  # noqa: E731
        None, a, 0, C, b, C, None, gate, 2 * C, None, 0, w, 1e-5, scale, shift, 2 * C, L, oh, oy, C, N, C)
    assert rr(vec, None, vec + 0x1000, vec + 0x2000, out, out + 0x10000) in (0, 9)  # disjoint: reaches the launch
    assert rr(vec, None, vec + 0x1000, out + 0x10000 + 512, out, out + 0x10000) == 7  # shift inside out_y
    assert rr(out + 256, None, None, None, out, out + 0x10000) == 7            # weight inside out_h
    assert rr(vec, out + ob - 64, None, None, out, out + 0x10000) == 7         # gate over out_h's end
    dyt_p = lambda o: lib.hb_dyt(None, a, 0, C, vec, o, C, N, C)  # noqa: E731
    assert dyt_p(vec - 1024) == 7 and dyt_p(vec + 256) == 7                    # out over the DyT parameters
    glu = lambda bias: lib.hb_glu(None, a, 0, 2 * C, bias, 0, out, C, N, C)  # noqa: E731
    assert glu(out + 512) == 7                                                 # bias inside out
    rd = lambda bias, dyt, oy: lib.hb_residual_dyt(None, a, 0, C, b, C, bias, dyt, out, oy, C, N, C)  # noqa: E731
    assert rd(out + 1024, None, None) == 7                                     # bias inside out_h
    assert rd(None, vec, vec - 256) == 7                                       # out_y over the DyT parameters
    assert rd(vec, vec + 0x1000, out + 0x10000) in (0, 9)                      # disjoint: reaches the launch
