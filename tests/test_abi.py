"""The C-ABI library without a GPU: it loads, exports every symbol the header
declares, and rejects bad arguments with the documented error codes before
touching the device (no call here reaches a kernel launch)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from kernels import _lib
from kernels._lib import GemmConfig

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "krk_gemm.h"

NONE, SILU = _lib.EPILOGUE_NONE, _lib.EPILOGUE_SILU_MUL
# Fake, well-aligned device addresses far apart: validation never dereferences them.
X, W, Y, WS = 0x10000000, 0x20000000, 0x30000000, 0x40000000


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(krk_\w+)\s*\(", text)))


def test_header_declares_expected_surface():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} is declared in krk_gemm.h but not exported"


def test_abi_version_and_config_layout(lib):
    """The library reports the header's KRK_ABI_VERSION and its
    krk_gemm_config size, and the binding checks both when it loads: a
    binding of another layout would read past, or short of, a config array."""
    version = int(re.search(r"#define KRK_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.krk_abi_version() == version == _lib.ABI_VERSION
    fields = re.search(r"typedef struct krk_gemm_config \{(.*?)\} krk_gemm_config;", HEADER.read_text(), re.S).group(1)
    ints = re.findall(r"^\s*int\s+(\w+);", fields, re.M)
    assert ints == [name for name, _ in GemmConfig._fields_]
    assert lib.krk_gemm_config_size() == ctypes.sizeof(GemmConfig) == 4 * len(ints)


def test_binding_refuses_another_abi(monkeypatch):
    """_lib.load() raises ImportError when the library's ABI version differs
    from the binding's (here: the binding pretends to expect version 2)."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "ABI_VERSION", 2)
    with pytest.raises(ImportError, match=r"ABI version \d+ with a 40-byte"):
        _lib.load()


def call(lib, x=X, ldx=2560, w=W, ldw=2560, y=Y, ldy=None, M=1, N=6144, K=2560, epi=NONE, ws=0, wsb=0):
    if ldy is None:
        ldy = N // 2 if epi == SILU else N
    return lib.krk_gemm_bf16(x, ldx, w, ldw, y, ldy, M, N, K, epi, ws, wsb, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(M=0), _lib.KRK_ERR_INVALID, "M >= 1"),
    (dict(N=0), _lib.KRK_ERR_INVALID, "N >= 1"),
    (dict(K=4, ldx=8, ldw=8), _lib.KRK_ERR_INVALID, "K >= 8"),
    (dict(K=2564, ldx=2568, ldw=2568), _lib.KRK_ERR_INVALID, "multiple of 8"),
    (dict(epi=7), _lib.KRK_ERR_INVALID, "epilogue"),
    (dict(epi=SILU, N=19455, ldy=9727), _lib.KRK_ERR_INVALID, "even N"),
    (dict(x=0), _lib.KRK_ERR_INVALID, "null operand"),
    (dict(y=0), _lib.KRK_ERR_INVALID, "null operand"),
    (dict(ldx=2552), _lib.KRK_ERR_INVALID, "ldx"),
    (dict(ldy=100), _lib.KRK_ERR_INVALID, "ldy"),
    (dict(ldx=2561), _lib.KRK_ERR_ALIGN, "multiples of 8"),
    (dict(x=X + 8), _lib.KRK_ERR_ALIGN, "16-byte aligned"),
    (dict(w=W + 2), _lib.KRK_ERR_ALIGN, "16-byte aligned"),
    (dict(y=Y + 1), _lib.KRK_ERR_ALIGN, "2-byte aligned"),
    (dict(y=X + 1024), _lib.KRK_ERR_ALIAS, "may not share"),
    (dict(y=W + 4096), _lib.KRK_ERR_ALIAS, "may not share"),
])
def test_argument_errors(lib, kw, code, msg):
    assert call(lib, **kw) == code
    assert msg in _lib.last_error()


def _split_shape(lib):
    """A shape whose plan splits K (down_proj at M = 24) and its workspace size."""
    M, N, K = 24, 2560, 9728
    cfg = GemmConfig()
    assert lib.krk_gemm_plan(M, N, K, NONE, ctypes.byref(cfg)) == 0 and cfg.splits > 1
    need = lib.krk_gemm_workspace_bytes(M, N, K, NONE)
    assert need > 0
    return M, N, K, need


def _channels_per_block(c, epi):
    if c["kernel"] == _lib.KERNEL_STREAM:
        return 8 if epi == SILU else 16
    if c["kernel"] == _lib.KERNEL_VALU:
        return c["waves"] * (c["n_tiles"] // 2 if epi == SILU else c["n_tiles"])
    if c["kernel"] in (_lib.KERNEL_MFMA_LDS, _lib.KERNEL_SLICE) and c["channels"]:
        return c["channels"]
    return 16 * (c["n_tiles"] // 2 if epi == SILU else c["n_tiles"])


def test_workspace_errors(lib):
    M, N, K, need = _split_shape(lib)
    kw = dict(M=M, N=N, K=K, ldx=K, ldw=K)
    assert call(lib, **kw) == _lib.KRK_ERR_WORKSPACE and "needs a" in _lib.last_error()
    assert call(lib, ws=WS, wsb=need - 1, **kw) == _lib.KRK_ERR_WORKSPACE
    assert call(lib, ws=WS + 4, wsb=need, **kw) == _lib.KRK_ERR_ALIGN
    assert call(lib, ws=Y, wsb=need, **kw) == _lib.KRK_ERR_ALIAS


def test_workspace_size_formula(lib):
    for M, N, K, epi in [(1, 2560, 4096, NONE), (4, 2560, 9728, NONE), (64, 2560, 9728, NONE),
                         (1, 6144, 2560, NONE), (8, 19456, 2560, SILU), (200, 2560, 9728, NONE),
                         (40, 3000, 5000, SILU), (64, 100000, 3000, NONE)]:
        cfg = GemmConfig()
        assert lib.krk_gemm_plan(M, N, K, epi, ctypes.byref(cfg)) == 0
        got = lib.krk_gemm_workspace_bytes(M, N, K, epi)
        if cfg.splits == 1:
            assert got == 0
            continue
        nout = N // 2 if epi == SILU else N
        nblocks = -(-nout // _channels_per_block(cfg.as_dict(), epi))
        ctr = -(-nblocks * 4 // 256) * 256
        assert got == ctr + cfg.splits * min(M, 64) * N * 4


def test_workspace_bytes_invalid_shape_is_zero(lib):
    assert lib.krk_gemm_workspace_bytes(0, 10, 16, NONE) == 0
    assert lib.krk_gemm_workspace_bytes(1, 10, 12, NONE) == 0
    assert lib.krk_gemm_workspace_bytes(1, 11, 16, SILU) == 0


QWEN = {"qkv": (6144, 2560, NONE), "o": (2560, 4096, NONE), "gate_up": (19456, 2560, SILU),
        "down": (2560, 9728, NONE), "lm_head": (151936, 2560, NONE)}


@pytest.mark.parametrize("shape", sorted(QWEN) + ["other_silu", "other_wide"])
@pytest.mark.parametrize("M", [1, 4, 8, 16, 17, 32, 33, 48, 64, 100])
def test_plan_covers_rows_and_fills_the_chip(lib, shape, M):
    """Every plan covers the rows, and streams from enough CUs: >= 150
    workgroups (measured: 160 one-per-CU workgroups stream a narrow shape at
    ~95% of the 256-workgroup rate), or the persistent stream kernel."""
    N, K, epi = QWEN.get(shape) or {"other_silu": (3000, 5000, SILU), "other_wide": (100000, 3000, NONE)}[shape]
    cfg = GemmConfig()
    assert lib.krk_gemm_plan(M, N, K, epi, ctypes.byref(cfg)) == 0
    c = cfg.as_dict()
    assert c["kernel"] in (_lib.KERNEL_MFMA, _lib.KERNEL_MFMA_LDS, _lib.KERNEL_STREAM, _lib.KERNEL_VALU,
                           _lib.KERNEL_SLICE)
    if c["kernel"] == _lib.KERNEL_SLICE:
        assert M <= 32 and epi == NONE and 1 <= c["channels"] <= 32
    if c["kernel"] == _lib.KERNEL_VALU:
        assert M <= 8 and c["m_tiles"] in (1, 2, 4, 8) and c["m_tiles"] >= M
    else:
        assert 16 * c["m_tiles"] >= min(M, 64) and c["m_tiles"] <= 4
    assert c["splits"] >= 1 and c["waves"] >= 1
    if c["kernel"] != _lib.KERNEL_STREAM:
        nout = N // 2 if epi == SILU else N
        blocks = -(-nout // _channels_per_block(c, epi)) * c["splits"]
        assert blocks >= 150, f"{shape} M={M}: {blocks} workgroups ({c})"


def test_x_preload_resolution(lib):
    """x_preload resolves to the plan's choice for MFMA_LDS (2 for qkv at
    M = 25-32, 1 at 33-64 and where x cannot be held), to 0 for the other kernels (the wave-sliced
    plans of qkv at M = 5-24, o at M = 5-32 and down at M = 2-24 among them), and a caller's 1 or 2
    is kept where it is valid."""
    def resolve(M, N, K, **kw):
        out = GemmConfig()
        assert lib.krk_gemm_resolve(M, N, K, NONE, ctypes.byref(GemmConfig.from_dict(kw)), ctypes.byref(out)) == 0
        return out.as_dict()
    assert resolve(12, 6144, 2560)["x_preload"] == 0  # SLICE
    assert resolve(28, 6144, 2560)["x_preload"] == 2
    assert resolve(20, 6144, 2560)["x_preload"] == 0  # SLICE
    assert resolve(32, 6144, 2560)["x_preload"] == 2
    assert resolve(33, 6144, 2560)["x_preload"] == 1
    assert resolve(12, 6144, 2560, kernel=3, k_chunk=256)["x_preload"] == 1  # the plan's 2 does not apply
    assert resolve(12, 6144, 2560, kernel=3, x_preload=1)["x_preload"] == 1
    assert resolve(24, 6144, 2560, kernel=3, n_tiles=1, k_chunk=512, x_preload=2)["x_preload"] == 2
    assert resolve(20, 2560, 4096)["x_preload"] == 0  # o: SLICE
    assert resolve(20, 2560, 4096, kernel=3, n_tiles=1, k_chunk=512, x_preload=2)["x_preload"] == 2  # 8 stages
    assert resolve(40, 2560, 4096, kernel=3)["x_preload"] == 1  # three x tiles: staged with every stage
    # down: 19 stages, one x tile and one weight tile
    assert resolve(14, 2560, 9728, kernel=3, n_tiles=1, k_chunk=512, x_preload=2)["x_preload"] == 2
    for nt, ok in ((1, True), (2, False)):
        want = GemmConfig.from_dict(dict(kernel=3, n_tiles=nt, k_chunk=512, splits=1, x_preload=2))
        rc = lib.krk_gemm_resolve(12, 2560, 9728, NONE, ctypes.byref(want), ctypes.byref(GemmConfig()))
        assert (rc == 0) == ok, (nt, _lib.last_error())
    for K, ok in ((4096, True), (4104, False)):  # at most 8 stages of 512
        want = GemmConfig.from_dict(dict(kernel=3, n_tiles=1, k_chunk=512, x_preload=2))
        rc = lib.krk_gemm_resolve(20, 2560, K, NONE, ctypes.byref(want), ctypes.byref(GemmConfig()))
        assert (rc == 0) == ok, (K, _lib.last_error())
    for kernel in (1, 2, 5, 6):
        assert resolve(8, 6144, 2560, kernel=kernel, x_preload=2)["x_preload"] == 0


@pytest.mark.parametrize("cfg,code,msg", [
    (dict(kernel=9), _lib.KRK_ERR_UNSUPPORTED, "unknown kernel"),
    (dict(kernel=1, m_tiles=1), _lib.KRK_ERR_INVALID, "cannot cover"),
    (dict(kernel=1, n_tiles=3), _lib.KRK_ERR_UNSUPPORTED, "n_tiles"),
    (dict(kernel=1, unroll=3), _lib.KRK_ERR_UNSUPPORTED, "unroll"),
    (dict(kernel=1, waves=8), _lib.KRK_ERR_UNSUPPORTED, "waves"),
    (dict(kernel=1, splits=33), _lib.KRK_ERR_UNSUPPORTED, "splits"),
    (dict(kernel=2), _lib.KRK_ERR_UNSUPPORTED, "VALU"),
    (dict(kernel=3, unroll=4), _lib.KRK_ERR_UNSUPPORTED, "unroll"),
    (dict(kernel=3, m_tiles=4, n_tiles=4, unroll=3), _lib.KRK_ERR_UNSUPPORTED, "unroll"),
    (dict(kernel=3, waves=4), _lib.KRK_ERR_UNSUPPORTED, "waves"),
    (dict(kernel=3, m_tiles=2, n_tiles=4, k_chunk=512), _lib.KRK_ERR_UNSUPPORTED, "k_chunk"),
    (dict(kernel=3, k_chunk=384), _lib.KRK_ERR_UNSUPPORTED, "k_chunk"),
    (dict(kernel=3, x_preload=3), _lib.KRK_ERR_UNSUPPORTED, "x_preload"),
    (dict(kernel=3, k_chunk=256, x_preload=2), _lib.KRK_ERR_UNSUPPORTED, "x_preload"),
    (dict(kernel=3, k_chunk=512, n_tiles=2, splits=2, x_preload=2), _lib.KRK_ERR_UNSUPPORTED, "x_preload"),
    (dict(kernel=3, m_tiles=3, n_tiles=1, k_chunk=512, x_preload=2), _lib.KRK_ERR_UNSUPPORTED, "x_preload"),
    (dict(kernel=6, k_chunk=256), _lib.KRK_ERR_UNSUPPORTED, "k_chunk"),
    (dict(kernel=6, channels=33), _lib.KRK_ERR_UNSUPPORTED, "channels"),
    (dict(kernel=6, unroll=4), _lib.KRK_ERR_UNSUPPORTED, "not instantiated"),
    (dict(kernel=6, k_chunk=128), _lib.KRK_ERR_UNSUPPORTED, "not instantiated"),
    (dict(kernel=6, splits=41), _lib.KRK_ERR_UNSUPPORTED, "splits"),
])
def test_config_errors(lib, cfg, code, msg):
    c = GemmConfig.from_dict(cfg)
    rc = lib.krk_gemm_bf16_config(X, 2560, W, 2560, Y, 6144, 20, 6144, 2560, NONE, ctypes.byref(c), 0, 0, None)
    assert rc == code
    assert msg in _lib.last_error()


@pytest.mark.parametrize("cfg,msg", [
    (dict(kernel=2, n_tiles=3), "n_tiles"),
    (dict(kernel=2, unroll=6), "unroll"),
    (dict(kernel=2, n_tiles=4, unroll=19), "unroll"),
    (dict(kernel=2, waves=16), "waves"),
    (dict(kernel=2, waves=9), "waves"),
    (dict(kernel=2, splits=6), "splits"),
])
def test_valu_config_errors(lib, cfg, msg):
    """K = 2560 is five 512-element blocks: at most 5 splits."""
    c = GemmConfig.from_dict(cfg)
    rc = lib.krk_gemm_bf16_config(X, 2560, W, 2560, Y, 6144, 4, 6144, 2560, NONE, ctypes.byref(c), 0, 0, None)
    assert rc == _lib.KRK_ERR_UNSUPPORTED
    assert msg in _lib.last_error()


def test_valu_x_slice_must_fit_lds(lib):
    """M = 8 keeps 8 x rows of a split's K range in LDS: K = 16384 unsplit is
    256 KB, over gfx950's 160 KB, and is refused; two splits fit."""
    c = GemmConfig.from_dict(dict(kernel=2, splits=1))
    assert lib.krk_gemm_config_workspace_bytes(8, 512, 16384, NONE, ctypes.byref(c)) == 0
    rc = lib.krk_gemm_bf16_config(X, 16384, W, 16384, Y, 512, 8, 512, 16384, NONE, ctypes.byref(c), 0, 0, None)
    assert rc == _lib.KRK_ERR_UNSUPPORTED and "LDS" in _lib.last_error()
    c = GemmConfig.from_dict(dict(kernel=2, splits=2))
    assert lib.krk_gemm_config_workspace_bytes(8, 512, 16384, NONE, ctypes.byref(c)) > 0


def test_silu_needs_even_tiles(lib):
    c = GemmConfig.from_dict(dict(kernel=1, n_tiles=1))
    rc = lib.krk_gemm_bf16_config(X, 2560, W, 2560, Y, 9728, 1, 19456, 2560, SILU, ctypes.byref(c), 0, 0, None)
    assert rc == _lib.KRK_ERR_UNSUPPORTED and "even n_tiles" in _lib.last_error()


def test_last_error_is_cleared_by_a_plan_call(lib):
    call(lib, M=0)
    assert _lib.last_error()
    cfg = GemmConfig()
    assert lib.krk_gemm_plan(1, 6144, 2560, NONE, ctypes.byref(cfg)) == 0
    assert _lib.last_error() == ""


def test_python_wrapper_rejects_cpu_and_bad_tensors():
    import torch

    from kernels.gemm import gemm_into

    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    w = torch.zeros(32, 64, dtype=torch.bfloat16)
    y = torch.zeros(2, 32, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        gemm_into(x, w, y)
    with pytest.raises(ValueError, match="bfloat16"):
        gemm_into(x.float(), w, y)
    with pytest.raises(ValueError, match="contiguous"):
        gemm_into(x.t().contiguous().t(), w, y)
    with pytest.raises(ValueError, match="rows"):
        gemm_into(x, w, y[:1])


def test_error_mapping():
    with pytest.raises(ValueError):
        _lib.check(_lib.KRK_ERR_ALIAS)
    with pytest.raises(_lib.KrkError):
        _lib.check(_lib.KRK_ERR_HIP)
    _lib.check(_lib.KRK_OK)


# ------------------------------------------------------------------ normed projections

D, G, XO = 0x50000000, 0x60000000, 0x70000000


def call_normed(lib, x=X, ldx=2560, d=D, ldd=2560, g=G, eps=1e-6, xo=XO, ldxo=2560, w=W, ldw=2560, y=Y, ldy=None,
                M=1, N=6144, K=2560, epi=NONE, ws=WS, wsb=1 << 30):
    if ldy is None:
        ldy = N // 2 if epi == SILU else N
    return lib.krk_gemm_bf16_normed(x, ldx, d, ldd, g, eps, xo, ldxo, w, ldw, y, ldy, M, N, K, epi, ws, wsb, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(d=0), _lib.KRK_ERR_INVALID, "null norm operand"),
    (dict(xo=0), _lib.KRK_ERR_INVALID, "null norm operand"),
    (dict(ldd=2552), _lib.KRK_ERR_INVALID, "ldd"),
    (dict(ldxo=2561), _lib.KRK_ERR_ALIGN, "multiples of 8"),
    (dict(d=D + 8), _lib.KRK_ERR_ALIGN, "16-byte aligned"),
    (dict(g=G + 2), _lib.KRK_ERR_ALIGN, "16-byte aligned"),
    (dict(eps=-1.0), _lib.KRK_ERR_INVALID, "eps"),
    (dict(eps=float("nan")), _lib.KRK_ERR_INVALID, "eps"),
    (dict(xo=X), _lib.KRK_ERR_ALIAS, "xout may not share"),
    (dict(xo=D + 1024), _lib.KRK_ERR_ALIAS, "xout may not share"),
    (dict(y=D), _lib.KRK_ERR_ALIAS, "may not share"),
    (dict(K=16392, ldx=16392, ldd=16392, ldxo=16392, ldw=16392), _lib.KRK_ERR_UNSUPPORTED, "K <="),
    (dict(ws=0, M=32), _lib.KRK_ERR_WORKSPACE, "workspace"),
    (dict(ws=XO, M=32), _lib.KRK_ERR_ALIAS, "workspace may not share"),
])
def test_normed_argument_errors(lib, kw, code, msg):
    assert call_normed(lib, **kw) == code
    assert msg in _lib.last_error()


def test_normed_fused_plans(lib):
    """The normed plans fuse the prologue where that measured fastest (qkv
    at M <= 4, gate_up and lm_head at M <= 2, on the VALU kernel) and
    otherwise run the plain plan behind the separate prologue kernel
    (prologue = 1).  A VALU configuration fuses when K is unsplit, the depth
    covers K = 2560 and there is a wave per 512-k block; an LDS-staged one
    when K is unsplit in at most five 512-k stages with one or two x tiles
    and one or two weight tiles; prologue = 1, split K, the stream and the
    register MFMA kernels never fuse."""
    for (N, K, epi), M, fused in [(QWEN["qkv"], 1, 1), (QWEN["qkv"], 4, 1), (QWEN["qkv"], 5, 0),
                                  (QWEN["qkv"], 8, 0), (QWEN["qkv"], 16, 0), (QWEN["qkv"], 17, 0),
                                  (QWEN["gate_up"], 1, 1), (QWEN["gate_up"], 2, 1), (QWEN["gate_up"], 8, 0),
                                  (QWEN["lm_head"], 1, 1), (QWEN["lm_head"], 2, 1), (QWEN["lm_head"], 4, 0),
                                  (QWEN["gate_up"], 32, 0), (QWEN["qkv"], 32, 0), (QWEN["lm_head"], 64, 0)]:
        assert lib.krk_gemm_normed_fused(M, N, K, epi, None) == fused, (N, M)
        cfg = GemmConfig()
        assert lib.krk_gemm_normed_plan(M, N, K, epi, ctypes.byref(cfg)) == 0
        assert cfg.prologue == 1 - fused, (N, M)
        assert lib.krk_gemm_normed_fused(M, N, K, epi, ctypes.byref(cfg)) == fused, (N, M)
    N, K, epi = QWEN["qkv"]
    for kw, fused in [(dict(n_tiles=2, waves=8), 1), (dict(n_tiles=1, waves=4), 0), (dict(n_tiles=1, waves=5), 1),
                      (dict(n_tiles=4, waves=6), 1), (dict(n_tiles=2, waves=8, splits=2), 0),
                      (dict(n_tiles=2, waves=8, prologue=1), 0)]:
        cfg = GemmConfig(kernel=_lib.KERNEL_VALU, unroll=5, **kw)
        assert lib.krk_gemm_normed_fused(4, N, K, epi, ctypes.byref(cfg)) == fused, kw
    for kernel in (_lib.KERNEL_STREAM, _lib.KERNEL_MFMA):
        cfg = GemmConfig(kernel=kernel)
        assert lib.krk_gemm_normed_fused(16, N, K, epi, ctypes.byref(cfg)) == 0
    # The LDS-staged kernel fuses with one or two 16-row x tiles (M <= 32),
    # 512-k stages, K unsplit and one or two weight tiles (with two of each,
    # two stages in flight).
    for M, kw, fused in [(16, dict(n_tiles=2, k_chunk=512), 1), (9, dict(n_tiles=1, k_chunk=512, unroll=3), 1),
                         (17, dict(n_tiles=2, k_chunk=512, unroll=2), 1), (32, dict(n_tiles=1, k_chunk=512, unroll=3), 1),
                         (32, dict(n_tiles=2, k_chunk=512, unroll=3), 0), (33, dict(n_tiles=1, k_chunk=512), 0),
                         (16, dict(n_tiles=2, k_chunk=256), 0),
                         (16, dict(n_tiles=2, k_chunk=512, splits=2), 0), (16, dict(n_tiles=4, k_chunk=256), 0),
                         (16, dict(n_tiles=2, k_chunk=512, prologue=1), 0)]:
        cfg = GemmConfig(kernel=_lib.KERNEL_MFMA_LDS, **kw)
        assert lib.krk_gemm_normed_fused(M, N, K, epi, ctypes.byref(cfg)) == fused, (M, kw)
    cfg = GemmConfig(kernel=_lib.KERNEL_MFMA_LDS, n_tiles=2, k_chunk=512)
    assert lib.krk_gemm_normed_fused(16, N, 4096, epi, ctypes.byref(cfg)) == 0  # 8 stages: more than it holds
    deep = GemmConfig(kernel=_lib.KERNEL_STREAM, splits=1)
    assert lib.krk_gemm_normed_fused(8, 2560, 9728, NONE, ctypes.byref(deep)) < 0  # 19 stages: not instantiated
    bad = GemmConfig(kernel=_lib.KERNEL_STREAM, prologue=2)
    assert lib.krk_gemm_normed_fused(8, 6144, 2560, NONE, ctypes.byref(bad)) == _lib.KRK_ERR_UNSUPPORTED
    assert lib.krk_gemm_normed_fused(0, 6144, 2560, NONE, None) == _lib.KRK_ERR_INVALID
    assert lib.krk_gemm_normed_plan(1, 6144, 2560, NONE, None) == _lib.KRK_ERR_INVALID


def _normed_rows_bytes(lib, M, N, K, epi, cfg=None):
    """Bytes of the normalised rows a prologue kernel writes: M x K bf16, or,
    in front of a stream-kernel launch (M <= 64), the kernel's fragment order
    over 16 * m_tiles rows and whole 512-k stages."""
    c = GemmConfig()
    assert lib.krk_gemm_resolve(M, N, K, epi, ctypes.byref(cfg) if cfg is not None else None, ctypes.byref(c)) == 0
    if c.kernel == _lib.KERNEL_STREAM and M <= 64:
        return 16 * c.m_tiles * -(-K // 512) * 512 * 2
    return M * K * 2


def test_normed_workspace_layouts(lib):
    """Prologue-kernel plans add the normalised rows after the split-K area
    (in the stream kernel's fragment order in front of that kernel); fused
    plans add nothing."""
    for (N, K, epi), M in [(QWEN["qkv"], 32), (QWEN["qkv"], 100), (QWEN["gate_up"], 64), (QWEN["lm_head"], 64),
                           (QWEN["gate_up"], 20), (QWEN["lm_head"], 100)]:
        assert lib.krk_gemm_normed_fused(M, N, K, epi, None) == 0
        plain = lib.krk_gemm_workspace_bytes(M, N, K, epi)
        normed = lib.krk_gemm_normed_workspace_bytes(M, N, K, epi, None)
        assert normed == -(-plain // 256) * 256 + _normed_rows_bytes(lib, M, N, K, epi), (N, M)
    assert _normed_rows_bytes(lib, 20, *QWEN["gate_up"]) == 32 * 2560 * 2  # two 16-row tiles
    assert _normed_rows_bytes(lib, 100, *QWEN["lm_head"]) == 100 * 2560 * 2  # two launches: rows
    sep = GemmConfig(kernel=_lib.KERNEL_STREAM, prologue=1)
    for (N, K, epi), M in [(QWEN["gate_up"], 16), (QWEN["lm_head"], 17), ((2 * 96, 1000, SILU), 17)]:
        plain = lib.krk_gemm_config_workspace_bytes(M, N, K, epi, ctypes.byref(sep))
        normed = lib.krk_gemm_normed_workspace_bytes(M, N, K, epi, ctypes.byref(sep))
        assert normed == -(-plain // 256) * 256 + _normed_rows_bytes(lib, M, N, K, epi, sep), (N, M)
    assert _normed_rows_bytes(lib, 17, 192, 1000, SILU, sep) == 32 * 1024 * 2  # ragged K: whole stages
    for (N, K, epi), M in [(QWEN["qkv"], 1), (QWEN["gate_up"], 2), (QWEN["lm_head"], 1)]:
        assert lib.krk_gemm_normed_fused(M, N, K, epi, None) == 1
        cfg = GemmConfig()
        assert lib.krk_gemm_normed_plan(M, N, K, epi, ctypes.byref(cfg)) == 0
        assert lib.krk_gemm_normed_workspace_bytes(M, N, K, epi, None) == \
            lib.krk_gemm_config_workspace_bytes(M, N, K, epi, ctypes.byref(cfg))


@pytest.mark.parametrize("kw,code", [
    (dict(M=0), _lib.KRK_ERR_INVALID),
    (dict(K=12), _lib.KRK_ERR_INVALID),
    (dict(eps=-2.0), _lib.KRK_ERR_INVALID),
    (dict(xo=D), _lib.KRK_ERR_ALIAS),
    (dict(out=X + 64), _lib.KRK_ERR_ALIAS),
    (dict(out=XO), _lib.KRK_ERR_ALIAS),
    (dict(xo=X, ldxo=2568), _lib.KRK_ERR_ALIAS),
    (dict(K=16392, ldx=16392, ldd=16392, ldxo=16392, ldo=16392), _lib.KRK_ERR_UNSUPPORTED),
])
def test_add_rms_norm_argument_errors(lib, kw, code):
    a = dict(x=X, ldx=2560, d=D, ldd=2560, g=G, eps=1e-6, xo=XO, ldxo=2560, out=Y, ldo=2560, M=4, K=2560)
    a.update(kw)
    if "ldx" not in kw and a["K"] > 2560:
        a["ldx"] = a["K"]
    rc = lib.krk_add_rms_norm_bf16(a["x"], a["ldx"], a["d"], a["ldd"], a["g"], a["eps"], a["xo"], a["ldxo"],
                                   a["out"], a["ldo"], a["M"], a["K"], None)
    assert rc == code, _lib.last_error()


# ------------------------------------------------------------------ token selection

# The lm_head weight spans 778 MB: select calls keep everything else far from it.
W_LM, IDX, WS_SEL, Y_SEL = 0x100000000, 0x300000000, 0x400000000, 0x500000000


def call_select(lib, x=X, ldx=2560, w=W_LM, ldw=2560, y=0, ldy=151936, M=1, N=151936, K=2560, k=1, idx=IDX, vals=0,
                ws=WS_SEL, wsb=1 << 30):
    return lib.krk_gemm_bf16_select(x, ldx, w, ldw, y, ldy, M, N, K, k, idx, vals, ws, wsb, None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(k=0), _lib.KRK_ERR_INVALID, "k="),
    (dict(k=9), _lib.KRK_ERR_INVALID, "k="),
    (dict(k=8, N=5, ldy=5), _lib.KRK_ERR_INVALID, "k="),
    (dict(idx=0), _lib.KRK_ERR_INVALID, "null operand"),
    (dict(idx=IDX + 4), _lib.KRK_ERR_ALIGN, "misaligned"),
    (dict(y=Y_SEL, ldy=100), _lib.KRK_ERR_INVALID, "ldy"),
    (dict(idx=X + 64), _lib.KRK_ERR_ALIAS, "may not share"),
    (dict(idx=W_LM + 4096), _lib.KRK_ERR_ALIAS, "may not share"),
    (dict(ws=IDX), _lib.KRK_ERR_ALIAS, "may not overlap"),
    (dict(y=Y_SEL, vals=Y_SEL + 64), _lib.KRK_ERR_ALIAS, "may not overlap"),
    (dict(ws=0), _lib.KRK_ERR_WORKSPACE, "workspace"),
    (dict(wsb=64), _lib.KRK_ERR_WORKSPACE, "workspace"),
    (dict(ws=WS_SEL + 16), _lib.KRK_ERR_ALIGN, "256-byte"),
])
def test_select_argument_errors(lib, kw, code, msg):
    assert call_select(lib, **kw) == code
    assert msg in _lib.last_error()


def _stream_groups(nblocks, cus=256):
    """Workgroups of the persistent stream kernel for nblocks blocks, K unsplit."""
    if nblocks <= cus:
        return nblocks
    best, best_eff = cus, 0.0
    for g in range(cus, cus // 2 - 1, -1):
        eff = nblocks / (-(-nblocks // g) * cus)
        if eff > best_eff + 1e-9:
            best, best_eff = g, eff
    return best


def test_select_plan_and_workspace(lib):
    """The projection plan is the plain table's (a fusing stream plan keeps a
    ring of at most 5 stages); argmax fuses into the VALU
    (M <= 4) and stream (from M = 5, K of 5 stages) plans and into
    LDS-staged MFMA configurations; top-k fuses into stream plans of up to
    16 rows only.  Workspace: the row counters, then the keys of each row
    and projection workgroup (fused: one for argmax, 8 for top-k; the
    stream kernel's workgroups each cover many blocks) or a logits buffer,
    then the per-chunk lists."""
    al = lambda v: -(-v // 256) * 256
    N, K = 151936, 2560
    for M, kernel in [(1, _lib.KERNEL_VALU), (4, _lib.KERNEL_VALU), (5, _lib.KERNEL_STREAM),
                      (16, _lib.KERNEL_STREAM), (17, _lib.KERNEL_STREAM), (64, _lib.KERNEL_STREAM),
                      (100, _lib.KERNEL_STREAM)]:
        Mc = min(M, 64)
        for k in (1, 8):
            cfg, plain = GemmConfig(), GemmConfig()
            assert lib.krk_gemm_select_plan(M, N, K, k, ctypes.byref(cfg)) == 0
            assert lib.krk_gemm_plan(M, N, K, NONE, ctypes.byref(plain)) == 0
            c, p = cfg.as_dict(), plain.as_dict()
            fused = lib.krk_gemm_select_fused(M, N, K, k, None)
            if fused and kernel == _lib.KERNEL_STREAM:
                p["unroll"] = min(p["unroll"], 5)
            assert c == p and c["kernel"] == kernel, (M, k, c)
            assert fused == int(k == 1 or (kernel == _lib.KERNEL_STREAM and Mc <= 16)), (M, k)
            if fused:
                G = -(-N // _channels_per_block(c, NONE))
                if kernel == _lib.KERNEL_STREAM:
                    G = _stream_groups(G) * (1 if k == 1 else 8)
                src = al(Mc * (-(-G // 2) * 2) * 8)  # one key per row and workgroup
                chunks = -(-G // 1024)
            else:
                src = al(Mc * (-(-N // 8) * 8) * 2)  # bf16 logits
                chunks = -(-N // 16384)
            want = 64 * 128 + src + al(Mc * chunks * k * 8)  # row counters 128 B apart
            assert lib.krk_gemm_select_workspace_bytes(M, N, K, k, None) == want, (M, k)
    # An LDS-staged MFMA configuration with 256-k stages fuses argmax.
    lds = GemmConfig.from_dict(dict(kernel=_lib.KERNEL_MFMA_LDS, n_tiles=2, unroll=3, k_chunk=256))
    assert lib.krk_gemm_select_fused(8, N, K, 1, ctypes.byref(lds)) == 1
    assert lib.krk_gemm_select_fused(8, N, K, 8, ctypes.byref(lds)) == 0
    keys = al(8 * (-(-(N // 32) // 2) * 2) * 8) + al(8 * -(-(N // 32) // 1024) * 8)
    assert lib.krk_gemm_select_workspace_bytes(8, N, K, 1, ctypes.byref(lds)) == 64 * 128 + keys
    # Any plain configuration is accepted; the stream kernel fuses argmax only
    # for a K of 5 stages and unsplit.
    stream = GemmConfig.from_dict(dict(kernel=_lib.KERNEL_STREAM))
    assert lib.krk_gemm_select_workspace_bytes(8, N, K, 1, ctypes.byref(stream)) > 0
    assert lib.krk_gemm_select_fused(8, N, K, 1, ctypes.byref(stream)) == 1
    assert lib.krk_gemm_select_fused(8, N, 1536, 1, ctypes.byref(stream)) == 0
    stream2 = GemmConfig.from_dict(dict(kernel=_lib.KERNEL_STREAM, splits=2))
    assert lib.krk_gemm_select_fused(8, N, K, 1, ctypes.byref(stream2)) == 0
    # A split-K projection reserves its partials after the counters.
    split = GemmConfig.from_dict(dict(kernel=_lib.KERNEL_VALU, splits=2))
    c = GemmConfig()
    assert lib.krk_gemm_select_fused(1, N, K, 1, ctypes.byref(split)) == 0
    assert lib.krk_gemm_select_workspace_bytes(1, N, K, 1, ctypes.byref(split)) > \
        lib.krk_gemm_select_workspace_bytes(1, N, K, 1, ctypes.byref(stream))
    assert lib.krk_gemm_select_fused(1, N, K, 9, None) == _lib.KRK_ERR_INVALID
    assert lib.krk_gemm_select_plan(1, N, K, 0, ctypes.byref(c)) == _lib.KRK_ERR_INVALID
    bad = GemmConfig.from_dict(dict(kernel=_lib.KERNEL_MFMA_LDS, k_chunk=384))
    assert lib.krk_gemm_select_workspace_bytes(32, N, K, 1, ctypes.byref(bad)) == 0


# ------------------------------------------------------------------ tuner search space

@pytest.mark.parametrize("M", [1, 4, 8, 9, 32, 64, 100])
def test_candidates_search_space(lib, M):
    """krk_gemm_candidates: the plan first, then distinct configurations the
    library accepts (resolved: no field left at 0), VALU only up to 8 rows;
    a short array receives the first cap entries."""
    for N, K, epi in QWEN.values():
        n = lib.krk_gemm_candidates(M, N, K, epi, None, 0)
        assert n > 8, (M, N, K, n)
        arr = (GemmConfig * n)()
        assert lib.krk_gemm_candidates(M, N, K, epi, arr, n) == n
        cfgs = [c.as_dict() for c in arr]
        plan = GemmConfig()
        assert lib.krk_gemm_plan(M, N, K, epi, ctypes.byref(plan)) == 0
        assert cfgs[0] == plan.as_dict()
        assert len({tuple(sorted(c.items())) for c in cfgs}) == n
        kinds = {c["kernel"] for c in cfgs}
        assert (_lib.KERNEL_VALU in kinds) == (min(M, 64) <= 8)
        assert (_lib.KERNEL_SLICE in kinds) == (min(M, 64) <= 32 and epi == NONE)
        assert {_lib.KERNEL_MFMA_LDS, _lib.KERNEL_STREAM} <= kinds
        for c in cfgs:
            assert c["kernel"] in (_lib.KERNEL_MFMA, _lib.KERNEL_VALU, _lib.KERNEL_MFMA_LDS, _lib.KERNEL_STREAM,
                                   _lib.KERNEL_SLICE)
            assert all(c[f] > 0 for f in ("m_tiles", "n_tiles", "unroll", "waves", "splits")), c
            if c["kernel"] == _lib.KERNEL_MFMA_LDS:
                assert c["k_chunk"] in (256, 512)
            if c["kernel"] == _lib.KERNEL_SLICE:
                assert c["k_chunk"] in (64, 128) and c["unroll"] in (2, 3) and c["waves"] == 8
            if epi == SILU and c["kernel"] != _lib.KERNEL_STREAM:
                assert c["n_tiles"] % 2 == 0, c
            # Each one is accepted again as an explicit configuration.
            cfg = GemmConfig.from_dict(c)
            if c["splits"] > 1:
                assert lib.krk_gemm_config_workspace_bytes(M, N, K, epi, ctypes.byref(cfg)) > 0, c
        short = (GemmConfig * 3)()
        assert lib.krk_gemm_candidates(M, N, K, epi, short, 3) == n
        assert [c.as_dict() for c in short] == cfgs[:3]
    assert lib.krk_gemm_candidates(1, 64, 12, NONE, None, 0) == _lib.KRK_ERR_INVALID
    assert lib.krk_gemm_candidates(1, 64, 64, NONE, None, -1) == _lib.KRK_ERR_INVALID
    assert lib.krk_gemm_candidates(1, 64, 64, NONE, None, 4) == _lib.KRK_ERR_INVALID


def test_package_loads_under_another_name():
    """The engine's own ``kernels`` package takes that name: krk_loader
    imports this one as a separate package, sharing the one HIP library."""
    import krk_loader
    import kernels

    krk = krk_loader.load("krk_alias_for_test")
    assert krk is not kernels and krk.gemm is not kernels.gemm
    assert callable(krk.step.decode_matmuls) and callable(krk.gemm.SkinnyMatmul)
    assert krk._lib.LIB_PATH == kernels._lib.LIB_PATH
    assert krk_loader.load("krk_alias_for_test") is krk
    assert krk.tune.candidates(1, 6144, 2560)[0] == kernels.gemm.plan(1, 6144, 2560)


def test_noalloc_rejects_before_touching_the_device(lib):
    """krk_gemm_bf16_noalloc checks the shape and whether the plan's split-K
    partials fit the static scratch before any device call (fake pointers)."""
    rc = lib.krk_gemm_bf16_noalloc(X, 2560, W, 2560, Y, 6144, 0, 6144, 2560, NONE, None)
    assert rc == _lib.KRK_ERR_INVALID
    # M=8, N=65536, K=32768: the plan splits K 8 ways, 16 MiB of partials
    rc = lib.krk_gemm_bf16_noalloc(X, 32768, W, 32768, Y, 65536, 8, 65536, 32768, NONE, None)
    assert rc == _lib.KRK_ERR_WORKSPACE and "static scratch" in _lib.last_error()
