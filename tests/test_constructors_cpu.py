"""The reference-shaped constructors (engine/kernels/gemm.py:251, 301, 333):
``SkinnyMatmul / SkinnyGateUp(M, N, K, device, block_n, block_k, split_k,
num_warps, num_stages, persist=0)`` and ``Gemv(..., gateup=False)`` build on
this library, translating the Triton tile arguments into a configuration it
instantiates.  Host logic only: the objects are built on the CPU device and
never called."""

from __future__ import annotations

import pytest
import torch

from kernels import _lib
from kernels import gemm as G

# The reference's own lists (engine/kernels/gemm.py:284-288, 364-375).
REF_CONFIGS = [
    dict(block_n=64, block_k=128, split_k=1, num_warps=4, num_stages=3),
    dict(block_n=32, block_k=128, split_k=1, num_warps=4, num_stages=3),
    dict(block_n=64, block_k=64, split_k=4, num_warps=4, num_stages=4),
    dict(block_n=32, block_k=128, split_k=4, num_warps=4, num_stages=3),
    dict(block_n=64, block_k=128, split_k=8, num_warps=4, num_stages=3),
    dict(block_n=32, block_k=64, split_k=8, num_warps=4, num_stages=4),
    dict(block_n=64, block_k=128, split_k=1, num_warps=4, num_stages=3, persist=1),
    dict(block_n=32, block_k=128, split_k=2, num_warps=4, num_stages=3, persist=2),
    dict(block_n=64, block_k=128, split_k=4, num_warps=4, num_stages=4, persist=2),
    dict(block_n=32, block_k=128, split_k=4, num_warps=4, num_stages=3, persist=2),
]
REF_GEMV_CONFIGS = [
    dict(block_n=32, block_k=256, split_k=1, num_warps=4, num_stages=3),
    dict(block_n=32, block_k=256, split_k=4, num_warps=4, num_stages=3),
    dict(block_n=16, block_k=256, split_k=8, num_warps=2, num_stages=3),
]
SHAPES = [(6144, 2560), (2560, 4096), (2560, 9728), (151936, 2560)]


@pytest.mark.parametrize("M", [1, 4, 8, 16, 32])
def test_every_reference_config_builds(M):
    for N, K in SHAPES:
        for cfg in REF_CONFIGS:
            mm = G.SkinnyMatmul(M, N, K, "cpu", **cfg)
            got = mm.resolved_config
            assert got["splits"] == min(cfg["split_k"], 32, -(-K // 512)) or got["kernel"] != _lib.KERNEL_VALU
            if cfg.get("persist"):
                assert got["kernel"] == _lib.KERNEL_STREAM and got["splits"] >= cfg["split_k"]
            elif M <= 8:
                assert got["kernel"] == _lib.KERNEL_VALU and got["waves"] == cfg["num_warps"]
            else:
                assert got["kernel"] == _lib.KERNEL_MFMA_LDS
                assert got["n_tiles"] == min(4, cfg["block_n"] // 16)
        for cfg in REF_CONFIGS[:6]:
            gu = G.SkinnyGateUp(M, 9728, 2560, "cpu", **cfg)
            assert gu.resolved_config["n_tiles"] % 2 == 0 and gu.N == 19456


def test_reference_gemv_configs_build():
    for cfg in REF_GEMV_CONFIGS:
        for gateup in (False, True):
            g = G.Gemv(1, 9728 if gateup else 6144, 2560, "cpu", gateup=gateup, **cfg)
            c = g.resolved_config
            assert c["kernel"] == _lib.KERNEL_VALU and c["splits"] == min(cfg["split_k"], 5)
            assert c["waves"] == cfg["num_warps"]
            assert g.epilogue == (_lib.EPILOGUE_SILU_MUL if gateup else _lib.EPILOGUE_NONE)


def test_positional_reference_call():
    mm = G.SkinnyMatmul(32, 2560, 9728, "cpu", 64, 128, 4, 4, 3)
    c = mm.resolved_config
    assert c["kernel"] == _lib.KERNEL_MFMA_LDS and c["n_tiles"] == 4 and c["splits"] == 4
    persistent = G.SkinnyMatmul(32, 151936, 2560, "cpu", 64, 128, 1, 4, 3, 1)
    assert persistent.resolved_config["kernel"] == _lib.KERNEL_STREAM


def test_argument_errors_are_value_errors():
    with pytest.raises(ValueError, match="missing"):
        G.SkinnyMatmul(8, 6144, 2560, "cpu", block_n=64)
    with pytest.raises(ValueError, match="either"):
        G.SkinnyMatmul(8, 6144, 2560, "cpu", config={"kernel": 2}, block_n=64, block_k=128, split_k=1,
                       num_warps=4, num_stages=3)
    with pytest.raises(ValueError, match="positive"):
        G.SkinnyMatmul(8, 6144, 2560, "cpu", 0, 128, 1, 4, 3)
    with pytest.raises(ValueError, match="at most 4"):
        G.Gemv(8, 6144, 2560, "cpu", **REF_GEMV_CONFIGS[0])
    # A configuration this build cannot run fails at construction, not later.
    with pytest.raises(ValueError, match="krk error"):
        G.SkinnyMatmul(64, 6144, 2560, "cpu", config={"kernel": _lib.KERNEL_VALU})


def test_default_and_config_forms_unchanged():
    plan = G.SkinnyMatmul(8, 6144, 2560, "cpu")
    assert plan.config is None and plan.resolved_config == G.plan(8, 6144, 2560)
    forced = G.SkinnyMatmul(8, 6144, 2560, "cpu", config={"kernel": _lib.KERNEL_MFMA_LDS})
    assert forced.resolved_config["kernel"] == _lib.KERNEL_MFMA_LDS
    assert isinstance(plan.workspace, (torch.Tensor, type(None)))


def test_stream_split_needs_a_k_stage_per_split():
    """A stream-kernel split with no K stage of its own would never take part
    in its blocks' fix-up (found by validating candidates on two weights):
    such configurations are rejected, and every candidate the tuner is given
    has at least one stage per split."""
    from kernels import tune

    with pytest.raises(ValueError, match="exceeds the 5 K stages"):
        G.resolve(8, 6144, 2560, 0, {"kernel": _lib.KERNEL_STREAM, "splits": 6})
    assert G.resolve(8, 6144, 2560, 0, {"kernel": _lib.KERNEL_STREAM, "splits": 5})["splits"] == 5
    for M, N, K, epi in ((8, 6144, 2560, 0), (32, 19456, 2560, 1), (64, 2560, 4096, 0), (4, 768, 2560, 0)):
        for c in tune.candidates(M, N, K, epi):
            if c["kernel"] == _lib.KERNEL_STREAM:
                assert c["splits"] <= -(-K // 512), (M, N, K, c)
