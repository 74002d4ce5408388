"""MI355X skinny decode GEMM kernels (import surface mirrors the reference's
engine/kernels/__init__.py:1-8 for the projection GEMM)."""

from .gemm import Gemv, SkinnyGateUp, SkinnyMatmul, gemm_into, pick_gateup, pick_matmul, plan

__all__ = ["Gemv", "SkinnyGateUp", "SkinnyMatmul", "gemm_into", "pick_gateup", "pick_matmul", "plan"]
