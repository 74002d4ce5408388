"""MI355X skinny decode GEMM kernels (import surface mirrors the reference's
engine/kernels/__init__.py:1-8 for the projection GEMM)."""

from .gemm import (Gemv, SkinnyGateUp, SkinnyMatmul, SkinnySelect, add_rms_norm, gemm_into, normed_fused, pick_gateup, pick_matmul,
                   pick_normed, plan, select_fused, select_plan, tune_projection)

__all__ = ["Gemv", "SkinnyGateUp", "SkinnyMatmul", "SkinnySelect", "add_rms_norm", "gemm_into", "normed_fused", "pick_gateup",
           "pick_matmul", "pick_normed", "plan", "select_fused", "select_plan", "tune_projection"]
