"""CPU oracle for the Qwen3-4B skinny decode GEMM.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import, call or load anything under
oracle/, and only as the checker (or the timed CPU baseline), never as the
thing measured or shipped.  The product (kernel-rush-kawk_amd/, libkrk_gemm.so)
does not import it.

Contents:
  gemm_ref.py  torch-CPU restatement of the reference's projection path
               (the library routine ``torch.nn.functional.linear`` the
               reference calls as ``a @ w.t()``), its SwiGLU epilogue and
               argmax, plus numpy fp64 brute force and error bounds that pin it.
  gemm_ref.c   plain-C restatement (fp32 sequential accumulation, fp64 exact
               sums, SwiGLU with three roundings, first-index argmax), built by
               oracle/build.py into oracle/_build/liboracle.so.

Pinning status of each function is recorded in gemm_ref.py's docstring.
"""
