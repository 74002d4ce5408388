"""Decode-step integration: the reference engine's projection dict and the
projection calls of one decode step, on libkrk_gemm.so.

* :func:`decode_matmuls` — drop-in for ``decode_matmuls(m, M, log)``
  (engine/model.py:137-178): the "qkv", "gu" and "lm" callables take
  ``(x, y, w_norm, xout, w)`` and fold the residual add and RMSNorm in front
  of the projection, "o" and "d" take ``(a, w)``.  Each is picked (and, with
  ``tune``, tuned) on this GPU by the pickers of :mod:`kernels.gemm`.  With
  ``ENGINE_NORM_FUSED`` set to anything but "1" the norm runs as its own
  kernel in front of a plain projection, as the reference does
  (model.py:161-171).  The reference's ``ENGINE_FORCE_CUBLAS`` switch
  (model.py:152-160) has no counterpart: every call stays on the HIP path.
  ``select_k`` adds "lm_select": the final norm, the lm_head projection and
  the per-row top-k indices (argmax for k = 1) in place of
  ``lm(...).argmax(-1)`` (engine/engine.py:196).
* :class:`GemmStep` — the projection data flow of ``run_layers``
  (engine/model.py:181-214): per layer qkv (normed), o, gate/up (normed),
  down, then the normed lm_head; 4 · layers + 1 calls, 145 for Qwen3-4B.
  Attention, q/k norm, RoPE and the KV cache are not part of this library:
  the o projection reads a caller-filled ``attn_out`` buffer and the qkv
  output is not consumed.  The residual stream uses the reference's two
  buffers (qkv reads ``cur`` and writes ``xa``, gate/up reads ``xa`` and
  writes ``xb``, lm reads ``xb`` and writes ``xa``), and :meth:`capture`
  records the whole step in one graph as the engine's ``capture`` does
  (engine/engine.py:187-207).
* :func:`synthetic_model` — a Model-shaped object (``cfg``, ``layers`` with
  ``in_norm``/``wqkv``/``wo``/``post_norm``/``wgu``/``wd``, ``lm_head``,
  ``final_norm``, ``device``) with seeded random weights, for tests and
  benchmarks (no checkpoints are loaded here).
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from types import SimpleNamespace

import torch

from . import gemm as G


def decode_matmuls(m, M: int, log=None, tune: bool = True, select_k: int | None = None) -> dict:
    """Per-shape projection callables for M-row decode steps (reference
    engine/model.py:137-178).  The gate/up pickers get each layer's down
    weight, so at 64 rows a tuned gate/up configuration is also checked
    through the down projection that consumes it (the reference's N32
    selector, engine/kernels/m64_gateup_n32_selection.py:73-105)."""
    cfg = m.cfg
    layer = m.layers[0]
    L = m.layers
    dev = m.device
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    rnd = lambda *shape: torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)
    x, y = rnd(M, cfg.hidden), rnd(M, cfg.hidden)
    a, act = rnd(M, cfg.heads * cfg.head_dim), rnd(M, cfg.intermediate)
    eps = cfg.eps
    if os.environ.get("ENGINE_NORM_FUSED", "1") != "1":
        qkv = G.pick_matmul(x, layer.wqkv, log, ws=[l.wqkv for l in L], tune=tune)
        gu = G.pick_gateup(x, layer.wgu, log, ws=[l.wgu for l in L], tune=tune, down=[l.wd for l in L])
        lm = G.pick_matmul(x, m.lm_head, log, tune=tune)
        mm = {
            "qkv": lambda x, y, wn, xout, w: qkv(G.add_rms_norm(x, y, wn, eps, xout), w),
            "o": G.pick_matmul(a, layer.wo, log, ws=[l.wo for l in L], tune=tune),
            "gu": lambda x, y, wn, xout, w: gu(G.add_rms_norm(x, y, wn, eps, xout), w),
            "d": G.pick_matmul(act, layer.wd, log, ws=[l.wd for l in L], tune=tune),
            "lm": lambda x, y, wn, xout, w: lm(G.add_rms_norm(x, y, wn, eps, xout), w),
        }
    else:
        mm = {
            "qkv": G.pick_normed("matmul", x, y, layer.in_norm, layer.wqkv, eps, log, ws=[l.wqkv for l in L], tune=tune),
            "o": G.pick_matmul(a, layer.wo, log, ws=[l.wo for l in L], tune=tune),
            "gu": G.pick_normed("gateup", x, y, layer.post_norm, layer.wgu, eps, log, ws=[l.wgu for l in L], tune=tune,
                                down=[l.wd for l in L]),
            "d": G.pick_matmul(act, layer.wd, log, ws=[l.wd for l in L], tune=tune),
            "lm": G.pick_normed("matmul", x, y, m.final_norm, m.lm_head, eps, log, tune=tune),
        }
    if select_k is not None:
        sel = G.SkinnySelect(M, m.lm_head.shape[0], cfg.hidden, dev, select_k)
        mm["lm_select"] = lambda x, y, wn, xout, w: sel(G.add_rms_norm(x, y, wn, eps, xout), w)
    return mm


class GemmStep:
    """The projection calls of one decode step over ``M`` rows (see the
    module docstring).  ``run(x)`` returns the logits ([M, vocab] bf16), or
    the selected indices ([M, k] int64) when built with ``select_k``."""

    def __init__(self, m, M: int, mm: dict | None = None, log=None, tune: bool = False,
                 select_k: int | None = None):
        self.m, self.M = m, M
        self.mm = mm if mm is not None else decode_matmuls(m, M, log, tune=tune, select_k=select_k)
        if select_k is not None and "lm_select" not in self.mm:
            raise ValueError("select_k needs an mm dict with an 'lm_select' entry")
        self.select = select_k is not None
        cfg, dev = m.cfg, m.device
        bf16 = torch.bfloat16
        self.xa = torch.empty((M, cfg.hidden), dtype=bf16, device=dev)
        self.xb = torch.empty((M, cfg.hidden), dtype=bf16, device=dev)
        self.zero = torch.zeros((M, cfg.hidden), dtype=bf16, device=dev)
        self.attn_out = torch.zeros((M, cfg.heads * cfg.head_dim), dtype=bf16, device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.out: torch.Tensor | None = None

    @property
    def calls(self) -> int:
        return 4 * len(self.m.layers) + 1

    def run(self, x: torch.Tensor) -> torch.Tensor:
        m, mm = self.m, self.mm
        xa, xb = self.xa, self.xb
        cur, y = x, self.zero
        for layer in m.layers:
            mm["qkv"](cur, y, layer.in_norm, xa, layer.wqkv)
            o = mm["o"](self.attn_out, layer.wo)
            act = mm["gu"](xa, o, layer.post_norm, xb, layer.wgu)
            y = mm["d"](act, layer.wd)
            cur = xb
        last = mm["lm_select"] if self.select else mm["lm"]
        return last(cur, y, m.final_norm, xa, m.lm_head)

    def capture(self, x: torch.Tensor) -> torch.cuda.CUDAGraph:
        """Record run(x) in one graph (after warm-up calls on a side stream);
        replay() then recomputes self.out from the current contents of x and
        attn_out."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                self.run(x)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.out = self.run(x)
        self.graph = g
        return g

    def replay(self) -> torch.Tensor:
        if self.graph is None:
            raise RuntimeError("capture() first")
        self.graph.replay()
        return self.out


@dataclass
class QwenConfig:
    hidden: int = 2560
    intermediate: int = 9728
    layers: int = 36
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    eps: float = 1e-6


def synthetic_model(device, layers: int | None = None, seed: int = 0, scale: float = 0.02, **cfg_overrides):
    """A Qwen3-4B-shaped model object with seeded N(0, scale) bf16 weights and
    N(1, 0.1) norm gains (real checkpoints are not loaded by this library)."""
    cfg = QwenConfig(**cfg_overrides)
    if layers is not None:
        cfg.layers = layers
    dev = torch.device(device)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def w(rows, cols):
        return torch.randn((rows, cols), generator=g, device=dev).mul_(scale).to(torch.bfloat16)

    def gain(n):
        return torch.randn((n,), generator=g, device=dev).mul_(0.1).add_(1.0).to(torch.bfloat16)

    qkv_rows = (cfg.heads + 2 * cfg.kv_heads) * cfg.head_dim
    Ls = [SimpleNamespace(in_norm=gain(cfg.hidden), wqkv=w(qkv_rows, cfg.hidden),
                          wo=w(cfg.hidden, cfg.heads * cfg.head_dim), post_norm=gain(cfg.hidden),
                          wgu=w(2 * cfg.intermediate, cfg.hidden), wd=w(cfg.hidden, cfg.intermediate))
          for _ in range(cfg.layers)]
    return SimpleNamespace(cfg=cfg, device=dev, layers=Ls, lm_head=w(cfg.vocab, cfg.hidden),
                           final_norm=gain(cfg.hidden))
