"""Decode-step integration on the GPU: the engine-facing projection dict and
the 4·layers + 1 projection calls of one step (kernels.step), against the CPU
oracle composed the same way, eager against graph replay, and the fused
token selection against the step's own logits.

Reference data flow: engine/model.py:181-214 (run_layers), 137-178
(decode_matmuls); graph capture engine/engine.py:187-207.
"""

from __future__ import annotations

import pytest
import torch

from kernels import gemm as G
from kernels import step as S
from oracle import gemm_ref as R

from test_gemm_gpu import assert_parity, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(device):
    return S.synthetic_model(device, layers=2, seed=11)


def _oracle_step(m, x, attn_out):
    """The same data flow in the oracle: bf16 roundings at every call."""
    cpu = lambda t: t.detach().cpu()
    eps = m.cfg.eps
    cur, y = cpu(x), torch.zeros_like(cpu(x))
    for layer in m.layers:
        xa, _ = R.add_rms_norm_bf16(cur, y, cpu(layer.in_norm), eps)
        o = R.linear_bf16(cpu(attn_out), cpu(layer.wo))
        xb, act = R.normed_gateup_bf16(xa, o, cpu(layer.post_norm), eps, cpu(layer.wgu))
        y = R.linear_bf16(act, cpu(layer.wd))
        cur = xb
    _, logits = R.normed_linear_bf16(cur, y, cpu(m.final_norm), eps, cpu(m.lm_head))
    return logits


@pytest.mark.parametrize("M", [1, 8, 32])
def test_step_matches_oracle_and_replays(device, model, M):
    st = S.GemmStep(model, M)
    assert st.calls == 4 * len(model.layers) + 1
    x = R.randn_bf16((M, model.cfg.hidden), 7700 + M).to(device)
    st.attn_out.copy_(R.randn_bf16(tuple(st.attn_out.shape), 7701 + M).to(device))
    say("step eager", M)
    eager = st.run(x).clone()
    torch.cuda.synchronize()
    assert_parity(eager.cpu(), _oracle_step(model, x, st.attn_out), f"step M={M}")
    say("step graph", M)
    st.capture(x)
    for rep in range(3):
        out = st.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager step"
    # New inputs in the captured buffers: the replay recomputes from them.
    x.copy_(R.randn_bf16((M, model.cfg.hidden), 7800 + M).to(device))
    again = st.run(x).clone()
    out = st.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, again)


@pytest.mark.parametrize("M,k", [(1, 1), (8, 1), (32, 8)])
def test_step_token_selection(device, model, M, k):
    """lm_select picks the top k of exactly the logits lm computes."""
    mm = S.decode_matmuls(model, M, tune=False, select_k=k)
    logits_step = S.GemmStep(model, M, mm=mm)
    select_step = S.GemmStep(model, M, mm=mm, select_k=k)
    x = R.randn_bf16((M, model.cfg.hidden), 7900 + M).to(device)
    for st in (logits_step, select_step):
        st.attn_out.copy_(R.randn_bf16(tuple(st.attn_out.shape), 7901 + M).to(device))
    say("step select", M, k)
    logits = logits_step.run(x)
    idx = select_step.run(x)
    torch.cuda.synchronize()
    ref_idx, _ = R.topk_rows(logits, k)
    assert torch.equal(idx.cpu(), ref_idx)
    select_step.capture(x)
    out = select_step.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref_idx)


def test_decode_matmuls_contract(device, model, monkeypatch):
    """The dict has the reference's keys and signatures, fused or with the
    norm as its own kernel (ENGINE_NORM_FUSED=0), and both agree."""
    M = 4
    fused = S.decode_matmuls(model, M, tune=False)
    monkeypatch.setenv("ENGINE_NORM_FUSED", "0")
    split = S.decode_matmuls(model, M, tune=False)
    assert set(fused) == set(split) == {"qkv", "o", "gu", "d", "lm"}
    layer = model.layers[0]
    x = R.randn_bf16((M, model.cfg.hidden), 7950).to(device)
    y = R.randn_bf16((M, model.cfg.hidden), 7951).to(device)
    outs = []
    for mm in (fused, split):
        xo = torch.empty_like(x)
        q = mm["qkv"](x, y, layer.in_norm, xo, layer.wqkv)
        g = mm["gu"](x, y, layer.post_norm, xo, layer.wgu)
        o = mm["o"](torch.zeros((M, 4096), dtype=torch.bfloat16, device=device), layer.wo)
        d = mm["d"](g, layer.wd)
        outs.append((xo.clone(), q, g, o, d))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
