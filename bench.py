#!/usr/bin/env python3
"""Benchmark of the MI355X skinny decode GEMM (one GPU).

Headline (one JSON line on stdout): the BASELINE C4 workload — a full
Qwen3-4B decode-step GEMM sweep at M = 32: 36 layers x {qkv 2560->6144,
o 4096->2560, gate_up 2560->19456 + SiLU*mul, down 9728->2560} + lm_head
2560->151936, every layer with its own seeded bf16 weights (8.04 GB, far past
the 256 MB Infinity Cache).  A step is one sweep (145 GEMM calls) replayed from
a HIP graph; ``value`` is algorithmic HBM bytes per second over K steps.

Also reported: the per-GEMM table of the metric (µs, GB/s, % of 8 TB/s at
M = 1, 8, 64 for every projection, torch F.linear on the GPU timed the same
way), each projection's pure-read floor (the fastest single launch that only
reads its weight bytes, libkrk_probe.so, swept over launch shapes), the
roofline of the dominant kernel, and the CPU baseline (torch bf16 F.linear on
this host's cores, the reference's own call).  The per-GEMM cells come last,
in the log and at the end of the JSON line (``per_gemm_summary``), so a
reader of the output's tail sees all fifteen.

Algorithmic bytes per call: 2·(N_w·K + M·K + M·N_out).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "kernel-rush-kawk_amd"))

HBM_PEAK_GBPS = 8000.0
# Calls per timed graph in the per-shape tables (the weights cycle through
# the available copies): a graph replay costs ~10 us beyond its kernels, which
# over 4 calls adds 2.5 us to each (lm_head with its 2 weight copies).
MIN_CALLS = 32
HIDDEN, INTER, VOCAB, LAYERS, QW = 2560, 9728, 151936, 36, 4096
# name -> (K, N_w, silu)
SHAPES = {
    "qkv": (HIDDEN, 6144, False),
    "o": (QW, HIDDEN, False),
    "gate_up": (HIDDEN, 2 * INTER, True),
    "down": (INTER, HIDDEN, False),
    "lm_head": (HIDDEN, VOCAB, False),
}
TENSOR_ID = {"x": 0, "qkv": 1, "o": 2, "gate_up": 3, "down": 4, "lm_head": 5}
# krk_gemm_config.kernel -> device function name (as rocprofv3 reports it)
KERNEL_NAMES = {1: "mfma_gemm_kernel", 2: "valu_gemm_kernel", 3: "mfma_lds_kernel", 5: "stream_gemm_kernel",
                6: "slice_gemm_kernel"}


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def algo_bytes(name: str, M: int) -> int:
    K, Nw, silu = SHAPES[name]
    nout = Nw // 2 if silu else Nw
    return 2 * (Nw * K + M * K + M * nout)


def seed_for(config: int, layer: int, tensor: str) -> int:
    return 1000 * config + 10 * layer + TENSOR_ID[tensor]


def randn_bf16(torch, shape, seed, scale, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    t = torch.randn(shape, generator=g, dtype=torch.float32, device=device)
    return t.mul_(scale).to(torch.bfloat16)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--M", type=int, default=32, help="rows of the headline sweep (C4: 32)")
    ap.add_argument("--no-table", action="store_true", help="skip the per-GEMM M=1/8/64 table")
    ap.add_argument("--no-torch", action="store_true", help="skip the torch-GPU comparison timings")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU-baseline sample length")
    ap.add_argument("--profile-shape", choices=sorted(SHAPES), default=None,
                    help="only replay one projection at --M over its distinct weights (graph of 36 launches, 8 for "
                         "lm_head, 4 replays) and a 256 MiB device copy: the counter workload of profiles/")
    ap.add_argument("--floor", action="store_true",
                    help="only measure the pure-read floor of every projection's weight bytes (launch-shape sweep of "
                         "libkrk_probe.so's read kernel over the rotating weight copies) and print it as JSON")
    ap.add_argument("--calls", type=int, default=0,
                    help="with --profile-shape: launches per graph (default 36, 8 for lm_head)")
    ap.add_argument("--profile-dominant", action="store_true",
                    help="only replay the dominant kernel (gate_up at --M over 36 layer weights, 3 graph replays) "
                         "and a 256 MiB device copy: the workload the committed rocprofv3 --pmc summaries measure")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (collectives are out of "
              "scope); run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    import torch.nn.functional as F

    from kernels import gemm as G
    from kernels.timing import GraphReplay, replay_ms

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} ({getattr(props, 'gcnArchName', '?')}), {props.multi_processor_count} CUs")

    if args.profile_dominant:
        return profile_dominant(torch, G, dev, args.M)
    if args.profile_shape:
        return profile_shape(torch, G, dev, args.profile_shape, args.M, args.calls)

    # ------------------------------------------------------------ weights
    t0 = time.time()
    cfgid = 4
    layers = []
    for l in range(LAYERS):
        layers.append({name: randn_bf16(torch, (SHAPES[name][1], SHAPES[name][0]), seed_for(cfgid, l, name), 0.02, dev)
                       for name in ("qkv", "o", "gate_up", "down")})
    lm = [randn_bf16(torch, (VOCAB, HIDDEN), seed_for(cfgid, 99, "lm_head") + i, 0.02, dev) for i in range(2)]
    torch.cuda.synchronize()
    log(f"weights: {sum(t.numel() for L in layers for t in L.values()) * 2 / 1e9 + 2 * lm[0].numel() * 2 / 1e9:.2f} GB "
        f"in {time.time() - t0:.1f}s")
    if args.floor:
        print(json.dumps({"floor": floor_table(torch, dev, layers, lm)}), flush=True)
        return 0

    # ------------------------------------------------------------ headline sweep
    M = args.M
    x = {name: randn_bf16(torch, (M, SHAPES[name][0]), seed_for(cfgid, 0, "x") + SHAPES[name][0], 1.0, dev)
         for name in ("qkv", "o", "gate_up", "down", "lm_head")}
    ops = {name: (G.SkinnyGateUp(M, SHAPES[name][1] // 2, SHAPES[name][0], dev) if SHAPES[name][2]
                  else G.SkinnyMatmul(M, SHAPES[name][1], SHAPES[name][0], dev))
           for name in SHAPES}
    outs = {name: torch.empty((M, SHAPES[name][1] // 2 if SHAPES[name][2] else SHAPES[name][1]),
                              dtype=torch.bfloat16, device=dev) for name in SHAPES}

    def sweep():
        for L in layers:
            for name in ("qkv", "o", "gate_up", "down"):
                ops[name].run(x[name], L[name], outs[name])
        ops["lm_head"].run(x["lm_head"], lm[0], outs["lm_head"])

    # parity spot check of the sweep's calls against torch on the GPU (not the oracle)
    sweep()
    torch.cuda.synchronize()
    for name in ("qkv", "o", "gate_up", "down"):
        ref = F.linear(x[name], layers[-1][name])
        if SHAPES[name][2]:
            ref = F.silu(ref[:, :INTER]) * ref[:, INTER:]
        err = (outs[name].float() - ref.float()).abs()
        tol = 2e-2 + 1e-2 * ref.float().abs()
        if not bool((err <= tol).all()):
            log(f"PARITY FAILURE in {name}: max err {err.max().item():.4g}")
            return 1
    # lm_head argmax of the sweep against the CPU oracle on the same bits
    # (the reference's torch F.linear on the host, fp32 accumulation).
    sys.path.insert(0, str(ROOT))
    from oracle import gemm_ref as R

    ref_lm = R.linear_bf16(x["lm_head"].cpu(), lm[0].cpu())
    argmax_ok = bool(torch.equal(R.argmax_rows(ref_lm), R.argmax_rows(outs["lm_head"].cpu())))
    log(f"C4 lm_head argmax equals the oracle's on all {M} rows: {argmax_ok}")

    sweep_bytes = LAYERS * sum(algo_bytes(n, M) for n in ("qkv", "o", "gate_up", "down")) + algo_bytes("lm_head", M)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        sweep()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g_sweep = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_sweep):
        sweep()
    for _ in range(args.warmup):
        g_sweep.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(args.steps):
        g_sweep.replay()
    ev1.record()
    torch.cuda.synchronize()
    ms_per_step = ev0.elapsed_time(ev1) / args.steps
    value = sweep_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"sweep M={M}: {ms_per_step * 1000:.1f} us/step, {value:.0f} GB/s ({100 * value / HBM_PEAK_GBPS:.1f}% of 8 TB/s)")

    # ------------------------------------------------------------ dominant kernel roofline
    # gate_up carries 45% of a sweep's bytes.  Its average launch duration is
    # timed with HIP events on the replay stream around a graph of 36
    # back-to-back launches over the 36 distinct layer weights.
    dom = "gate_up"
    dom_calls = [(lambda L=L: ops[dom].run(x[dom], L[dom], outs[dom])) for L in layers]
    dom_ms = replay_ms(dom_calls, reps=max(5, args.steps // 4))
    dom_bytes = algo_bytes(dom, M)
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    traffic = measured_traffic(dom, M, ops[dom].resolved_config)
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                "kernel": f"{dom} M={M} ({KERNEL_NAMES[ops[dom].resolved_config['kernel']]}, SiLU*mul)",
                "config": ops[dom].resolved_config, "us_per_launch": round(dom_ms * 1000, 2),
                "bytes_per_launch": dom_bytes}
    log(f"roofline {dom}: {dom_ms * 1000:.2f} us/launch, {achieved:.0f} GB/s")

    # ------------------------------------------------------------ per-GEMM table (M = 1, 8, 64)
    table = []
    if not args.no_table:
        for Mt in (1, 8, 64):
            for name in SHAPES:
                K, Nw, silu = SHAPES[name]
                xt = randn_bf16(torch, (Mt, K), 77 + Mt + K, 1.0, dev)
                op = G.SkinnyGateUp(Mt, Nw // 2, K, dev) if silu else G.SkinnyMatmul(Mt, Nw, K, dev)
                ot = torch.empty((Mt, Nw // 2 if silu else Nw), dtype=torch.bfloat16, device=dev)
                ws = lm if name == "lm_head" else [L[name] for L in layers]
                n = max(MIN_CALLS, len(ws))
                calls = [(lambda w=ws[i % len(ws)]: op.run(xt, w, ot)) for i in range(n)]
                ms = replay_ms(calls)
                row = {"shape": name, "M": Mt, "us": round(ms * 1000, 2),
                       "GBps": round(algo_bytes(name, Mt) / (ms * 1e-3) / 1e9, 1)}
                row["pct_peak"] = round(100 * row["GBps"] / HBM_PEAK_GBPS, 1)
                row["config"] = op.resolved_config
                if not args.no_torch:
                    if silu:
                        tcalls = [(lambda w=ws[i % len(ws)]: (lambda r: F.silu(r[:, :INTER]) * r[:, INTER:])(F.linear(xt, w)))
                                  for i in range(n)]
                    else:
                        tcalls = [(lambda w=ws[i % len(ws)]: F.linear(xt, w)) for i in range(n)]
                    tms = replay_ms(tcalls)
                    row["torch_gpu_us"] = round(tms * 1000, 2)
                table.append(row)
        floors = floor_table(torch, dev, layers, lm)
        for row in table:
            row["floor_us"] = floors[row["shape"]]["us"]
            row["x_floor"] = round(row["us"] / row["floor_us"], 3)

    # ------------------------------------------------------------ one GPU's 8-way tensor-parallel shard
    # The per-GPU shapes of an 8-GPU deployment (QKV, gate_up and lm_head
    # column-parallel, o and down row-parallel), at their real sizes: the
    # dispatch rule's plan, the warm-up tuner's choice (3 s budget per shape),
    # and torch, each over enough distinct weight copies to exceed the
    # 256 MB Infinity Cache.
    shards = []
    if not args.no_table:
        from kernels import budget as B
        from kernels import tune as T

        tp8 = {"qkv": (2560, 768, False), "gate_up": (2560, 2 * 1216, True), "o": (512, 2560, False),
               "down": (1216, 2560, False), "lm_head": (2560, 18992, False)}
        for name, (K, Nw, silu) in tp8.items():
            copies = min(128, -(-(300 << 20) // (Nw * K * 2)))
            wsh = [randn_bf16(torch, (Nw, K), 7000 + 131 * i + Nw, 0.02, dev) for i in range(copies)]
            for Mt in (1, 32):
                xt = randn_bf16(torch, (Mt, K), 7001 + Mt + K, 1.0, dev)
                epi = G.EPILOGUE_SILU_MUL if silu else G.EPILOGUE_NONE
                op = G.SkinnyGateUp(Mt, Nw // 2, K, dev) if silu else G.SkinnyMatmul(Mt, Nw, K, dev)
                ot = torch.empty((Mt, Nw // 2 if silu else Nw), dtype=torch.bfloat16, device=dev)
                n = max(MIN_CALLS, len(wsh))
                calls = [(lambda w=wsh[i % len(wsh)]: op.run(xt, w, ot)) for i in range(n)]
                ms = replay_ms(calls)
                B.start(3.0)
                try:
                    tuned = G.tune_projection(xt, wsh[0], epi, ws=wsh, cache=T.TuneCache())
                finally:
                    B.clear()
                nout = Nw // 2 if silu else Nw
                bytes_ = 2 * (Nw * K + Mt * K + Mt * nout)
                row = {"shard": name, "N_w": Nw, "K": K, "M": Mt, "us": round(ms * 1000, 2),
                       "GBps": round(bytes_ / (ms * 1e-3) / 1e9, 1), "config": op.resolved_config,
                       "tuned_us": round(tuned.us, 2), "tuned_config": tuned.config, "candidates_timed": len(tuned.trials)}
                if not args.no_torch:
                    if silu:
                        tc = [(lambda w=wsh[i % len(wsh)]: (lambda r: F.silu(r[:, :Nw // 2]) * r[:, Nw // 2:])(F.linear(xt, w)))
                              for i in range(n)]
                    else:
                        tc = [(lambda w=wsh[i % len(wsh)]: F.linear(xt, w)) for i in range(n)]
                    tms = replay_ms(tc)
                    row["torch_gpu_us"] = round(tms * 1000, 2)
                shards.append(row)
                log(f"tp8 shard {name:8s} M={Mt:3d} {row['us']:8.2f} us {row['GBps']:8.1f} GB/s   tuned {row['tuned_us']:8.2f} us"
                    + (f"   torch {row['torch_gpu_us']:8.2f} us" if "torch_gpu_us" in row else ""))
            del wsh

    # ------------------------------------------------------------ normed projections
    # The qkv, gate_up and lm_head calls of a decode step take rms_norm(x + y)
    # as input (the reference's pick_normed contract).  Three ways of running
    # one, each over the same rotating weights: the library's normed call
    # (one launch where the plan fuses the prologue), the stand-alone prologue
    # kernel followed by the plain projection (two launches), and the torch
    # composition followed by F.linear.
    normed = []
    if not args.no_table:
        eps = 1e-6
        for Mt in (1, 4, 8, 32, 64):
            for name in ("qkv", "gate_up", "lm_head"):
                K, Nw, silu = SHAPES[name]
                xt = randn_bf16(torch, (Mt, K), 91 + Mt, 1.0, dev)
                yt = randn_bf16(torch, (Mt, K), 92 + Mt, 0.5, dev)
                wn = randn_bf16(torch, (K,), 93, 1.0, dev)
                xo = torch.empty_like(xt)
                op = G.SkinnyGateUp(Mt, Nw // 2, K, dev) if silu else G.SkinnyMatmul(Mt, Nw, K, dev)
                ot = torch.empty((Mt, Nw // 2 if silu else Nw), dtype=torch.bfloat16, device=dev)
                ws = lm if name == "lm_head" else [L[name] for L in layers]
                n = max(MIN_CALLS, len(ws))
                fused_ms = replay_ms([(lambda w=ws[i % len(ws)]: op.run(xt, w, ot, norm=(yt, wn, xo, eps)))
                                                    for i in range(n)])
                two_ms = replay_ms([(lambda w=ws[i % len(ws)]: op.run(G.add_rms_norm(xt, yt, wn, eps, xout=xo), w, ot))
                                                  for i in range(n)])
                row = {"shape": name, "M": Mt, "us": round(fused_ms * 1000, 2),
                       "prologue_kernel_plus_gemm_us": round(two_ms * 1000, 2),
                       "one_launch": G.normed_fused(Mt, Nw, K, G.EPILOGUE_SILU_MUL if silu else G.EPILOGUE_NONE)}
                row["plain_gemm_us"] = round(replay_ms([(lambda w=ws[i % len(ws)]: op.run(xt, w, ot))
                                                        for i in range(n)]) * 1000, 2)
                if not args.no_torch:
                    def torch_normed(w):
                        s_ = (xt.float() + yt.float()).to(torch.bfloat16)
                        sf = s_.float()
                        nrm = ((sf * torch.rsqrt((sf * sf).mean(-1, keepdim=True) + eps)).to(torch.bfloat16).float()
                               * wn.float()).to(torch.bfloat16)
                        r = F.linear(nrm, w)
                        return F.silu(r[:, :INTER]) * r[:, INTER:] if silu else r
                    tms = replay_ms([(lambda w=ws[i % len(ws)]: torch_normed(w)) for i in range(n)])
                    row["torch_gpu_us"] = round(tms * 1000, 2)
                normed.append(row)
                log(f"normed M={Mt:3d} {name:8s} {row['us']:8.2f} us ({'1 launch' if row['one_launch'] else '2 launches'})"
                    f"   prologue+gemm {row['prologue_kernel_plus_gemm_us']:8.2f} us   plain gemm {row['plain_gemm_us']:8.2f} us"
                    + (f"   torch {row['torch_gpu_us']:8.2f} us" if "torch_gpu_us" in row else ""))

    # ------------------------------------------------------------ token selection
    # lm_head followed by the per-row argmax (k = 1) or top-8, no caller
    # logits (argmax fused into the VALU / LDS-staged MFMA projections writes
    # none; other plans write them to the workspace and select from there),
    # against the plain projection followed by torch.argmax / torch.topk on
    # its logits (what the reference runs).
    select = []
    if not args.no_table:
        K, Nw, _ = SHAPES["lm_head"]
        for Mt in (1, 8, 32, 64):
            xt = randn_bf16(torch, (Mt, K), 95 + Mt, 1.0, dev)
            plain = G.SkinnyMatmul(Mt, Nw, K, dev)
            lg = torch.empty((Mt, Nw), dtype=torch.bfloat16, device=dev)
            for k in (1, 8):
                op = G.SkinnySelect(Mt, Nw, K, dev, k)
                idx = torch.empty((Mt, k), dtype=torch.int64, device=dev)
                n = max(MIN_CALLS, len(lm))
                f_ms = replay_ms([(lambda w=lm[i % len(lm)]: op.run(xt, w, idx)) for i in range(n)])
                if k == 1:
                    sel = lambda: torch.argmax(lg, dim=-1)
                else:
                    sel = lambda: torch.topk(lg, k, dim=-1).indices
                u_ms = replay_ms([(lambda w=lm[i % len(lm)]: (plain.run(xt, w, lg), sel())) for i in range(n)])
                row = {"M": Mt, "k": k, "us": round(f_ms * 1000, 2), "plain_gemm_plus_torch_select_us": round(u_ms * 1000, 2),
                       "fused": op.fused, "config": op.resolved_config}
                select.append(row)
                log(f"select M={Mt:3d} k={k}  {'fused' if op.fused else 'logits'} {row['us']:8.2f} us   lm_head + torch "
                    f"{'argmax' if k == 1 else 'topk'} {row['plain_gemm_plus_torch_select_us']:8.2f} us")

    # ------------------------------------------------------------ decode step through the engine adapter
    # The 145 projection calls of one decode step as the reference engine
    # issues them (engine/model.py:181-214): kernels.step.decode_matmuls
    # builds the engine's mm dict on the library (normed qkv / gate_up /
    # lm_head, plain o / down), GemmStep runs the residual data flow over the
    # 36 layer weights and is captured in one graph.  Reported: µs per step,
    # the sum of the same calls timed in isolation (each call type in its own
    # graph over the 36 layer weights), their difference per call (the gap
    # between consecutive launches in a replayed step), and the torch
    # composition of the same step (F.linear + torch norm / SwiGLU ops).
    step_rows = []
    if not args.no_table:
        from types import SimpleNamespace

        from kernels import step as S

        gen = torch.Generator(device=dev)
        gen.manual_seed(4321)
        gain = lambda: torch.randn((HIDDEN,), generator=gen, device=dev).mul_(0.1).add_(1.0).to(torch.bfloat16)
        cfg = S.QwenConfig()
        model = SimpleNamespace(cfg=cfg, device=dev, lm_head=lm[0], final_norm=gain(),
                                layers=[SimpleNamespace(in_norm=gain(), wqkv=L["qkv"], wo=L["o"], post_norm=gain(),
                                                        wgu=L["gate_up"], wd=L["down"]) for L in layers])
        eps = cfg.eps
        for Mt in (1, 32):
            st = S.GemmStep(model, Mt)
            xs = randn_bf16(torch, (Mt, HIDDEN), 501 + Mt, 1.0, dev)
            st.attn_out.copy_(randn_bf16(torch, tuple(st.attn_out.shape), 502 + Mt, 1.0, dev))
            st.capture(xs)
            for _ in range(3):
                st.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 10
            e0.record()
            for _ in range(reps):
                st.replay()
            e1.record()
            torch.cuda.synchronize()
            step_us = e0.elapsed_time(e1) / reps * 1000
            mm = st.mm
            xo = torch.empty((Mt, HIDDEN), dtype=torch.bfloat16, device=dev)
            yy = randn_bf16(torch, (Mt, HIDDEN), 503 + Mt, 1.0, dev)
            act = randn_bf16(torch, (Mt, INTER), 504 + Mt, 1.0, dev)
            per = {
                "qkv": [(lambda Lm=Lm: mm["qkv"](xs, yy, Lm.in_norm, xo, Lm.wqkv)) for Lm in model.layers],
                "o": [(lambda Lm=Lm: mm["o"](st.attn_out, Lm.wo)) for Lm in model.layers],
                "gu": [(lambda Lm=Lm: mm["gu"](xs, yy, Lm.post_norm, xo, Lm.wgu)) for Lm in model.layers],
                "d": [(lambda Lm=Lm: mm["d"](act, Lm.wd)) for Lm in model.layers],
                "lm": [(lambda w=w: mm["lm"](xs, yy, model.final_norm, xo, w)) for w in lm * 4],
            }
            iso = {k: replay_ms(v) * 1000 for k, v in per.items()}
            iso_sum = LAYERS * (iso["qkv"] + iso["o"] + iso["gu"] + iso["d"]) + iso["lm"]
            row = {"M": Mt, "calls": st.calls, "us_per_step": round(step_us, 1),
                   "isolated_sum_us": round(iso_sum, 1),
                   "gap_us_per_call": round((step_us - iso_sum) / st.calls, 3),
                   "isolated_us": {k: round(v, 2) for k, v in iso.items()}}
            if not args.no_torch:
                def rms(xx, yv, wn, xout):
                    s_ = (xx.float() + yv.float()).to(torch.bfloat16)
                    xout.copy_(s_)
                    sf = s_.float()
                    r_ = torch.rsqrt(sf.pow(2).mean(-1, keepdim=True) + eps)
                    return ((sf * r_).to(torch.bfloat16).float() * wn.float()).to(torch.bfloat16)

                def torch_step():
                    xa_, xb_ = st.xa, st.xb
                    cur, yv = xs, st.zero
                    for Lm in model.layers:
                        F.linear(rms(cur, yv, Lm.in_norm, xa_), Lm.wqkv)
                        o_ = F.linear(st.attn_out, Lm.wo)
                        gu_ = F.linear(rms(xa_, o_, Lm.post_norm, xb_), Lm.wgu)
                        yv = F.linear(F.silu(gu_[:, :INTER]) * gu_[:, INTER:], Lm.wd)
                        cur = xb_
                    return F.linear(rms(cur, yv, model.final_norm, xa_), model.lm_head)

                tms = replay_ms([torch_step], reps=5)
                row["torch_us_per_step"] = round(tms * 1000, 1)
            step_rows.append(row)
            log(f"decode step M={Mt:3d}: {row['us_per_step']:8.1f} us/step ({st.calls} calls), isolated sum "
                f"{row['isolated_sum_us']:8.1f} us, gap {row['gap_us_per_call']:.2f} us/call"
                + (f", torch {row['torch_us_per_step']:8.1f} us/step" if "torch_us_per_step" in row else ""))
            del st
        del model

    # ------------------------------------------------------------ CPU baseline
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, layers[0], lm[0], x, M, args.cpu_seconds)

    result = {
        "metric": "HBM GB/s (% of peak) & µs per Qwen3-4B decode GEMM at M=1/8/64",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) bf16 weights, random init)",
        "config": {"workload": f"C4 decode-step GEMM sweep, M={M}: 36 layers x {{qkv 2560->6144, o 4096->2560, "
                               "gate_up 2560->19456 + SiLU*mul, down 9728->2560} + lm_head 2560->151936, "
                               "distinct weights per layer", "M": M, "calls_per_step": 4 * LAYERS + 1,
                   "bytes_per_step": sweep_bytes, "graph": True},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2),
        "lm_head_argmax_matches_oracle": argmax_ok,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "normed": normed,
        "select": select,
        "decode_step": step_rows,
        "tp8_shard": shards,
        "per_gemm": table,
        # The metric's own cells, last: shape -> M -> [µs, GB/s, % of 8 TB/s,
        # µs / pure-read floor], plus the floor µs per shape.
        "per_gemm_summary": gemm_summary(table),
    }
    for row in table:
        log(f"M={row['M']:3d} {row['shape']:8s} {row['us']:8.2f} us {row['GBps']:8.1f} GB/s {row['pct_peak']:5.1f}%"
            f"   {row['x_floor']:.2f}x the {row['floor_us']:.2f} us read floor"
            + (f"   torch {row['torch_gpu_us']:8.2f} us" if "torch_gpu_us" in row else ""))
    print(json.dumps(result), flush=True)
    return 0


def gemm_summary(table: list) -> dict:
    out = {}
    for row in table:
        d = out.setdefault(row["shape"], {"floor_us": row["floor_us"]})
        d[str(row["M"])] = [row["us"], row["GBps"], row["pct_peak"], row["x_floor"]]
    return out


PROBE_PATH = ROOT / "kernel-rush-kawk_amd" / "libkrk_probe.so"
FLOOR_BLOCKS = (256, 512, 1024, 2048, 4096)
FLOOR_UNROLL = (2, 4, 8, 16)
FLOOR_ORDER = ("chunked", "interleaved")


def floor_table(torch, dev, layers, lm) -> dict:
    """Pure-read floor of each projection's weight bytes: libkrk_probe.so's
    read kernel (krk_probe_read: workgroups of 512 threads streaming 16-byte
    nontemporal loads, each workgroup one contiguous chunk or groups taken in
    turn, `unroll` loads in flight per thread, nothing else) swept over
    FLOOR_ORDER x FLOOR_BLOCKS x FLOOR_UNROLL, each launch shape timed like
    the GEMMs (graph replay over the same rotating weight copies); the
    fastest launch per shape."""
    import ctypes

    from kernels.timing import replay_ms

    if not PROBE_PATH.exists():
        raise RuntimeError(f"{PROBE_PATH} is missing: build it with __graft_entry__.build()")
    probe = ctypes.CDLL(str(PROBE_PATH))
    probe.krk_probe_read.restype = ctypes.c_int
    probe.krk_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_void_p]
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    out = {}
    for name in SHAPES:
        ws = lm if name == "lm_head" else [L[name] for L in layers]
        nbytes = ws[0].numel() * ws[0].element_size()
        n = max(MIN_CALLS, len(ws))
        best = None
        for order in FLOOR_ORDER:
            for blocks in FLOOR_BLOCKS:
                for unroll in FLOOR_UNROLL:
                    def read(w, blocks=blocks, unroll=unroll, inter=int(order == "interleaved")):
                        rc = probe.krk_probe_read(w.data_ptr(), nbytes, sink.data_ptr(), blocks, unroll, inter,
                                                  torch.cuda.current_stream().cuda_stream)
                        if rc:
                            raise RuntimeError(f"krk_probe_read failed ({rc})")
                    ms = replay_ms([(lambda w=ws[i % len(ws)]: read(w)) for i in range(n)])
                    if best is None or ms < best[0]:
                        best = (ms, order, blocks, unroll)
        ms, order, blocks, unroll = best
        gbps = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"bytes": nbytes, "us": round(ms * 1000, 2), "GBps": round(gbps, 1),
                     "pct_peak": round(100 * gbps / HBM_PEAK_GBPS, 1), "order": order, "blocks": blocks,
                     "unroll": unroll}
        log(f"read floor {name:8s} {nbytes / 1e6:7.2f} MB  {ms * 1000:8.2f} us  {gbps:7.1f} GB/s "
            f"({order}, {blocks} workgroups, {unroll} loads in flight per thread)")
    return out


TRAFFIC_FILE = ROOT / "profiles" / "stream_gemm_gate_up_M32_traffic.json"


def measured_traffic(name: str, M: int, config: dict):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE, each scaled by what
    the counter reads for a device copy of known size), when that summary was
    taken on this exact kernel configuration; None otherwise."""
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    if rec.get("shape") != name or rec.get("M") != M or rec.get("config") != config:
        return None
    return rec.get("traffic_bytes_per_launch")


def profile_shape(torch, G, dev, name: str, M: int, calls: int = 0) -> int:
    """Workload for the counter runs: replays of a graph of launches of one
    projection over distinct weights (the 36 layer weights of the sweep; for
    lm_head 2 copies, 8 launches; ``calls`` launches when given, cycling the
    copies), then 4 copies of a 256 MiB buffer for the counters' byte
    calibration.  Prints the configuration and the event-timed µs per launch
    of the graph (median of 3 replays, after the timer's ~10 ms of untimed
    ones)."""
    K, Nw, silu = SHAPES[name]
    if name == "lm_head":
        ws = [randn_bf16(torch, (Nw, K), seed_for(4, 99, "lm_head") + i, 0.02, dev) for i in range(2)]
        ws = ws * 4
    else:
        ws = [randn_bf16(torch, (Nw, K), seed_for(4, l, name), 0.02, dev) for l in range(LAYERS)]
    if calls > 0:
        ws = [ws[i % len(ws)] for i in range(calls)]
    x = randn_bf16(torch, (M, K), seed_for(4, 0, "x") + K, 1.0, dev)
    op = G.SkinnyGateUp(M, Nw // 2, K, dev) if silu else G.SkinnyMatmul(M, Nw, K, dev)
    out = torch.empty((M, Nw // 2 if silu else Nw), dtype=torch.bfloat16, device=dev)
    calls = [(lambda w=w: op.run(x, w, out)) for w in ws]
    from kernels.timing import GraphReplay

    replay = GraphReplay(calls)  # 3 eager warm-up calls, then the capture and one replay
    ms = replay.ms_per_call(reps=3)  # untimed replays first bring the clocks up
    a = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"profile": name, "shape": name, "M": M, "config": op.resolved_config,
                      "kernel": KERNEL_NAMES[op.resolved_config["kernel"]], "us_per_launch": round(ms * 1000, 3),
                      "algorithmic_bytes": algo_bytes(name, M), "launches_per_replay": len(calls),
                      "copy_bytes": 256 << 20, "copies": 4}), flush=True)
    return 0


def profile_dominant(torch, G, dev, M: int) -> int:
    """The dominant kernel's counter workload (gate_up at --M)."""
    return profile_shape(torch, G, dev, "gate_up", M)


def cpu_baseline(torch, layer0, lm0, x, M, seconds):
    """The reference's CPU path (torch bf16 F.linear, the oracle's routine) on
    this host's cores, over one layer's four projections + lm_head at the sweep
    shape, with the same weight bits as the GPU layer 0."""
    sys.path.insert(0, str(ROOT))
    from oracle import gemm_ref as R

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    w = {k: v.cpu() for k, v in layer0.items()}
    wl = lm0.cpu()
    xc = {k: v.cpu() for k, v in x.items()}
    calls = [lambda: R.linear_bf16(xc["qkv"], w["qkv"]), lambda: R.linear_bf16(xc["o"], w["o"]),
             lambda: R.gateup_bf16(xc["gate_up"], w["gate_up"]), lambda: R.linear_bf16(xc["down"], w["down"]),
             lambda: R.linear_bf16(xc["lm_head"], wl)]
    nbytes = sum(algo_bytes(nm, M) for nm in ("qkv", "o", "gate_up", "down", "lm_head"))
    for c in calls * 2:
        c()
    times = []
    t_end = time.time() + seconds
    while time.time() < t_end or len(times) < 5:
        t = time.perf_counter()
        for c in calls:
            c()
        times.append(time.perf_counter() - t)
    times.sort()
    med = times[len(times) // 2]
    cpu_model = platform.processor() or "?"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    gbps = nbytes / med / 1e9
    log(f"cpu baseline: {med * 1000:.1f} ms per sample, {gbps:.1f} GB/s on {n} threads ({cpu_model})")
    return {"value": round(gbps, 2), "unit": "GB/s", "cores": n, "kind": "port",
            "sample": f"torch bf16 F.linear (fp32 accumulate) on host copies of layer 0's qkv, o, gate_up+SiLU*mul, "
                      f"down and lm_head at M={M} (0.98 GB of weights); median of {len(times)} samples "
                      f"over ~{seconds:.0f}s after 2 warm-ups; {cpu_model}",
            "ms_per_sample": round(med * 1000, 2)}


if __name__ == "__main__":
    sys.exit(main())
