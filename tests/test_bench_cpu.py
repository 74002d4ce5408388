"""bench.py's contract on the host: it measures one GPU and says so when
asked for more (the build has no multi-GPU path), before touching a GPU."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _run(*args, env=None):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, env=env, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2 and r.stdout == ""
    assert "one GPU" in r.stderr


def test_a_multi_rank_launch_is_refused():
    env = dict(os.environ, WORLD_SIZE="4", RANK="0", LOCAL_RANK="0")
    r = _run("--gpus", "1", env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_traffic_record_matches_the_dominant_plan():
    """The committed rocprofv3 traffic record is on the configuration the
    dispatch table picks for the headline's dominant kernel (gate_up at
    M = 32), so bench.py's roofline.traffic is filled, not null."""
    import importlib.util
    import json

    sys.path.insert(0, str(ROOT / "kernel-rush-kawk_amd"))
    from kernels import gemm as G

    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    rec = json.loads(bench.TRAFFIC_FILE.read_text())
    cfg = G.plan(32, 19456, 2560, G.EPILOGUE_SILU_MUL)
    assert rec["config"] == cfg
    assert bench.measured_traffic("gate_up", 32, cfg) == rec["traffic_bytes_per_launch"]
    assert 1.0 <= rec["traffic_bytes_per_launch"] / rec["algorithmic_bytes_per_launch"] < 1.1


def test_probe_library_exports_and_checks_arguments():
    """libkrk_probe.so (bench.py's pure-read floor) exports the function
    include/krk_probe.h declares and rejects bad arguments before any
    launch (no GPU is touched here)."""
    import ctypes
    import re

    lib_path = ROOT / "kernel-rush-kawk_amd" / "libkrk_probe.so"
    header = (ROOT / "include" / "krk_probe.h").read_text()
    declared = set(re.findall(r"\b(krk_\w+)\s*\(", re.sub(r"/\*.*?\*/", "", header, flags=re.S)))
    assert declared == {"krk_probe_read"}
    lib = ctypes.CDLL(str(lib_path))
    f = lib.krk_probe_read
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                  ctypes.c_void_p]
    P, S = 0x10000000, 0x20000000  # never dereferenced: every case fails its checks first
    for args in [(0, 1024, S, 256, 8, 0), (P, 1000, S, 256, 8, 0), (P + 8, 1024, S, 256, 8, 0),
                 (P, 1024, 0, 256, 8, 0), (P, 1024, S, 0, 8, 0), (P, 1024, S, 70000, 8, 0),
                 (P, 1024, S, 256, 3, 1), (P, 0, S, 256, 8, 1)]:
        assert f(*args, None) == -1, args
