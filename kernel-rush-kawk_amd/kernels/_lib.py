"""ctypes binding of libkrk_gemm.so (C ABI declared in include/krk_gemm.h).

torch is imported first so that its HIP runtime (soname libamdhip64.so.7) is
the one the library binds to; the process then has a single HIP runtime.
Loading fails loudly when the library has not been built: there is no
fallback path.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = Path(__file__).resolve().parent.parent / "libkrk_gemm.so"

KRK_OK = 0
KRK_ERR_INVALID = -1
KRK_ERR_ALIGN = -2
KRK_ERR_ALIAS = -3
KRK_ERR_WORKSPACE = -4
KRK_ERR_HIP = -5
KRK_ERR_UNSUPPORTED = -6

EPILOGUE_NONE = 0
EPILOGUE_SILU_MUL = 1

KERNEL_AUTO = 0
KERNEL_MFMA = 1
KERNEL_VALU = 2
KERNEL_MFMA_LDS = 3
KERNEL_STREAM = 5
KERNEL_SLICE = 6

#: Every function the header declares, with (restype, argtypes).
_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_size = ctypes.c_size_t


class GemmConfig(ctypes.Structure):
    """``krk_gemm_config``: kernel, m_tiles, n_tiles, unroll, waves, splits, k_chunk, prologue, channels,
    x_preload."""

    _fields_ = [
        ("kernel", _int),
        ("m_tiles", _int),
        ("n_tiles", _int),
        ("unroll", _int),
        ("waves", _int),
        ("splits", _int),
        ("k_chunk", _int),
        ("prologue", _int),
        ("channels", _int),
        ("x_preload", _int),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}

    @classmethod
    def from_dict(cls, d: dict | None) -> "GemmConfig":
        c = cls()
        for k, v in (d or {}).items():
            if k not in dict(cls._fields_):
                raise ValueError(f"unknown config field {k!r}")
            setattr(c, k, int(v))
        return c


SIGNATURES = {
    "krk_gemm_bf16": (_int, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64,
                              _int, _int, _int, _int, _c_void_p, _size, _c_void_p]),
    "krk_gemm_workspace_bytes": (_size, [_int, _int, _int, _int]),
    "krk_gemm_plan": (_int, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig)]),
    "krk_gemm_config_workspace_bytes": (_size, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig)]),
    "krk_gemm_resolve": (_int, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig), ctypes.POINTER(GemmConfig)]),
    "krk_gemm_bf16_config": (_int, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64,
                                     _int, _int, _int, _int, ctypes.POINTER(GemmConfig),
                                     _c_void_p, _size, _c_void_p]),
    "krk_gemm_bf16_normed": (_int, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, ctypes.c_float, _c_void_p, _i64,
                                     _c_void_p, _i64, _c_void_p, _i64, _int, _int, _int, _int,
                                     _c_void_p, _size, _c_void_p]),
    "krk_gemm_bf16_normed_config": (_int, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, ctypes.c_float, _c_void_p,
                                            _i64, _c_void_p, _i64, _c_void_p, _i64, _int, _int, _int, _int,
                                            ctypes.POINTER(GemmConfig), _c_void_p, _size, _c_void_p]),
    "krk_gemm_normed_workspace_bytes": (_size, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig)]),
    "krk_gemm_normed_fused": (_int, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig)]),
    "krk_gemm_normed_plan": (_int, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig)]),
    "krk_add_rms_norm_bf16": (_int, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, ctypes.c_float, _c_void_p, _i64,
                                      _c_void_p, _i64, _int, _int, _c_void_p]),
    "krk_gemm_bf16_select": (_int, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _int, _int, _int, _int,
                                     _c_void_p, _c_void_p, _c_void_p, _size, _c_void_p]),
    "krk_gemm_bf16_select_config": (_int, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _int, _int, _int, _int,
                                            _c_void_p, _c_void_p, ctypes.POINTER(GemmConfig), _c_void_p, _size,
                                            _c_void_p]),
    "krk_gemm_select_workspace_bytes": (_size, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig)]),
    "krk_gemm_select_plan": (_int, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig)]),
    "krk_gemm_select_fused": (_int, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig)]),
    "krk_gemm_bf16_noalloc": (_int, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64,
                                      _int, _int, _int, _int, _c_void_p]),
    "krk_gemm_candidates": (_int, [_int, _int, _int, _int, ctypes.POINTER(GemmConfig), _int]),
    "krk_last_error": (ctypes.c_char_p, []),
    "krk_abi_version": (_int, []),
    "krk_gemm_config_size": (_size, []),
}

#: The ABI this binding was written against (KRK_ABI_VERSION in include/krk_gemm.h).
ABI_VERSION = 4

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load (once) and return the library.  Raises ImportError if it is not built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `python kernel-rush-kawk_amd/build_lib.py` (there is no fallback GEMM)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            abi, size = lib.krk_abi_version(), lib.krk_gemm_config_size()
            if abi != ABI_VERSION or size != ctypes.sizeof(GemmConfig):
                raise ImportError(f"{LIB_PATH}: ABI version {abi} with a {size}-byte krk_gemm_config; this binding "
                                  f"expects version {ABI_VERSION} and {ctypes.sizeof(GemmConfig)} bytes (rebuild the "
                                  "library or update the binding)")
            _lib = lib
    return _lib


_tag = None


def library_tag() -> str:
    """A short digest of the loaded library file: tuned configurations are
    cached under it, so a rebuilt library never reuses another build's
    choices (a configuration may be slower, or no longer instantiated)."""
    global _tag
    with _lock:
        if _tag is None:
            import hashlib

            _tag = hashlib.sha1(LIB_PATH.read_bytes()).hexdigest()[:12]
    return _tag


def last_error() -> str:
    return load().krk_last_error().decode(errors="replace")


class KrkError(RuntimeError):
    """A krk_* call returned an error code; ``code`` is the KRK_ERR_* value."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"krk error {code}: {msg}")
        self.code = code


def check(rc: int) -> None:
    """Raise for a non-zero krk return code.  Argument errors (invalid shape,
    alignment, aliasing, workspace) raise ValueError like the reference's
    launchers (engine/kernels/gateup64.py:63-74); runtime errors RuntimeError."""
    if rc == KRK_OK:
        return
    msg = last_error()
    if rc in (KRK_ERR_INVALID, KRK_ERR_ALIGN, KRK_ERR_ALIAS, KRK_ERR_WORKSPACE, KRK_ERR_UNSUPPORTED):
        raise ValueError(f"krk error {rc}: {msg}")
    raise KrkError(rc, msg)
