"""Import this library's ``kernels`` package under another name.

The reference engine has its own ``kernels`` package (engine/kernels/, on
sys.path as ``kernels``), so this one cannot also be imported as ``kernels``
in the engine's process.  ``load("krk")`` imports it as ``krk`` instead; its
modules use relative imports only, and the HIP library is found next to the
package directory whatever the package is called::

    sys.path.insert(0, "/path/to/repo/kernel-rush-kawk_amd")
    import krk_loader
    krk = krk_loader.load()            # krk.gemm, krk.step, krk.tune, krk.budget
    from krk.step import decode_matmuls
"""

from __future__ import annotations

import importlib
import importlib.util
import sys
from pathlib import Path

_PKG = Path(__file__).resolve().parent / "kernels"


def load(name: str = "krk"):
    """The package imported under ``name`` (once per process), with its
    submodules ``gemm``, ``step``, ``tune`` and ``budget`` loaded."""
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, _PKG / "__init__.py", submodule_search_locations=[str(_PKG)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    try:
        spec.loader.exec_module(mod)
        for sub in ("gemm", "step", "tune", "budget"):
            importlib.import_module(f"{name}.{sub}")
    except BaseException:
        for key in [k for k in sys.modules if k == name or k.startswith(name + ".")]:
            del sys.modules[key]
        raise
    return mod
