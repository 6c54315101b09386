"""Install this package under the reference's import name.

Callers of the reference import ``scmp_kernels`` (``from scmp_kernels import sc_matmul``,
``from scmp_kernels.quant import ...``; scmp_kernels/__init__.py:1-3). A caller that cannot
change its imports runs, once at start-up,

    import scmp_kernels_amd.compat
    scmp_kernels_amd.compat.install()

after which ``scmp_kernels`` and every module path of the reference's call surface
(``scmp_kernels.sc``, ``.sc.matmul``, ``.sc.kernels``, ``.sc.config_helpers``,
``.sc.lfsr_taps``, ``.sc.sng``, ``.sc.rng``, ``.sc.constants``, ``.quant``, ``.quant.fused``,
``.quant.grouped``, ``.quant.smoothquant``, ``.mp``, ``.mp.config``) resolve to this
package's modules. Submodules of the reference that this package does not provide (the MP
auto-calibrator, ``qwt``, ``sensitivity``) stay unimportable under the alias.
"""
from __future__ import annotations

import importlib
import sys

ALIAS = "scmp_kernels"
_SUBMODULES = ("", ".sc", ".sc.matmul", ".sc.kernels", ".sc.config_helpers", ".sc.lfsr_taps",
               ".sc.sng", ".sc.rng", ".sc.constants", ".quant", ".quant.fused",
               ".quant.grouped", ".quant.smoothquant", ".mp", ".mp.config")
_OWN = __name__.rsplit(".", 1)[0]


def install(name: str = ALIAS) -> None:
    """Register this package's modules as ``name`` and ``name.<submodule>``. Raises
    ImportError when another package of that name is already imported (the reference
    itself, for example); installing twice is harmless."""
    have = sys.modules.get(name)
    if have is not None and getattr(have, "__name__", None) != _OWN:
        raise ImportError(f"'{name}' is already imported from "
                          f"{getattr(have, '__file__', '?')}; install the alias before "
                          f"anything imports the reference")
    for sub in _SUBMODULES:
        mod = importlib.import_module(_OWN + sub)
        sys.modules[name + sub] = mod


def uninstall(name: str = ALIAS) -> None:
    """Remove the alias entries that ``install`` added."""
    for sub in _SUBMODULES:
        mod = sys.modules.get(name + sub)
        if mod is not None and getattr(mod, "__name__", "").startswith(_OWN):
            del sys.modules[name + sub]
