"""The ``smaq`` import path, served by ``smaq_amd``.

Code written against the reference imports module paths such as
``smaq.score`` or ``smaq.integration.vllm``, and the quantizer reaches its
kernel seam as ``smaq.triton_kernels``.  Each of those paths is registered
here as an alias of the ``smaq_amd`` module that implements it (the module
objects are shared, so state such as the adapter's current mode is one), and
the package re-exports ``smaq_amd``'s public names.  Only the kernel seam has
a different module name: ``smaq.triton_kernels`` is ``smaq_amd.kernels``,
whose ``smaq_attention_scores`` runs the HIP score kernel.
"""

from __future__ import annotations

import importlib
import sys

# reference module path (under smaq.) -> implementing module
_MODULES = {
    "backends": "smaq_amd.backends",
    "block_vq": "smaq_amd.block_vq",
    "calibration": "smaq_amd.calibration",
    "capture": "smaq_amd.capture",
    "core": "smaq_amd.core",
    "kv_cache": "smaq_amd.kv_cache",
    "layout": "smaq_amd.layout",
    "quantizer": "smaq_amd.quantizer",
    "score": "smaq_amd.score",
    "ssf": "smaq_amd.ssf",
    "store": "smaq_amd.store",
    "strategies": "smaq_amd.strategies",
    "triton_kernels": "smaq_amd.kernels",
    "weighted_scalar": "smaq_amd.weighted_scalar",
    "integration": "smaq_amd.integration",
    "integration.vllm": "smaq_amd.integration.vllm",
    "vllm_attn_backend": "smaq_amd.vllm_attn_backend",
}

for _path, _target in _MODULES.items():
    _mod = importlib.import_module(_target)
    sys.modules[f"{__name__}.{_path}"] = _mod
    _parent, _, _leaf = f"{__name__}.{_path}".rpartition(".")
    setattr(sys.modules[_parent], _leaf, _mod)

from smaq_amd import *  # noqa: E402,F401,F403
from smaq_amd import __version__  # noqa: E402,F401
