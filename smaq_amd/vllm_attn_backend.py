"""Legacy vLLM entry point (drop-in for smaq/vllm_attn_backend.py).

The legacy API names three modes: ``shadow`` and ``accumulate`` capture K/V
into the compressed store while vLLM keeps serving attention, ``active``
serves decode steps from the store (hybrid attention).  They map onto the
adapter's capture-only and hybrid modes (``smaq_amd.integration.vllm``),
which does all the work; this module keeps the legacy names, the module-wide
current mode, and the no-alloc start-up hook.

No-alloc start-up: ``enable_no_alloc`` records a configuration and, when
vLLM is importable, wraps two of its methods once per process --
``Executor.get_kv_cache_specs`` first installs the hooks (active, no_alloc)
on every worker through the executor's ``collective_rpc`` and then sizes the
KV cache as before; ``GPUModelRunner._update_hybrid_attention_mamba_layout``
first gives layers that share another layer's KV cache that layer's entry.
Without vLLM it logs a warning and does nothing else.
"""

from __future__ import annotations

import functools
import logging
from typing import Any, Callable, Optional

import smaq_amd.integration.vllm as _adapter

# the reference's logger name (smaq/vllm_attn_backend.py:14)
logger = logging.getLogger("smaq.attn")

MODE_SHADOW = "shadow"
MODE_ACCUMULATE = "accumulate"
MODE_ACTIVE = "active"
_VALID_MODES = (MODE_SHADOW, MODE_ACCUMULATE, MODE_ACTIVE)

# legacy mode -> what the adapter does in it
_ADAPTER_MODE = {MODE_SHADOW: _adapter.MODE_CAPTURE_ONLY,
                 MODE_ACCUMULATE: _adapter.MODE_CAPTURE_ONLY,
                 MODE_ACTIVE: _adapter.MODE_HYBRID}

_GLOBAL_MODE = MODE_ACCUMULATE
# the configuration enable_no_alloc recorded (None until it is called)
_SMAQ_NO_ALLOC_CONFIG: Optional[dict] = None


def set_mode(mode: str) -> None:
    """Switch every installed layer's behaviour (smaq/vllm_attn_backend.py:31-36)."""
    global _GLOBAL_MODE
    if mode not in _ADAPTER_MODE:
        raise ValueError(f"Invalid mode: {mode}. Valid: {_VALID_MODES}")
    _adapter.set_mode(_ADAPTER_MODE[mode])
    _GLOBAL_MODE = mode


def get_mode() -> str:
    return _GLOBAL_MODE


def install_smaq_hooks(model_runner, calibration_covariances=None, key_bits: int = 3, value_bits: int = 2,
                       value_group_size: int = 32, buffer_size: int = 128, initial_layers_count: int = 4,
                       initial_layers_key_bits: int | None = None, mode: str = MODE_ACCUMULATE,
                       no_alloc: bool = False, paged: bool = False):
    """Hook every attention layer of ``model_runner`` (smaq/vllm_attn_backend.py:43-75).

    ``buffer_size`` is the exact recent window (the capture ring's capacity);
    an unknown ``mode`` installs capture-only hooks.  The layer states are
    returned and kept on the runner (``_smaq_states``), with the no-alloc
    flag (``_smaq_no_alloc``).  ``paged`` is the adapter's paged-pool
    extension."""
    global _GLOBAL_MODE
    states = _adapter.install_hooks(
        model_runner, calibration_covariances=calibration_covariances, key_bits=key_bits,
        value_bits=value_bits, value_group_size=value_group_size, ring_capacity=buffer_size,
        initial_layers_count=initial_layers_count, initial_layers_key_bits=initial_layers_key_bits,
        mode=_ADAPTER_MODE.get(mode, _adapter.MODE_CAPTURE_ONLY), no_alloc=no_alloc, paged=paged)
    model_runner._smaq_states = states
    model_runner._smaq_no_alloc = no_alloc
    _GLOBAL_MODE = mode
    return states


def _wrap_once(cls: Any, method: str, marker: str, make: Callable[[Callable], Callable]) -> None:
    """Replace cls.method by make(original), once per class (``marker`` flags it)."""
    if getattr(cls, marker, False):
        return
    setattr(cls, method, make(getattr(cls, method)))
    setattr(cls, marker, True)


def _install_on_worker(cfg: dict, worker) -> dict:
    """Runs inside each vLLM worker (via collective_rpc): hooks from the
    configuration it was sent, serving from the store, vLLM's KV cache unused.
    The configuration travels with the call (bound by functools.partial), so
    workers in other processes see it too."""
    states = install_smaq_hooks(worker.model_runner, mode=MODE_ACTIVE, no_alloc=True, **cfg)
    return {"hooks": len(states)}


def _specs_after_install(original: Callable) -> Callable:
    def get_kv_cache_specs(self):
        cfg = _SMAQ_NO_ALLOC_CONFIG
        if cfg is not None:
            try:
                self.collective_rpc(functools.partial(_install_on_worker, dict(cfg)))
            except Exception as exc:   # workers keep vLLM's own attention
                logger.exception("[SMAQ] collective_rpc failed during no-alloc install: %s", exc)
        return original(self)
    return get_kv_cache_specs


def _layout_with_shared_layers(original: Callable) -> Callable:
    def update_layout(self, kv_caches):
        for layer, owner in getattr(self, "shared_kv_cache_layers", {}).items():
            if layer not in kv_caches and owner in kv_caches:
                kv_caches[layer] = kv_caches[owner]
        return original(self, kv_caches)
    return update_layout


def enable_no_alloc(calibration_covariances=None, key_bits: int = 3, value_bits: int = 2, buffer_size: int = 128,
                    initial_layers_count: int = 4):
    """Have vLLM install the hooks (active, no_alloc) on every worker while
    it sizes its KV cache (smaq/vllm_attn_backend.py:78-149)."""
    global _SMAQ_NO_ALLOC_CONFIG
    _SMAQ_NO_ALLOC_CONFIG = {"calibration_covariances": calibration_covariances, "key_bits": key_bits,
                             "value_bits": value_bits, "buffer_size": buffer_size,
                             "initial_layers_count": initial_layers_count}
    try:
        from vllm.v1.executor.abstract import Executor
        from vllm.v1.worker.gpu_model_runner import GPUModelRunner
    except ImportError:
        logger.warning("[SMAQ] vLLM is not installed; enable_no_alloc is inert.")
        return
    if getattr(Executor, "_smaq_patched", False):
        return
    _wrap_once(GPUModelRunner, "_update_hybrid_attention_mamba_layout", "_smaq_layout_patch",
               _layout_with_shared_layers)
    _wrap_once(Executor, "get_kv_cache_specs", "_smaq_patched", _specs_after_install)
    logger.info("[SMAQ] Patched Executor for automatic no-alloc hook installation")


def free_kv_cache(model_runner):
    """Release vLLM's paged KV cache of the hooked layers (smaq/vllm_attn_backend.py:152-154)."""
    return _adapter.free_kv_cache(model_runner)
