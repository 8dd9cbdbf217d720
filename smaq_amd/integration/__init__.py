"""vLLM integration (drop-in for smaq/integration/__init__.py)."""

from smaq_amd.integration.vllm import (MODE_CAPTURE_ONLY, MODE_FULL_SMAQ, MODE_HYBRID, MODE_OFF, free_kv_cache,
                                       get_mode, get_stats, install_hooks, set_mode)

__all__ = ["MODE_CAPTURE_ONLY", "MODE_FULL_SMAQ", "MODE_HYBRID", "MODE_OFF", "free_kv_cache", "get_mode",
           "get_stats", "install_hooks", "set_mode"]
