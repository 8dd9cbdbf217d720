"""Spectral shaping of the query metric (drop-in for smaq/ssf.py:8-29).

Runs once per layer (or per block) on the host and produces kernel inputs:
``E`` and ``E_inv``.  It always computes on the CPU in fp32 so that the metric
a GPU encoder receives is the same, bit for bit, whichever device the caller
keeps the calibration data on.
"""

from __future__ import annotations

import torch


def ssf_log(eigvals: torch.Tensor, c: float = 5.0) -> torch.Tensor:
    """Log-compressed, volume-normalised spectrum: exp(l - mean l) with
    l = log(max(log1p(c * max(lambda, 0)), 1e-8))  (smaq/ssf.py:8-18)."""
    shaped = torch.log1p(c * eigvals.clamp(min=0))
    logs = torch.log(shaped.clamp(min=1e-8))
    return torch.exp(logs - logs.mean())


def build_smaq_metric(Sigma_q: torch.Tensor, c: float = 5.0) -> tuple[torch.Tensor, torch.Tensor]:
    """E = V diag(sqrt s) V^T and E_inv = V diag(1/sqrt s) V^T from
    eigh(Sigma_q) (smaq/ssf.py:21-29).  Returned on Sigma_q's device."""
    dev = Sigma_q.device
    sig = Sigma_q.detach().to("cpu", torch.float32)
    evals, evecs = torch.linalg.eigh(sig)
    s = ssf_log(evals, c)
    E = evecs @ torch.diag(s.sqrt()) @ evecs.T
    E_inv = evecs @ torch.diag(1.0 / s.sqrt()) @ evecs.T
    return E.to(dev), E_inv.to(dev)
