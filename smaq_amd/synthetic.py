"""Seeded synthetic KV workloads shaped like the benchmark configurations.

Keys follow N(0, Sigma) with Sigma = U diag(1/i) U^T for a seeded, sign-fixed
random orthogonal U (a spectrally decaying query/key covariance); values are
N(0, 1).  Used by bench.py and the tests; everything is generated on the
requested device in chunks so multi-GB caches never need a CPU copy.
"""

from __future__ import annotations

import torch


def spectral_sigma(d: int = 128, seed: int = 0):
    """(Sigma, U, lam) with Sigma = U diag(lam) U^T, lam_i = 1/i (fp32, CPU)."""
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(d, d, generator=g, dtype=torch.float64)
    q, r = torch.linalg.qr(a)
    q = q * torch.sign(torch.diagonal(r)).unsqueeze(0)
    lam = 1.0 / torch.arange(1, d + 1, dtype=torch.float64)
    return ((q * lam) @ q.T).float(), q.float(), lam.float()


def sample_keys(n: int, d: int = 128, seed: int = 1, sigma_seed: int = 0, device="cpu",
                dtype=torch.float32, chunk: int = 1 << 22) -> torch.Tensor:
    """n keys ~ N(0, Sigma) computed as z diag(sqrt lam) U^T."""
    _, u, lam = spectral_sigma(d, sigma_seed)
    dev = torch.device(device)
    mix = (u * lam.sqrt().unsqueeze(0)).T.contiguous().to(dev)   # diag(sqrt lam) U^T
    g = torch.Generator(device=dev).manual_seed(seed)
    out = torch.empty(n, d, dtype=dtype, device=dev)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        z = torch.randn(e - s, d, generator=g, device=dev)
        out[s:e] = (z @ mix).to(dtype)
    return out


def sample_values(n: int, d: int = 128, seed: int = 2, device="cpu", dtype=torch.float32) -> torch.Tensor:
    g = torch.Generator(device=torch.device(device)).manual_seed(seed)
    return torch.randn(n, d, generator=g, device=device).to(dtype)


def student_t(shape, generator: torch.Generator, device, df: int = 3, dtype=torch.bfloat16) -> torch.Tensor:
    """Heavy-tailed keys: each element Student-t(df) = N(0,1) / sqrt(chi2_df / df),
    with the chi-square drawn as a sum of df squared normals (all from
    `generator`, on `device`)."""
    z = torch.randn(shape, generator=generator, device=device)
    chi = torch.randn((*shape, df), generator=generator, device=device).square().sum(-1) / float(df)
    return (z / chi.sqrt()).to(dtype)


def paged_lengths_and_table(batch: int, block_size: int, seed: int, lo: int = 1024, hi: int = 16384):
    """Sequence lengths U[lo, hi] and a shuffled block table over exactly the
    blocks they need: (lens int64 [batch], table int32 [batch, max_blocks],
    physical block count)."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (batch,), generator=g)
    nblk = (lens + block_size - 1) // block_size
    total = int(nblk.sum())
    perm = torch.randperm(total, generator=g)
    table = torch.zeros(batch, int(nblk.max()), dtype=torch.int32)
    o = 0
    for b in range(batch):
        table[b, :nblk[b]] = perm[o:o + nblk[b]].to(torch.int32)
        o += int(nblk[b])
    return lens, table, total
