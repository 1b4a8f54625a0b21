"""Shared helpers for the parity tests (seeded inputs, error metrics)."""

import torch

BF16 = torch.bfloat16

# Seeds used throughout (weights, activations, adapters, lengths/ranks/ids).
SEED_W, SEED_X, SEED_A, SEED_META = 0, 1, 2, 3

# Tolerance for floating-point kernels: normalised max error
#   max|gpu - oracle| / max|oracle| <= 1e-2
# i.e. the "1e-2 max relative error" bar, measured against the largest
# magnitude of the reference output so that near-zero entries do not blow up.
REL_TOL = 1e-2


def randn(shape, seed, std=1.0, dtype=BF16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(dtype)


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    den = b.abs().max().item()
    num = (a - b).abs().max().item()
    if den == 0:
        return num
    return num / den


def assert_close(a, b, tol=REL_TOL, what=""):
    e = rel_err(a, b)
    assert e <= tol, f"{what}: normalised max error {e:.3e} > {tol:.1e}"


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    a = a.detach().cpu().contiguous()
    b = b.detach().cpu().contiguous()
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    return torch.equal(a.view(torch.int16) if a.dtype == BF16 else a, b.view(torch.int16) if b.dtype == BF16 else b)
