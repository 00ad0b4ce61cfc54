"""Routes of the PoM mixer that are dense products rather than streaming
reductions, run as GPU library operations (no CPU path).

* Dense (B, M, N) masks — ``full_mask_mixer`` (pom/pom.py:41-45): the
  per-token polynomial features are formed on the GPU and mixed with the mask
  as one batched GEMM on the matrix cores, divided by the mask's row sums.
  This is O(M * N * P) by nature; frame-causal video masks should use the
  O(N) ``block_causal(frame_len)`` descriptor instead.

It follows the reference's operation order (pom/pom.py:83-99) so autograd
gives the reference's gradients.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib


def poly_features(x: torch.Tensor, coeff: torch.Tensor, k: int) -> torch.Tensor:
    """(B, N, P) -> (B, N, P) per-token p(act(x)) — pom/pom.py:83-88."""
    _lib.require_device(x)
    h = torch.clamp(F.leaky_relu(x, 0.01), min=-0.1, max=6).unsqueeze(-1)
    hp, powers = h, [h]
    for _ in range(k - 1):
        hp = hp * h
        powers.append(hp)
    return (torch.cat(powers, dim=-1) * coeff.to(x.dtype)).sum(-1)


def full_mask_mix(h: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """(B, N, P) features, (B, M, N) mask -> (B, M, P) — pom/pom.py:41-45, as
    a batched GEMM (mask @ h) divided by the mask's row sums."""
    m = mask.to(device=h.device, dtype=h.dtype)
    if m.dim() != 3 or m.shape[0] != h.shape[0] or m.shape[2] != h.shape[1]:
        raise ValueError(f"mask must have shape (B, M, N) = ({h.shape[0]}, M, {h.shape[1]}), got {tuple(m.shape)}")
    out = torch.bmm(m.contiguous(), h.contiguous())
    return out / m.sum(dim=2, keepdim=True)
