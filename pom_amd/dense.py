"""Routes of the PoM mixer that are dense products rather than streaming
reductions, run as GPU library operations (no CPU path).

* Dense (B, M, N) masks — ``full_mask_mixer`` (pom/pom.py:41-45): the
  per-token polynomial features come from the HIP feature kernels and are
  mixed with the mask as one batched GEMM on the matrix cores, divided by the
  mask's row sums.
  This is O(M * N * P) by nature; frame-causal video masks should use the
  O(N) ``block_causal(frame_len)`` descriptor instead.

It follows the reference's operation order (pom/pom.py:83-99) so autograd
gives the reference's gradients.
"""
from __future__ import annotations

import torch

from . import ops


def poly_features(x: torch.Tensor, coeff: torch.Tensor, k: int) -> torch.Tensor:
    """(B, N, P) -> (B, N, P) per-token p(act(x)) — pom/pom.py:83-88 — on the
    HIP feature kernels (pom_features_fwd / _bwd)."""
    return ops.poly_features_hip(x, coeff, k)


class _FullMaskMix(torch.autograd.Function):
    """out = (m @ h) / m.sum(-1): forward and backward as batched GEMMs whose
    operands are made contiguous first (no transposed views reach bmm)."""

    @staticmethod
    def forward(ctx, h, m):
        r = m.sum(dim=2, keepdim=True)
        out = torch.bmm(m.contiguous(), h.contiguous()) / r
        ctx.save_for_backward(h, m, r, out)
        return out

    @staticmethod
    def backward(ctx, go):
        h, m, r, out = ctx.saved_tensors
        g = (go / r).contiguous()
        gh = gm = None
        if ctx.needs_input_grad[0]:
            gh = torch.bmm(m.transpose(1, 2).contiguous(), g)
        if ctx.needs_input_grad[1]:
            # d out[i] / d m[i, j] = (h[j] - out[i]) / r[i]
            gm = torch.bmm(g, h.transpose(1, 2).contiguous()) - (g * out).sum(dim=2, keepdim=True)
        return gh, gm


def full_mask_mix(h: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """(B, N, P) features, (B, M, N) mask -> (B, M, P) — pom/pom.py:41-45, as
    a batched GEMM (mask @ h) divided by the mask's row sums."""
    m = mask.to(device=h.device, dtype=h.dtype)
    if m.dim() != 3 or m.shape[0] != h.shape[0] or m.shape[2] != h.shape[1]:
        raise ValueError(f"mask must have shape (B, M, N) = ({h.shape[0]}, M, {h.shape[1]}), got {tuple(m.shape)}")
    return _FullMaskMix.apply(h, m)
