"""Polynomial Mixer (PoM) module API on MI355X HIP kernels.

Drop-in for the reference module ``pom.pom`` (pom/pom.py): same class and
function names, constructor arguments, parameter names, initialisation order
and ``state_forward`` carry format.  Every aggregation and gating step runs in
the HIP kernels of libpom_amd.so; the projections are bf16/fp32 GEMMs on
hipBLASLt through torch.  There is no CPU path: CPU tensors raise.

Mask forms accepted by ``forward`` / ``polynomial_aggregation_``:
  None                          mean over tokens                 -> (B, 1, P)
  "causal"                      token-causal prefix mean         -> (B, N, P)
  (B, N) tensor                 weighted (key-padding) mean      -> (B, 1, P)
  ("block_causal", frame_len)   frame-causal mean (video frames) -> compact (B, N/L, P)
                                from polynomial_aggregation_; expanded per token
                                inside the module.  Equivalent to the reference's
                                dense block-lower-triangular (B, N, N) mask.
  (B, M, N) tensor              dense cross mask (pom/pom.py:41-45) as a batched GEMM
                                on the GPU (dense.full_mask_mix)                 -> (B, M, P)
"""
from __future__ import annotations

from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import dense, ops
from ._lib import require_device

__all__ = ["PoM", "pom", "pom_activation", "polynomial_aggregation_", "polynomial_selection_",
           "block_causal"]


def pom_activation(x: torch.Tensor) -> torch.Tensor:
    """clamp(leaky_relu(x, 0.01), -0.1, 6) — pom/pom.py:27-28 (elementwise helper;
    the kernels fuse it into the aggregation)."""
    return torch.clamp(F.leaky_relu(x, 0.01, inplace=False), min=-0.1, max=6)


def block_causal(frame_len: int) -> Tuple[str, int]:
    """Mask descriptor for frame-causal mixing with frames of ``frame_len`` tokens."""
    return ("block_causal", int(frame_len))


def _frame_len_of(mask, n: int) -> Optional[int]:
    if isinstance(mask, tuple) and len(mask) == 2 and mask[0] == "block_causal":
        fl = int(mask[1])
        if fl <= 0 or n % fl:
            raise ValueError(f"frame_len {fl} must divide the sequence length {n}")
        return fl
    return None


def polynomial_aggregation_(x: torch.Tensor, coeff: torch.Tensor, k: int, mask=None) -> torch.Tensor:
    """Polynomial aggregation over the sequence — pom/pom.py:52-100.

    Returns (B, 1, D) for mask=None or a (B, N) mask, (B, N, D) for "causal",
    (B, N/L, D) for ("block_causal", L).
    """
    require_device(x)
    if mask is None:
        return ops.poly_agg_mean_hip(x, coeff, k)
    if isinstance(mask, str):
        if mask == "causal":
            return ops.poly_agg_causal_hip(x, coeff, k)
        raise ValueError(f'Unsupported mask: expected None, "causal", or a 2/3-D tensor.')
    fl = _frame_len_of(mask, x.shape[1])
    if fl is not None:
        return ops.poly_agg_block_causal_hip(x, coeff, k, fl)
    if isinstance(mask, torch.Tensor):
        if mask.dim() == 2:
            return ops.poly_agg_masked_hip(x, mask, coeff, k)
        if mask.dim() == 3:
            return dense.full_mask_mix(dense.poly_features(x, coeff, k), mask)
    raise ValueError(f'Unsupported mask: expected None, "causal", or a 2/3-D tensor.')


def polynomial_selection_(s: torch.Tensor, h: torch.Tensor, n_sel_heads: int) -> torch.Tensor:
    """Gated selection — pom/pom.py:103-122 (broadcast product helper; the
    module path fuses it into the gating kernel)."""
    b, g, dh = h.shape
    t = s.shape[1]
    assert g == 1 or t == 1 or g == t, f"incompatible shapes: g={g} t={t}"
    if n_sel_heads <= 1:
        return (s * h).view(b, max(g, t), dh)
    s = s.unsqueeze(-1)
    h = h.view(b, g, n_sel_heads, dh // n_sel_heads)
    return (s * h).view(b, max(g, t), dh)


def pom(xq: torch.Tensor, xc: torch.Tensor, coeff: torch.Tensor, k: int, n_sel_heads: int,
        mask=None) -> torch.Tensor:
    """Polynomial Mixer: aggregate context polynomially, gate with query — pom/pom.py:125-135."""
    h = polynomial_aggregation_(xc, coeff, k, mask)
    if h.shape[1] not in (1, xq.shape[1]):
        h = h.repeat_interleave(xq.shape[1] // h.shape[1], dim=1)
    return polynomial_selection_(xq, h, n_sel_heads)


class PoM(nn.Module):
    """Polynomial Mixer — pom/pom.py:142-280.

    Args match the reference; n_groups, n_sel_heads and bias default to 1, 1,
    False (the README calls ``PoM(dim, degree, expand)``).
    """

    def __init__(self, dim: int, degree: int, expand: int, n_groups: int = 1, n_sel_heads: int = 1,
                 bias: bool = False):
        super().__init__()
        self.dim = dim
        self.order = degree
        self.order_expand = expand
        self.n_groups = n_groups
        self.n_sel_heads = n_sel_heads
        assert dim % n_groups == 0, "dim must be divisible by n_groups"
        assert n_sel_heads <= 1 or dim * expand % n_sel_heads == 0, \
            "dim * expand must be divisible by n_sel_heads"
        self.head_dim = dim * expand // max(n_sel_heads, 1)
        self._po_dim = expand * dim
        self._se_dim = n_sel_heads if n_sel_heads > 1 else expand * dim
        # Same parameters, names and RNG draw order as pom/pom.py:180-191.
        if n_groups > 1:
            self.po_proj = nn.Conv1d(dim, expand * dim, kernel_size=1, bias=bias, groups=n_groups)
            self.se_proj = nn.Linear(dim, self._se_dim, bias=True)
        else:
            self.qc_proj = nn.Linear(dim, self._po_dim + self._se_dim, bias=False)
            self.se_bias = nn.Parameter(torch.zeros(self._se_dim))
        self.po_coeff = nn.Parameter(torch.randn(dim * expand, degree).clamp(-0.001, 0.001))
        self.ag_proj = nn.Linear(expand * dim, dim, bias=bias)

    # ------------------------------------------------------------------
    def _fused_ok(self, xq, xc) -> bool:
        return self.n_groups == 1 and xq is xc

    def _h_and_gate_input(self, xq, xc):
        """Context projection h and gate pre-activation y_s (without se_bias) —
        pom/pom.py:201-213: one GEMM for self-mixing, sliced into [h | y_s]."""
        if self.n_groups > 1:
            # grouped 1x1 convolution over channels; its output is channel-strided
            h = self.po_proj(xc.transpose(1, 2)).transpose(1, 2).contiguous()
            return h, F.linear(xq, self.se_proj.weight), self.se_proj.bias
        w = self.qc_proj.weight
        if xq is xc:
            y = F.linear(xq, w)
            return y[..., :self._po_dim], y[..., self._po_dim:], self.se_bias
        return F.linear(xc, w[:self._po_dim]), F.linear(xq, w[self._po_dim:]), self.se_bias

    def _aggregate(self, h, mask, frame_len, rope_h=None, rot_h=None):
        """h_agg of the projected context for every mask form (RoPE: rope_h is the
        kernel's table description, rot_h the same rotation as a tensor op)."""
        k = self.order
        if isinstance(mask, torch.Tensor) and mask.dim() == 3:
            p = dense.poly_features(h, self.po_coeff, k)
            return dense.full_mask_mix(rot_h(p) if rot_h is not None else p, mask)
        if isinstance(mask, torch.Tensor) and mask.dim() == 2:
            return ops.poly_agg_masked_hip(h, mask, self.po_coeff, k, rope_h)
        fl = h.shape[1] if frame_len is None else frame_len
        return ops._PolyAgg.apply(h, self.po_coeff, k, fl, None, rope_h, None, 0)

    def _select(self, ys, bias, h_agg, rope_s=None):
        """Gate + selection — pom/pom.py:207 and :103-122 (query-side RoPE
        pom/pom_rope.py:522, :417-437).  One HIP kernel for n_sel_heads <= 1
        (full-width gate), the per-head kernels for n_sel_heads > 1 (one
        scalar gate per head and token)."""
        T, G = ys.shape[1], h_agg.shape[1]
        if G not in (1, T) and T % G:
            raise ValueError("query length must be a multiple of the aggregate's group count")
        if self.n_sel_heads > 1:
            return ops.gate_heads_hip(ys, bias, h_agg, self.n_sel_heads, rope_s)
        return ops.gate_hip(ys, bias, h_agg, rope_s)

    def _mix(self, xq, xc, mask, frame_len, rope_h=None, rope_s=None, rot_h=None):
        """Unfused route: projections, aggregation, gating, out-projection."""
        h, ys, bias = self._h_and_gate_input(xq, xc)
        h_agg = self._aggregate(h, mask, frame_len, rope_h, rot_h)
        return self.ag_proj(self._select(ys, bias, h_agg, rope_s))

    def _frame_len(self, mask, n: int) -> Optional[int]:
        if mask is None:
            return None
        if isinstance(mask, str):
            if mask == "causal":
                return 1
            raise ValueError(f'Unsupported mask: expected None, "causal", or a 2/3-D tensor.')
        return _frame_len_of(mask, n)

    def forward(self, xq: torch.Tensor, xc: Optional[torch.Tensor] = None, mask=None) -> torch.Tensor:
        """pom/pom.py:216-231.  xq (B, T, D); xc (B, N, D) or None (self-mixing)."""
        if xc is None:
            xc = xq
        require_device(xq, xc)
        fl = self._frame_len(mask, xc.shape[1])
        if self._fused_ok(xq, xc) and (fl is not None or mask is None or
                                        (isinstance(mask, torch.Tensor) and mask.dim() == 2)):
            m = mask if isinstance(mask, torch.Tensor) else None
            out, _ = ops.pom_layer(xq, self.qc_proj.weight, self.se_bias, self.po_coeff,
                                   self.ag_proj.weight, self.ag_proj.bias, self.order, fl, m,
                                   heads=self.n_sel_heads)
            return out
        return self._mix(xq, xc, mask, fl)

    def state_forward(self, xq: torch.Tensor, xc: Optional[torch.Tensor] = None,
                      state: Optional[Dict[str, Any]] = None) -> Tuple[torch.Tensor, Dict[str, Any]]:
        """Incremental forward with the running-mean carry — pom/pom.py:233-262.

        'n' counts calls (the reference's h_current.shape[1] is 1 per call) and
        'h' (B, 1, P) is kept in the input dtype.
        """
        if xc is None:
            xc = xq
        require_device(xq, xc)
        carry = None if state is None else state["h"]
        n_past = 0 if state is None else int(state["n"])
        if n_past == 0:
            carry = None   # a fresh or reset() state: (0 * h + h_cur) / 1 == h_cur
        elif not torch.is_tensor(carry):
            carry = torch.full((xq.shape[0], 1, self._po_dim), float(carry), dtype=xq.dtype,
                               device=xq.device)
        if self._fused_ok(xq, xc):
            out, h = ops.pom_layer(xq, self.qc_proj.weight, self.se_bias, self.po_coeff,
                                   self.ag_proj.weight, self.ag_proj.bias, self.order,
                                   carry=carry, n_past=n_past, heads=self.n_sel_heads)
            return out, {"h": h, "n": n_past + 1}
        h_raw, ys, bias = self._h_and_gate_input(xq, xc)
        h = ops.poly_agg_state_hip(h_raw, self.po_coeff, self.order, carry, n_past)
        return self.ag_proj(self._select(ys, bias, h)), {"h": h, "n": n_past + 1}

    @torch.no_grad()
    def ar_forward(self, xq: torch.Tensor, state: Dict[str, Any]) -> Tuple[torch.Tensor, Dict[str, Any]]:
        """Autoregressive forward without aggregation — pom/pom.py:264-275: the gate
        multiplies the raw projected context token by token."""
        require_device(xq)
        B, T, D = xq.shape
        h, ys, bias = self._h_and_gate_input(xq, xq)
        out = self.ag_proj(self._select(ys, bias, h))
        return out, {"max_len": state["max_len"], "h": h, "n": state["n"] + T}

    def reset(self, state: Dict[str, Any]) -> Dict[str, Any]:
        """pom/pom.py:277-280."""
        state["h"] = 0.
        state["n"] = 0
        return state
