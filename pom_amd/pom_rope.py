"""PoM with rotary position embedding on MI355X HIP kernels.

Drop-in for the reference ``pom.pom_rope`` (pom/pom_rope.py): same tables,
buffer names, rotation conventions and ``PoMRoPE.forward`` signature.  The
rotation of every context token's polynomial features is fused into the
aggregation kernel and the query-side rotation of the gate into the gating
kernel, for 1-D and 2-D (axial row/column) RoPE alike.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib, ops
from ._lib import RopeSpec, require_device
from .pom import PoM

__all__ = ["PoMRoPE", "precompute_freqs_1d", "precompute_freqs_2d", "apply_rope_1d", "apply_rope_2d"]


def precompute_freqs_1d(dim: int, max_seq_len: int, base: float = 10000.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables (max_seq_len, dim/2) with theta_i = base^(-i/(dim/2)) — pom/pom_rope.py:93-117."""
    assert dim % 2 == 0, f"dim must be even for 1-D RoPE, got {dim}"
    half = dim // 2
    inv_freq = 1.0 / (base ** (torch.arange(0, half, dtype=torch.float32) / half))
    angles = torch.outer(torch.arange(max_seq_len, dtype=torch.float32), inv_freq)
    return angles.cos(), angles.sin()


def precompute_freqs_2d(dim: int, max_h: int, max_w: int, base: float = 10000.0):
    """Row/column tables (max_h|max_w, dim/4) with theta_i = base^(-i/(dim/4)) — pom/pom_rope.py:120-149."""
    assert dim % 4 == 0, f"dim must be divisible by 4 for 2-D RoPE, got {dim}"
    quarter = dim // 4
    inv_freq = 1.0 / (base ** (torch.arange(0, quarter, dtype=torch.float32) / quarter))
    row = torch.outer(torch.arange(max_h, dtype=torch.float32), inv_freq)
    col = torch.outer(torch.arange(max_w, dtype=torch.float32), inv_freq)
    return row.cos(), row.sin(), col.cos(), col.sin()


def apply_rope_1d(x, positions, freqs_cos, freqs_sin):
    """Rotate-half 1-D RoPE on a (B, N, D) tensor — pom/pom_rope.py:152-180 (helper)."""
    half = x.shape[-1] // 2
    c, s = freqs_cos[positions], freqs_sin[positions]
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)


def apply_rope_2d(x, positions_hw, row_cos, row_sin, col_cos, col_sin):
    """Axial 2-D RoPE on a (B, N, D) tensor — pom/pom_rope.py:183-235 (helper)."""
    q = x.shape[-1] // 4
    r, c = positions_hw[:, 0], positions_hw[:, 1]
    rc, rs, cc, cs = row_cos[r], row_sin[r], col_cos[c], col_sin[c]
    a1, a2, b1, b2 = x[..., :q], x[..., q:2 * q], x[..., 2 * q:3 * q], x[..., 3 * q:]
    return torch.cat([a1 * rc - a2 * rs, a2 * rc + a1 * rs, b1 * cc - b2 * cs, b2 * cc + b1 * cs], dim=-1)


# Contiguous per-head gate tables, one per RoPE buffer (and buffer version).
_HEAD_TABLES: dict = {}


class PoMRoPE(PoM):
    """PoM with RoPE after the polynomial and before gating — pom/pom_rope.py:303-526."""

    def __init__(self, dim: int, degree: int, expand: int, n_groups: int = 1, n_sel_heads: int = 1,
                 bias: bool = False, max_seq_len: int = 4096, max_h: int = 64, max_w: int = 64,
                 rope_base: float = 10000.0, rope_2d: bool = False):
        super().__init__(dim, degree, expand, n_groups, n_sel_heads, bias)
        self.rope_2d = rope_2d
        rope_dim = dim * expand
        if n_sel_heads > 1:
            hd = rope_dim // n_sel_heads
            if rope_2d:
                assert n_sel_heads % 4 == 0, f"n_sel_heads ({n_sel_heads}) must be divisible by 4 for 2-D RoPE"
                assert hd >= 4, f"head_dim ({hd}) must be ≥ 4 for 2-D RoPE with n_sel_heads > 1"
            else:
                assert n_sel_heads % 2 == 0, f"n_sel_heads ({n_sel_heads}) must be even for 1-D RoPE"
                assert hd >= 2, f"head_dim ({hd}) must be ≥ 2 for 1-D RoPE with n_sel_heads > 1"
        if rope_2d:
            assert rope_dim % 4 == 0, f"dim * expand ({rope_dim}) must be divisible by 4 for 2-D RoPE"
            rc, rs, cc, cs = precompute_freqs_2d(rope_dim, max_h, max_w, rope_base)
            self.register_buffer("row_cos", rc)
            self.register_buffer("row_sin", rs)
            self.register_buffer("col_cos", cc)
            self.register_buffer("col_sin", cs)
        else:
            assert rope_dim % 2 == 0, f"dim * expand ({rope_dim}) must be even for 1-D RoPE"
            fc, fs = precompute_freqs_1d(rope_dim, max_seq_len, rope_base)
            self.register_buffer("freqs_cos", fc)
            self.register_buffer("freqs_sin", fs)

    def _spec(self, n: int, positions, positions_hw, device) -> RopeSpec:
        """Device RoPE description for tokens with the given positions —
        pom/pom_rope.py:386-437 (full-width tables)."""
        if self.rope_2d:
            if positions_hw is None:
                raise ValueError("positions_hw (N, 2) must be provided when rope_2d=True")
            if positions_hw.shape != (n, 2):
                raise ValueError(f"positions_hw must have shape ({n}, 2), got {tuple(positions_hw.shape)}")
            return RopeSpec(_lib.ROPE_2D, [self.row_cos, self.row_sin, self.col_cos, self.col_sin],
                            positions_hw, device)
        n_max = None
        if positions is None:
            positions, n_max = torch.arange(n, device=device), n
        if positions.shape != (n,):
            raise ValueError(f"positions must have shape ({n},), got {tuple(positions.shape)}")
        return RopeSpec(_lib.ROPE_1D, [self.freqs_cos, self.freqs_sin], positions, device, n_max)

    def _spec_heads(self, n: int, positions, positions_hw, device) -> RopeSpec:
        """Device RoPE description for the n_sel_heads-channel gate: the
        full-width tables taken every head_dim / 2 (1-D) or head_dim (2-D)
        columns, as pom/pom_rope.py:417-437 index them, made contiguous once
        per buffer version."""
        H = self.n_sel_heads
        if self.rope_2d:
            if positions_hw is None:
                raise ValueError("positions_hw (N, 2) must be provided when rope_2d=True")
            if positions_hw.shape != (n, 2):
                raise ValueError(f"positions_hw must have shape ({n}, 2), got {tuple(positions_hw.shape)}")
            st, q = self.head_dim, H // 4
            tabs = [_lib.derived(_HEAD_TABLES, t, lambda u: u[:, ::st][:, :q].float().contiguous())
                    for t in (self.row_cos, self.row_sin, self.col_cos, self.col_sin)]
            return RopeSpec(_lib.ROPE_2D, tabs, positions_hw, device)
        n_max = None
        if positions is None:
            positions, n_max = torch.arange(n, device=device), n
        if positions.shape != (n,):
            raise ValueError(f"positions must have shape ({n},), got {tuple(positions.shape)}")
        st, half = self.head_dim // 2, H // 2
        tabs = [_lib.derived(_HEAD_TABLES, t, lambda u: u[:, ::st][:, :half].float().contiguous())
                for t in (self.freqs_cos, self.freqs_sin)]
        return RopeSpec(_lib.ROPE_1D, tabs, positions, device, n_max)

    def _rope_torch(self, x: torch.Tensor, positions, positions_hw) -> torch.Tensor:
        """PoMRoPE._rope — pom/pom_rope.py:386-437 as tensor ops: full-width
        tables for P channels, tables strided by head_dim (2-D) or head_dim / 2
        (1-D) for the n_sel_heads-channel gate."""
        n, d = x.shape[1], x.shape[-1]
        if self.rope_2d:
            if positions_hw is None:
                raise ValueError("positions_hw (N, 2) must be provided when rope_2d=True")
            pos = positions_hw.to(x.device)
            if d == self._po_dim:
                return apply_rope_2d(x, pos, self.row_cos, self.row_sin, self.col_cos, self.col_sin)
            st, q = self.head_dim, d // 4
            return apply_rope_2d(x, pos, self.row_cos[:, ::st][:, :q], self.row_sin[:, ::st][:, :q],
                                 self.col_cos[:, ::st][:, :q], self.col_sin[:, ::st][:, :q])
        pos = torch.arange(n, device=x.device) if positions is None else positions.to(x.device)
        if d == self._po_dim:
            return apply_rope_1d(x, pos, self.freqs_cos, self.freqs_sin)
        st, half = self.head_dim // 2, d // 2
        return apply_rope_1d(x, pos, self.freqs_cos[:, ::st][:, :half], self.freqs_sin[:, ::st][:, :half])

    def forward(self, xq: torch.Tensor, xc: Optional[torch.Tensor] = None, mask=None,
                positions: Optional[torch.Tensor] = None, ctx_positions: Optional[torch.Tensor] = None,
                positions_hw: Optional[torch.Tensor] = None,
                ctx_positions_hw: Optional[torch.Tensor] = None) -> torch.Tensor:
        """pom/pom_rope.py:443-526.  Context features are rotated before they are
        aggregated (inside the aggregation kernel), the query gate after the
        hardsigmoid (inside the gating kernel; the per-head kernels for
        n_sel_heads > 1)."""
        self_mixing = xc is None or xc is xq
        if xc is None:
            xc = xq
        require_device(xq, xc)
        eff_ctx = ctx_positions if ctx_positions is not None else (positions if self_mixing else None)
        eff_ctx_hw = ctx_positions_hw if ctx_positions_hw is not None else (positions_hw if self_mixing else None)
        rope_h = self._spec(xc.shape[1], eff_ctx, eff_ctx_hw, xc.device)
        rot_h = lambda t: self._rope_torch(t, eff_ctx, eff_ctx_hw)
        fl = self._frame_len(mask, xc.shape[1])
        spec_s = self._spec_heads if self.n_sel_heads > 1 else self._spec
        rope_s = spec_s(xq.shape[1], positions, positions_hw, xq.device)
        if self._fused_ok(xq, xc) and (mask is None or fl is not None or
                                        (isinstance(mask, torch.Tensor) and mask.dim() == 2)):
            m = mask if isinstance(mask, torch.Tensor) else None
            out, _ = ops.pom_layer(xq, self.qc_proj.weight, self.se_bias, self.po_coeff,
                                   self.ag_proj.weight, self.ag_proj.bias, self.order, fl, m,
                                   rope_h, rope_s, heads=self.n_sel_heads)
            return out
        return self._mix(xq, xc, mask, fl, rope_h, rope_s, rot_h)
