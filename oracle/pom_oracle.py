"""CPU oracle for the PoM hot path — TEST INFRASTRUCTURE ONLY.

This module restates, op for op, the pure-PyTorch algorithm of the reference
Polynomial Mixer (davidpicard/pom) so that the HIP kernels of ``pom_amd`` can
be checked against it.  It is the checker, never the thing measured or
shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it.  The product package never imports it.

Every function cites the reference file:line it follows.  Functions run on
any dtype the caller chooses (fp64 for gradchecks, fp32 for parity); they are
written for clarity, not speed.

Pinning (how each function is checked, see tests/test_oracle.py):
  activation, activation_grad   special points + torch.autograd
  poly_features                 brute-force Python loop on tiny inputs
  agg_mean / agg_masked         brute force; dense mask == mean
  agg_causal                    brute force; last row == mean; tril-einsum form
  agg_block_causal              frame_len=N == mean; frame_len=1 == causal;
                                equals the dense 3-D block mask of the reference
  frame_loop (state_forward)    == full block-causal for equal frames
  running_mean_frames           the reference's state_forward arithmetic on bf16
                                tensors (CPU torch, division differences
                                bounded) and, on the GPU box, bit for bit
  rope tables / apply_rope_*    closed-form angle of one pair; positions 0 ==
                                identity; rotation preserves pair norms
  PoM / PoMRoPE composition     golden fixtures written by the reference itself
                                (tests/golden/make_golden.py)
  ar_forward                    golden fixtures of PoM.ar_forward + reset
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

__all__ = [
    "activation", "poly_features", "agg_mean", "agg_masked", "agg_full_mask",
    "agg_causal", "agg_block_causal", "aggregate", "selection",
    "hardsigmoid", "precompute_freqs_1d", "precompute_freqs_2d",
    "apply_rope_1d", "apply_rope_2d", "OracleParams", "init_params",
    "get_h_s", "pom_forward", "state_forward", "rope_forward",
    "block_causal_dense_mask", "running_mean_frames", "ar_forward",
]


# ---------------------------------------------------------------------------
# Activation and polynomial expansion
# ---------------------------------------------------------------------------

def activation(x: torch.Tensor) -> torch.Tensor:
    """clamp(leaky_relu(x, 0.01), -0.1, 6)  — pom/pom.py:27-28."""
    return torch.clamp(F.leaky_relu(x, 0.01), min=-0.1, max=6.0)


def poly_features(x: torch.Tensor, coeff: torch.Tensor, k: int) -> torch.Tensor:
    """Per-token polynomial p(h) = sum_{j<k} coeff[:, j] * h^(j+1), h = act(x).

    Follows the PyTorch fallback of pom/pom.py:83-88 (also
    pom/pom_rope.py:242-265): powers are built by repeated multiplication,
    stacked on a trailing axis and contracted with ``coeff`` (D, K).
    """
    h = activation(x).unsqueeze(-1)
    powers = [h]
    hp = h
    for _ in range(k - 1):
        hp = hp * h
        powers.append(hp)
    return (torch.cat(powers, dim=-1) * coeff).sum(-1)


# ---------------------------------------------------------------------------
# Aggregations over the sequence axis
# ---------------------------------------------------------------------------

def agg_mean(h: torch.Tensor) -> torch.Tensor:
    """Mean over tokens, (B, N, D) -> (B, 1, D) — pom/pom.py:90-91."""
    return h.mean(dim=1, keepdim=True)


def agg_masked(h: torch.Tensor, mask: torch.Tensor, empty_is_zero: bool = True) -> torch.Tensor:
    """Mask-weighted mean, (B, N, D), (B, N) -> (B, 1, D) — pom/pom.py:35-38.

    The CPU fallback divides 0/0 for a row whose mask is all zero (NaN); the
    GPU kernel the reference ships returns 0 there
    (pom/pom_triton_masked.py:165-167).  ``empty_is_zero`` selects the GPU
    convention, which is the one the HIP path replaces.
    """
    m = mask.to(h.dtype).unsqueeze(-1)
    num = (h * m).sum(dim=1, keepdim=True)
    den = m.sum(dim=1, keepdim=True)
    if empty_is_zero:
        safe = torch.where(den != 0, den, torch.ones_like(den))
        return torch.where(den != 0, num / safe, torch.zeros_like(num))
    return num / den


def agg_full_mask(h: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """Dense cross mask (B, M, N): out[b,m] = sum_n mask*h / sum_n mask — pom/pom.py:41-45."""
    mask = mask.to(h.dtype)
    out = torch.einsum("bnd,bmn->bmd", h, mask)
    return out / mask.sum(dim=2, keepdim=True)


def agg_causal(h: torch.Tensor) -> torch.Tensor:
    """Token-causal prefix mean (B, N, D) -> (B, N, D) — pom/pom.py:92-95.

    The reference builds a dense tril mask; the running-sum form used here is
    the same sum (checked against the tril form in the oracle tests).
    """
    n = h.shape[1]
    csum = torch.cumsum(h, dim=1)
    cnt = torch.arange(1, n + 1, dtype=h.dtype, device=h.device).view(1, n, 1)
    return csum / cnt


def block_causal_dense_mask(batch: int, n: int, frame_len: int, dtype=torch.float32) -> torch.Tensor:
    """The (B, N, N) block-lower-triangular mask a reference user would pass to
    ``PoM.forward`` (pom/pom.py:98-99) for frame-causal mixing: query token m may
    see context token n iff frame(n) <= frame(m)."""
    f = torch.arange(n) // frame_len
    m = (f.view(n, 1) >= f.view(1, n)).to(dtype)
    return m.unsqueeze(0).expand(batch, n, n)


def agg_block_causal(h: torch.Tensor, frame_len: int) -> torch.Tensor:
    """Frame-causal mean, compact form (B, N, D) -> (B, N // frame_len, D).

    Row f is the mean of all tokens in frames 0..f.  Expanding it to every
    token of frame f gives exactly ``agg_full_mask(h, block_causal_dense_mask)``
    (the reference's only full-sequence route, pom/pom.py:41-45); for equal
    frames it is also what the ``state_forward`` loop carries
    (pom/pom.py:252-259).
    """
    b, n, d = h.shape
    assert n % frame_len == 0
    nf = n // frame_len
    fsum = h.reshape(b, nf, frame_len, d).sum(dim=2)
    csum = torch.cumsum(fsum, dim=1)
    cnt = (torch.arange(1, nf + 1, dtype=h.dtype, device=h.device) * frame_len).view(1, nf, 1)
    return csum / cnt


def aggregate(h: torch.Tensor, mask) -> torch.Tensor:
    """Mask dispatch on per-token features — pom/pom_rope.py:268-296 and the
    fallback branches of pom/pom.py:90-100."""
    if mask is None:
        return agg_mean(h)
    if isinstance(mask, str):
        if mask == "causal":
            return agg_causal(h)
        raise ValueError(f"unsupported mask {mask!r}")
    if isinstance(mask, tuple) and mask and mask[0] == "block_causal":
        return agg_block_causal(h, int(mask[1]))
    if isinstance(mask, torch.Tensor):
        if mask.dim() == 2:
            return agg_masked(h, mask)
        if mask.dim() == 3:
            return agg_full_mask(h, mask)
    raise ValueError(f"unsupported mask {mask!r}")


# ---------------------------------------------------------------------------
# Gating
# ---------------------------------------------------------------------------

def hardsigmoid(z: torch.Tensor) -> torch.Tensor:
    """relu6(z + 3) / 6, the function F.hardsigmoid computes (pom/pom.py:207)."""
    return F.hardsigmoid(z)


def selection(s: torch.Tensor, h: torch.Tensor, n_sel_heads: int) -> torch.Tensor:
    """Gated selection — pom/pom.py:103-122.

    n_sel_heads <= 1: s (B, T, D) * h (B, G, D) with G in {1, T}.
    n_sel_heads  > 1: s (B, T, H) scales each of H channel groups of h.
    A compact block-causal h (B, F, D) with T = F * L is expanded per frame.
    """
    b, g, dh = h.shape
    t = s.shape[1]
    if g not in (1, t) and t % g == 0:
        h = h.repeat_interleave(t // g, dim=1)
        g = t
    assert g == 1 or t == 1 or g == t
    if n_sel_heads <= 1:
        return (s * h).reshape(b, max(g, t), dh)
    hv = h.reshape(b, g, n_sel_heads, dh // n_sel_heads)
    return (s.unsqueeze(-1) * hv).reshape(b, max(g, t), dh)


# ---------------------------------------------------------------------------
# RoPE — pom/pom_rope.py:93-235
# ---------------------------------------------------------------------------

def precompute_freqs_1d(dim: int, max_seq_len: int, base: float = 10000.0):
    """cos/sin tables (max_seq_len, dim/2), theta_i = base^(-i/(dim/2)) —
    pom/pom_rope.py:93-117."""
    assert dim % 2 == 0
    half = dim // 2
    inv = 1.0 / (base ** (torch.arange(0, half, dtype=torch.float32) / half))
    ang = torch.outer(torch.arange(max_seq_len, dtype=torch.float32), inv)
    return ang.cos(), ang.sin()


def precompute_freqs_2d(dim: int, max_h: int, max_w: int, base: float = 10000.0):
    """Row and column tables (max_h|max_w, dim/4), theta_i = base^(-i/(dim/4)) —
    pom/pom_rope.py:120-149."""
    assert dim % 4 == 0
    q = dim // 4
    inv = 1.0 / (base ** (torch.arange(0, q, dtype=torch.float32) / q))
    ra = torch.outer(torch.arange(max_h, dtype=torch.float32), inv)
    ca = torch.outer(torch.arange(max_w, dtype=torch.float32), inv)
    return ra.cos(), ra.sin(), ca.cos(), ca.sin()


def _rotate_pair(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, s: torch.Tensor):
    return a * c - b * s, b * c + a * s


def apply_rope_1d(x, positions, fcos, fsin):
    """Rotate-half: channel i pairs with i + D/2 — pom/pom_rope.py:152-180."""
    half = x.shape[-1] // 2
    c, s = fcos[positions], fsin[positions]
    r1, r2 = _rotate_pair(x[..., :half], x[..., half:], c, s)
    return torch.cat([r1, r2], dim=-1)


def apply_rope_2d(x, positions_hw, rcos, rsin, ccos, csin):
    """Quarter layout: [0,q)<->[q,2q) by row, [2q,3q)<->[3q,4q) by column —
    pom/pom_rope.py:183-235."""
    q = x.shape[-1] // 4
    ri, ci = positions_hw[:, 0], positions_hw[:, 1]
    a1, a2 = _rotate_pair(x[..., :q], x[..., q:2 * q], rcos[ri], rsin[ri])
    b1, b2 = _rotate_pair(x[..., 2 * q:3 * q], x[..., 3 * q:], ccos[ci], csin[ci])
    return torch.cat([a1, a2, b1, b2], dim=-1)


# ---------------------------------------------------------------------------
# Module composition
# ---------------------------------------------------------------------------

@dataclass
class OracleParams:
    """Parameters of one PoM / PoMRoPE layer (n_groups == 1)."""
    dim: int
    degree: int
    expand: int
    n_sel_heads: int
    w_qc: torch.Tensor          # (P + S, D), rows [0, P) produce h, [P, P+S) produce s
    se_bias: torch.Tensor       # (S,)
    po_coeff: torch.Tensor      # (P, K)
    w_ag: torch.Tensor          # (D, P)
    b_ag: Optional[torch.Tensor]
    rope: Optional[dict] = None  # tables for PoMRoPE
    n_groups: int = 1
    po_w: Optional[torch.Tensor] = None   # n_groups > 1: Conv1d weight (P, D / G, 1)
    po_b: Optional[torch.Tensor] = None
    se_w: Optional[torch.Tensor] = None   # n_groups > 1: se_proj Linear (S, D) with bias
    se_b: Optional[torch.Tensor] = None

    @property
    def po_dim(self) -> int:
        return self.dim * self.expand

    @property
    def head_dim(self) -> int:
        return self.po_dim // max(self.n_sel_heads, 1)

    def to(self, dtype) -> "OracleParams":
        cv = lambda t: None if t is None else t.detach().to(dtype)
        rope = None if self.rope is None else {k: (cv(v) if torch.is_tensor(v) else v)
                                               for k, v in self.rope.items()}
        return OracleParams(self.dim, self.degree, self.expand, self.n_sel_heads,
                            cv(self.w_qc), cv(self.se_bias), cv(self.po_coeff),
                            cv(self.w_ag), cv(self.b_ag), rope, self.n_groups,
                            cv(self.po_w), cv(self.po_b), cv(self.se_w), cv(self.se_b))


def init_params(dim: int, degree: int, expand: int, n_sel_heads: int = 1, bias: bool = False,
                rope_2d: Optional[bool] = None, max_seq_len: int = 4096, max_h: int = 64,
                max_w: int = 64, rope_base: float = 10000.0) -> OracleParams:
    """Draw parameters in the reference's order from the global torch RNG —
    pom/pom.py:180-191 (n_groups == 1): qc_proj Linear(D, P+S, no bias),
    se_bias zeros, po_coeff randn(P, K).clamp(+-1e-3), ag_proj Linear(P, D).
    ``rope_2d`` not None adds the PoMRoPE tables (pom/pom_rope.py:361-380)."""
    p = dim * expand
    s = n_sel_heads if n_sel_heads > 1 else p
    qc = nn.Linear(dim, p + s, bias=False)
    se_bias = torch.zeros(s)
    coeff = torch.randn(p, degree).clamp(-0.001, 0.001)
    ag = nn.Linear(p, dim, bias=bias)
    rope = None
    if rope_2d is not None:
        if rope_2d:
            rc, rs, cc, cs = precompute_freqs_2d(p, max_h, max_w, rope_base)
            rope = {"rope_2d": True, "row_cos": rc, "row_sin": rs, "col_cos": cc, "col_sin": cs}
        else:
            fc, fs = precompute_freqs_1d(p, max_seq_len, rope_base)
            rope = {"rope_2d": False, "freqs_cos": fc, "freqs_sin": fs}
    return OracleParams(dim, degree, expand, n_sel_heads, qc.weight.detach().clone(),
                        se_bias, coeff, ag.weight.detach().clone(),
                        None if ag.bias is None else ag.bias.detach().clone(), rope)


def get_h_s(prm: OracleParams, xq: torch.Tensor, xc: torch.Tensor, self_mixing: bool = True):
    """Projected context h and hardsigmoid gate s — pom/pom.py:193-214."""
    p = prm.po_dim
    if prm.n_groups > 1:
        h = F.conv1d(xc.transpose(1, 2), prm.po_w, prm.po_b, groups=prm.n_groups).transpose(1, 2)
        return h, hardsigmoid(F.linear(xq, prm.se_w, prm.se_b))
    if self_mixing:
        y = F.linear(xq, prm.w_qc)
        return y[..., :p], hardsigmoid(y[..., p:] + prm.se_bias)
    h = F.linear(xc, prm.w_qc[:p])
    s = hardsigmoid(F.linear(xq, prm.w_qc[p:]) + prm.se_bias)
    return h, s


def _out_proj(prm: OracleParams, sh: torch.Tensor) -> torch.Tensor:
    return F.linear(sh, prm.w_ag, prm.b_ag)


def pom_forward(prm: OracleParams, xq: torch.Tensor, xc: Optional[torch.Tensor] = None,
                mask=None) -> torch.Tensor:
    """PoM.forward — pom/pom.py:216-231 (pom() at :125-135)."""
    self_mixing = xc is None or xc is xq
    xc = xq if xc is None else xc
    h, s = get_h_s(prm, xq, xc, self_mixing)
    h_agg = aggregate(poly_features(h, prm.po_coeff, prm.degree), mask)
    return _out_proj(prm, selection(s, h_agg, prm.n_sel_heads))


def state_forward(prm: OracleParams, xq: torch.Tensor, xc: Optional[torch.Tensor] = None,
                  state: Optional[dict] = None) -> Tuple[torch.Tensor, dict]:
    """PoM.state_forward — pom/pom.py:233-262.

    The per-call aggregate is the plain mean (B, 1, P); 'n' counts calls
    (h_current.shape[1] == 1, :253), so 'h' is the running mean of per-call
    means.  The carry is kept in the input dtype, as the reference does.
    """
    self_mixing = xc is None or xc is xq
    xc = xq if xc is None else xc
    h_raw, s = get_h_s(prm, xq, xc, self_mixing)
    h_cur = agg_mean(poly_features(h_raw, prm.po_coeff, prm.degree))
    n_cur = h_cur.shape[1]
    if state is not None:
        n_past = state["n"]
        h = (n_past * state["h"] + n_cur * h_cur) / (n_past + n_cur)
    else:
        h, n_past = h_cur, 0
    out = _out_proj(prm, selection(s, h, prm.n_sel_heads))
    return out, {"h": h, "n": n_past + n_cur}


def ar_forward(prm: OracleParams, xq: torch.Tensor, state: dict) -> Tuple[torch.Tensor, dict]:
    """PoM.ar_forward — pom/pom.py:264-275: no aggregation; the gate multiplies
    the raw projected context token by token, 'n' advances by T."""
    t = xq.shape[1]
    h, s = get_h_s(prm, xq, xq, True)
    out = _out_proj(prm, selection(s, h, prm.n_sel_heads))
    return out, {"max_len": state["max_len"], "h": h, "n": state["n"] + t}


def running_mean_frames(means: torch.Tensor, dtype, carry: Optional[torch.Tensor] = None,
                        n_past: int = 0) -> torch.Tensor:
    """The carry of a PoM.state_forward loop (pom/pom.py:255-259) over frames.

    ``means`` (B, F, P) holds the per-call means; each is a tensor of ``dtype``
    in the reference (pom/pom_triton.py:348).  Every step is evaluated the way
    torch's GPU kernels evaluate ``(n * h + 1 * m) / (n + 1)`` on ``dtype``
    tensors: each op computes in fp32 and rounds to ``dtype``, and dividing by
    the int ``n + 1`` multiplies by its fp32 reciprocal (ATen's true-divide
    kernel with a host-scalar divisor).  Returns (B, F, P) in ``dtype``.
    """
    out = []
    h = None if carry is None else carry.to(dtype)
    n = n_past
    one = torch.tensor(1.0, dtype=torch.float32)
    for f in range(means.shape[1]):
        m = means[:, f].to(dtype)
        if h is None:
            h = m
        else:
            a = (h.float() * float(n)).to(dtype)
            c = (a.float() + m.float()).to(dtype)
            inv = one / torch.tensor(float(n + 1), dtype=torch.float32)
            h = (c.float() * inv).to(dtype)
        out.append(h)
        n += 1
    return torch.stack(out, dim=1)


def _rope(prm: OracleParams, x: torch.Tensor, positions, positions_hw):
    """PoMRoPE._rope — pom/pom_rope.py:386-437, including the strided tables
    for the n_sel_heads-channel gate."""
    r = prm.rope
    n, d = x.shape[1], x.shape[-1]
    full = prm.po_dim
    if r["rope_2d"]:
        if positions_hw is None:
            raise ValueError("positions_hw (N, 2) must be provided when rope_2d=True")
        if d == full:
            return apply_rope_2d(x, positions_hw, r["row_cos"], r["row_sin"], r["col_cos"], r["col_sin"])
        st, q = prm.head_dim, d // 4
        return apply_rope_2d(x, positions_hw, r["row_cos"][:, ::st][:, :q], r["row_sin"][:, ::st][:, :q],
                             r["col_cos"][:, ::st][:, :q], r["col_sin"][:, ::st][:, :q])
    if positions is None:
        positions = torch.arange(n, device=x.device)
    if d == full:
        return apply_rope_1d(x, positions, r["freqs_cos"], r["freqs_sin"])
    st, half = prm.head_dim // 2, d // 2
    return apply_rope_1d(x, positions, r["freqs_cos"][:, ::st][:, :half], r["freqs_sin"][:, ::st][:, :half])


def rope_forward(prm: OracleParams, xq, xc=None, mask=None, positions=None, ctx_positions=None,
                 positions_hw=None, ctx_positions_hw=None):
    """PoMRoPE.forward — pom/pom_rope.py:443-526 (PyTorch route: poly -> RoPE ->
    aggregate, then query-side rotation of the gate)."""
    self_mixing = xc is None or xc is xq
    xc = xq if xc is None else xc
    h_proj, s = get_h_s(prm, xq, xc, self_mixing)
    ectx = ctx_positions if ctx_positions is not None else (positions if self_mixing else None)
    ectx_hw = ctx_positions_hw if ctx_positions_hw is not None else (positions_hw if self_mixing else None)
    h = _rope(prm, poly_features(h_proj, prm.po_coeff, prm.degree), ectx, ectx_hw)
    h_agg = aggregate(h, mask)
    s = _rope(prm, s, positions, positions_hw)
    return _out_proj(prm, selection(s, h_agg, prm.n_sel_heads))
