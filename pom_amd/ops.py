"""Autograd operators over the HIP kernels (C ABI in include/pom_amd.h).

Kernel-level entry points mirror the reference's Triton entry points, same
arguments, return shapes and dtypes:

  poly_agg_mean_hip(x, coeff, k)             ~ poly_agg_mean_triton        pom/pom_triton.py:383-403
  poly_agg_masked_hip(x, mask, coeff, k)     ~ poly_agg_masked_triton      pom/pom_triton_masked.py:402-428
  poly_agg_causal_hip(x, coeff, k)           ~ poly_agg_causal_triton      pom/pom_triton_causal.py:400-423
  poly_agg_rope_mean_hip(x, coeff, k, fc, fs, positions)
                                             ~ poly_agg_rope_mean_triton   pom/pom_triton_rope.py:985-1017
  poly_agg_rope_causal_hip(...)              ~ poly_agg_rope_causal_triton pom/pom_triton_rope.py:1020-1053
  poly_agg_block_causal_hip(x, coeff, k, frame_len)   frame-causal mean, compact (B, N/L, P)

and the fused layer operator ``pom_layer`` (projection GEMMs + aggregation +
gating) used by the modules.  Inputs are borrowed, never copied: the
aggregation reads a strided view (e.g. the h-half of the fused projection)
and its backward writes grad_x straight into the matching half of dY.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import RopeSpec, check, derived as _derived, dtype_code, ptr, rope_ptr, view3, workspace, stream_handle
from . import gemm_select
from .gemm_select import tuned_gemms


# Optional per-launch timing: when ``kernel_timer`` is a list, every launch
# site below appends (name, start_event, end_event) recorded on the stream the
# launch goes to.  bench.py uses it to time each kernel inside its timed region.
kernel_timer: Optional[list] = None
kernel_timer_only: Optional[set] = None   # record only these names (None: all)


class _Span:
    __slots__ = ("name", "ev")

    def __init__(self, name: str):
        self.name = name
        self.ev = None

    def __enter__(self):
        if kernel_timer is not None and (kernel_timer_only is None or self.name in kernel_timer_only):
            self.ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            self.ev[0].record()
        return self

    def __exit__(self, *exc):
        if self.ev is not None:
            self.ev[1].record()
            kernel_timer.append((self.name, self.ev[0], self.ev[1]))
        return False


# The backward GEMMs in 16-bit types run on operands that are contiguous along
# the reduction dimension (x^T, g^T, sh^T, dY^T for the weight gradients and
# the transposed weights for the data gradients), which the matrix-core GEMMs
# run markedly faster than the strided forms.  POM_AMD_NT_GEMMS=0 disables.
_NT_GEMMS = os.environ.get("POM_AMD_NT_GEMMS", "1") != "0"

# How the token-contiguous copies of sh and dY are made: "fused" (default)
# has the gate / aggregation kernels write them in the same pass (pom_tview
# outputs); "side" transposes them on a second stream (default priority)
# while the next GEMM runs on the current one.  Fused measured faster: the
# overlapped copies slow the concurrent GEMMs by more than they save.  x^T and
# g^T (inputs of the layer) are always transposed on the second stream.
_NT_COPIES = os.environ.get("POM_AMD_NT_COPIES", "fused")
_copy_streams: dict = {}
# POM_AMD_COPY_STREAM=0: the x^T / g^T transposes run on the current stream.
_COPY_STREAM = os.environ.get("POM_AMD_COPY_STREAM", "1") != "0"

# POM_AMD_OVERLAP_GEMMS=1: the weight-gradient GEMMs (off the data-gradient
# chain) also run on the second stream, concurrently with the gating /
# aggregation backward and the data-gradient GEMMs.
_OVERLAP_GEMMS = os.environ.get("POM_AMD_OVERLAP_GEMMS", "0") == "1"
# POM_AMD_SIDE_WGRAD=1: dW_ag on pom_gemm runs on the second stream, beside
# ag_dgrad and the gate / aggregation backward (its units fill fewer CUs
# than the chip has).
_SIDE_WGRAD = os.environ.get("POM_AMD_SIDE_WGRAD", "0") == "1"


def _copy_stream(device: torch.device) -> torch.cuda.Stream:
    if not _COPY_STREAM:
        return torch.cuda.current_stream(device)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    s = _copy_streams.get(idx)
    if s is None:
        s = _copy_streams[idx] = torch.cuda.Stream(device=idx)
    return s


def _check_degree(k: int) -> None:
    if k > _lib.MAX_DEGREE:
        raise NotImplementedError(f"pom_amd kernels support degree k <= {_lib.MAX_DEGREE} (got {k})")
    if k < 1:
        raise ValueError(f"degree must be >= 1 (got {k})")


_f32_cache: dict = {}
_wt_cache: dict = {}
_pad_cache: dict = {}


def _param(t: torch.Tensor) -> torch.Tensor:
    """A coefficient / bias parameter as the kernels take it: the tensor itself
    when it is contiguous fp32, bf16 or fp16 (the kernels read it, and write its
    gradient, in that dtype), else an fp32 contiguous copy cached per
    parameter version."""
    if t.dtype in _lib.DTYPE_CODES and t.is_contiguous():
        return t.detach()
    return _derived(_f32_cache, t, lambda u: u.detach().float().contiguous())


def transpose(t: torch.Tensor, name: str = "transpose") -> torch.Tensor:
    """Contiguous (C, R) copy of a 2-D (R, C) tensor with unit column stride,
    on the HIP transpose kernel (pom_transpose)."""
    _lib.require_device(t)
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError(f"transpose needs a 2-D tensor with unit column stride, got {tuple(t.shape)} "
                         f"strides {t.stride()}")
    lib = _lib.load()
    R, C = t.shape
    out = torch.empty(C, R, dtype=t.dtype, device=t.device)
    with _Span(name):
        rc = lib.pom_transpose(dtype_code(t), R, C, t.data_ptr(), max(t.stride(0), C), out.data_ptr(), R,
                               stream_handle(t.device))
    check(rc, "pom_transpose")
    return out


def invalidate_derived() -> None:
    """Drop every cached parameter-derived copy (fp32 coefficients, transposed
    and padded weights, fp32 RoPE tables), as an optimizer update of all
    parameters would."""
    _lib.invalidate_derived()


def _transpose_into(src: torch.Tensor, dst: torch.Tensor, name: str) -> None:
    """dst (C, R) <- src (R, C)^T; both 2-D with unit inner stride."""
    R, C = src.shape
    with _Span(name):
        rc = _lib.load().pom_transpose(dtype_code(src), R, C, src.data_ptr(), max(src.stride(0), C),
                                       dst.data_ptr(), dst.stride(0), stream_handle(src.device))
    check(rc, "pom_transpose")


def _with_copy(call, out_t, src_rows: torch.Tensor, name: str, what: str, B: int, N: int) -> None:
    """Run a launch that can also write a channel-major copy ``out_t`` of its
    (B, N, C) output.  ``call(tv)`` launches with tv (a PomTView pointer or
    None) and returns the status.  When the kernels do not build the copy for
    this shape (POM_ERR_UNSUPPORTED, raised before any launch), the launch runs
    without it and the copy is made from ``src_rows`` (the output as (B*N, C))
    by the transpose kernel."""
    if out_t is None:
        check(call(None), what)
        return
    rc = call(_lib.tview(out_t, B, N))
    if rc == _lib.POM_ERR_UNSUPPORTED:
        check(call(None), what)
        _transpose_into(src_rows, out_t, name)
        return
    check(rc, what)


# Projection GEMMs on the library's own matrix-core kernel (pom_gemm), which
# reads every operand in its natural layout.  POM_AMD_HIP_GEMMS names the
# products that use it: "wgrad" (default: the two weight gradients), "all",
# "none", or a comma list of gemm_qc_fwd, gemm_ag_fwd, gemm_ag_dgrad,
# gemm_qc_dgrad, gemm_ag_wgrad, gemm_qc_wgrad.  A product whose shape no tile
# of the kernel divides, or whose operands are not bf16, stays on hipBLASLt.
_GEMM_NAMES = ("gemm_qc_fwd", "gemm_ag_fwd", "gemm_ag_dgrad", "gemm_qc_dgrad", "gemm_ag_wgrad", "gemm_qc_wgrad")


def _hip_gemm_set() -> frozenset:
    v = os.environ.get("POM_AMD_HIP_GEMMS", "wgrad").strip()
    if v == "all":
        return frozenset(_GEMM_NAMES)
    if v == "none" or not v:
        return frozenset()
    if v == "wgrad":
        return frozenset(("gemm_ag_wgrad", "gemm_qc_wgrad"))
    names = frozenset(n.strip() for n in v.split(","))
    bad = names - set(_GEMM_NAMES)
    if bad:
        raise ValueError(f"POM_AMD_HIP_GEMMS: unknown product(s) {sorted(bad)}")
    return names


_HIP_GEMMS = _hip_gemm_set()
_plan_cache: dict = {}


def hip_gemm_fits(name: str, M: int, N: int, K: int, dt: torch.dtype) -> bool:
    """Whether product `name` of shape (M, N, K) runs on pom_gemm."""
    if name not in _HIP_GEMMS or dt != torch.bfloat16:
        return False
    key = (M, N, K)
    ok = _plan_cache.get(key)
    if ok is None:
        t, sp = ctypes.c_int(), ctypes.c_int()
        ok = _plan_cache[key] = _lib.load().pom_gemm_plan(M, N, K, 0, 0, ctypes.byref(t), ctypes.byref(sp)) == 0
    return ok


def hip_gemm(a: torch.Tensor, a_mn: bool, b: torch.Tensor, b_mn: bool, out_dtype: torch.dtype = torch.bfloat16,
             name: str = "gemm") -> torch.Tensor:
    """C = A B on pom_gemm, bf16 operands, fp32 accumulation.  a is (M, K) with
    a_mn False or (K, M) with a_mn True; b is (N, K) with b_mn False (an
    nn.Linear weight: y = x W^T) or (K, N) with b_mn True.  Both 2-D with unit
    inner stride.  Returns a fresh (M, N) tensor in out_dtype (bf16 or fp32)."""
    _lib.require_device(a, b)
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise ValueError("hip_gemm takes bf16 operands")
    if a.dim() != 2 or b.dim() != 2 or a.stride(1) != 1 or b.stride(1) != 1:
        raise ValueError("hip_gemm operands must be 2-D with unit inner stride")
    K, M = (a.shape[0], a.shape[1]) if a_mn else (a.shape[1], a.shape[0])
    Kb, N = (b.shape[0], b.shape[1]) if b_mn else (b.shape[1], b.shape[0])
    if Kb != K:
        raise ValueError(f"hip_gemm: inner dimensions differ ({K} and {Kb})")
    lib = _lib.load()
    c = torch.empty(M, N, dtype=out_dtype, device=a.device)
    wsb = lib.pom_gemm_workspace_size(M, N, K, -1, 0)
    ws = torch.empty(wsb, dtype=torch.uint8, device=a.device) if wsb else None
    with _Span(name):
        rc = lib.pom_gemm(1 if a_mn else 0, 1 if b_mn else 0, M, N, K, a.data_ptr(), a.stride(0), b.data_ptr(),
                          b.stride(0), dtype_code(c), c.data_ptr(), c.stride(0), -1, 0,
                          None if ws is None else ws.data_ptr(), wsb, stream_handle(a.device))
    check(rc, "pom_gemm")
    return c


def _wgrad_dtype(param_dtype: torch.dtype) -> torch.dtype:
    """Output dtype of a weight gradient: the parameter's, fp32 for anything but bf16."""
    return torch.bfloat16 if param_dtype == torch.bfloat16 else torch.float32


def _weight_t(w: torch.Tensor) -> torch.Tensor:
    """Transposed copy of a projection weight, cached per weight version."""
    return _derived(_wt_cache, w, lambda u: transpose(u.detach(), "transpose_w"))


def _padded_width(p: int, s: int) -> int:
    """Projection width P + S rounded up to 64 columns: 128-byte-aligned rows of
    Y / dY for the streaming kernels and an aligned GEMM dimension (per-head
    gating makes P + S = P + n_sel_heads, which is rarely aligned)."""
    return (p + s + 63) // 64 * 64


_zero_cache: dict = {}


def _zero_rows(n: int, cols: int, dt: torch.dtype, device: torch.device) -> torch.Tensor:
    """A cached all-zero (n, cols) block; it is only ever read.  Under stream
    capture a fresh block (the graph's own memory, filled on every replay)."""
    if torch.cuda.is_current_stream_capturing():
        return torch.zeros(n, cols, dtype=dt, device=device)
    key = (n, cols, dt, device)
    z = _zero_cache.get(key)
    if z is None:
        z = _zero_cache[key] = torch.zeros(n, cols, dtype=dt, device=device)
    return z


def _qc_weight(w: torch.Tensor, dt: torch.dtype, rows: int) -> torch.Tensor:
    """W_qc in dtype dt with zero rows appended up to ``rows`` (the padded
    projection width), cached per weight version."""
    def make(u):
        u = u.detach().to(dt)
        if u.shape[0] == rows:
            return u
        return torch.cat([u, _zero_rows(rows - u.shape[0], u.shape[1], dt, u.device)])   # one kernel
    if w.dtype == dt and w.shape[0] == rows:
        return w
    return _derived(_pad_cache, w, make)


def _coeff_param(coeff: torch.Tensor, p: int, k: int) -> torch.Tensor:
    if coeff.shape != (p, k):
        raise ValueError(f"coeff must have shape ({p}, {k}), got {tuple(coeff.shape)}")
    return _param(coeff)


# ---------------------------------------------------------------------------
# Raw launches (no autograd)
# ---------------------------------------------------------------------------

def agg_forward(x: torch.Tensor, coeff: torch.Tensor, k: int, frame_len: int,
                mask32: Optional[torch.Tensor] = None, carry: Optional[torch.Tensor] = None,
                n_past: int = 0, rope: Optional[RopeSpec] = None):
    """Launch pom_agg_fwd.  Returns (out (B, N/frame_len, P) x.dtype, count or None)."""
    lib = _lib.load()
    B, N, P = x.shape
    dt = dtype_code(x)
    out = torch.empty(B, N // frame_len, P, dtype=x.dtype, device=x.device)
    count = torch.empty(B, dtype=torch.float32, device=x.device) if mask32 is not None else None
    rk = rope.kind if rope is not None else _lib.ROPE_NONE
    nbytes = lib.pom_agg_workspace_size(dt, B, N, P, k, frame_len, rk, 0)
    ws = workspace(x.device, nbytes)   # a zero size (invalid shape) is reported by the launch
    xv = view3(x)
    if carry is not None:
        carry = carry.reshape(B, P).contiguous()
        if carry.dtype != x.dtype:
            carry = carry.to(x.dtype)
    with _Span("agg_fwd"):
        rc = lib.pom_agg_fwd(dt, dtype_code(coeff), B, N, P, k, ctypes.byref(xv), coeff.data_ptr(), ptr(mask32),
                             mask32.stride(0) if mask32 is not None else 0,
                             mask32.stride(1) if mask32 is not None else 0,
                             frame_len, ptr(carry), n_past, rope_ptr(rope), out.data_ptr(), ptr(count),
                             ws.data_ptr(), ws.numel(), stream_handle(x.device))
    check(rc, "pom_agg_fwd")
    return out, count


def agg_backward(x: torch.Tensor, coeff: torch.Tensor, k: int, frame_len: int, go32: torch.Tensor,
                 grad_x: torch.Tensor, mask32: Optional[torch.Tensor] = None,
                 count: Optional[torch.Tensor] = None, n_past: int = 0,
                 rope: Optional[RopeSpec] = None, grad_x_t: Optional[torch.Tensor] = None,
                 grad_x_rows: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Launch pom_agg_bwd; writes grad_x in place (and, when given, its
    channel-major copy grad_x_t (P, B*N); grad_x_rows is grad_x as (B*N, P))
    and returns grad_coeff (P, K) in coeff.dtype."""
    lib = _lib.load()
    B, N, P = x.shape
    dt = dtype_code(x)
    gc = torch.empty(P, k, dtype=coeff.dtype, device=x.device)
    rk = rope.kind if rope is not None else _lib.ROPE_NONE
    nbytes = lib.pom_agg_workspace_size(dt, B, N, P, k, frame_len, rk, 1)
    ws = workspace(x.device, nbytes)
    xv, gv = view3(x), view3(grad_x)
    go32 = go32.float().contiguous()
    def call(tv):
        with _Span("agg_bwd"):
            return lib.pom_agg_bwd(dt, dtype_code(coeff), B, N, P, k, ctypes.byref(xv), coeff.data_ptr(),
                                   ptr(mask32),
                                   mask32.stride(0) if mask32 is not None else 0,
                                   mask32.stride(1) if mask32 is not None else 0, ptr(count),
                                   frame_len, n_past, rope_ptr(rope), go32.data_ptr(), ctypes.byref(gv), tv,
                                   gc.data_ptr(), ws.data_ptr(), ws.numel(), stream_handle(x.device))
    _with_copy(call, grad_x_t, grad_x_rows, "transpose_dy", "pom_agg_bwd", B, N)
    return gc


def _pdt(t: Optional[torch.Tensor]) -> int:
    """pom_dtype code of an optional parameter (fp32 when absent)."""
    return 0 if t is None else dtype_code(t)


def _hagg(hagg: torch.Tensor, ys: torch.Tensor) -> torch.Tensor:
    """The gate reads the aggregate in the element type of y_s, contiguous."""
    if hagg.dtype != ys.dtype:
        hagg = hagg.to(ys.dtype)
    return hagg.contiguous()


def gate_forward(ys: torch.Tensor, bias: Optional[torch.Tensor], hagg: torch.Tensor,
                 rope: Optional[RopeSpec] = None, out: Optional[torch.Tensor] = None,
                 out_t: Optional[torch.Tensor] = None) -> torch.Tensor:
    """sh = R hardsigmoid(ys + bias) * hagg[group], via pom_gate_fwd; with
    out_t (P, B*N), also its channel-major copy."""
    lib = _lib.load()
    B, N, P = ys.shape
    hagg = _hagg(hagg, ys)
    G = hagg.shape[1]
    sh = torch.empty(B, N, P, dtype=ys.dtype, device=ys.device) if out is None else out
    yv, sv = view3(ys), view3(sh)

    def call(tv):
        with _Span("gate_fwd"):
            return lib.pom_gate_fwd(dtype_code(ys), _pdt(bias), B, N, P, ctypes.byref(yv), ptr(bias),
                                    hagg.data_ptr(), G,
                                    rope_ptr(rope), ctypes.byref(sv), tv, stream_handle(ys.device))
    _with_copy(call, out_t, sh.view(B * N, P) if out_t is not None else None, "transpose_sh", "pom_gate_fwd",
               B, N)
    return sh


def gate_backward(ys: torch.Tensor, bias: Optional[torch.Tensor], hagg: torch.Tensor,
                  grad_sh: torch.Tensor, grad_ys: torch.Tensor, rope: Optional[RopeSpec] = None,
                  want_bias: bool = True, grad_ys_t: Optional[torch.Tensor] = None,
                  grad_ys_rows: Optional[torch.Tensor] = None):
    """Writes grad_ys in place (and, when given, its channel-major copy
    grad_ys_t (P, B*N); grad_ys_rows is grad_ys as (B*N, P)); returns
    (grad_hagg (B, G, P) fp32, grad_bias (P,) in bias.dtype or None)."""
    lib = _lib.load()
    B, N, P = ys.shape
    hagg = _hagg(hagg, ys)
    G = hagg.shape[1]
    dt = dtype_code(ys)
    gh = torch.empty(B, G, P, dtype=torch.float32, device=ys.device)
    gb = torch.empty(P, dtype=bias.dtype if bias is not None else torch.float32,
                     device=ys.device) if want_bias else None
    rk = rope.kind if rope is not None else _lib.ROPE_NONE
    nbytes = lib.pom_gate_workspace_size(dt, B, N, P, G, rk)
    ws = workspace(ys.device, nbytes)
    yv, gv, dv = view3(ys), view3(grad_sh), view3(grad_ys)
    def call(tv):
        with _Span("gate_bwd"):
            return lib.pom_gate_bwd(dt, _pdt(bias if bias is not None else gb), B, N, P, ctypes.byref(yv),
                                    ptr(bias), hagg.data_ptr(), G,
                                    rope_ptr(rope), ctypes.byref(gv), ctypes.byref(dv), tv, gh.data_ptr(),
                                    ptr(gb), ws.data_ptr(), ws.numel(), stream_handle(ys.device))
    _with_copy(call, grad_ys_t, grad_ys_rows, "transpose_dy", "pom_gate_bwd", B, N)
    return gh, gb


def features_forward(x: torch.Tensor, coeff: torch.Tensor, k: int) -> torch.Tensor:
    """Per-token polynomial features poly(act(x)) (B, N, P) in x.dtype, via
    pom_features_fwd."""
    lib = _lib.load()
    B, N, P = x.shape
    out = torch.empty(B, N, P, dtype=x.dtype, device=x.device)
    xv, ov = view3(x), view3(out)
    with _Span("features_fwd"):
        rc = lib.pom_features_fwd(dtype_code(x), _pdt(coeff), B, N, P, k, ctypes.byref(xv), coeff.data_ptr(),
                                  ctypes.byref(ov), stream_handle(x.device))
    check(rc, "pom_features_fwd")
    return out


def features_backward(x: torch.Tensor, coeff: torch.Tensor, k: int, grad_out: torch.Tensor):
    """Returns (grad_x in x.dtype, grad_coeff in coeff.dtype) via pom_features_bwd."""
    lib = _lib.load()
    B, N, P = x.shape
    if grad_out.dtype != x.dtype:
        grad_out = grad_out.to(x.dtype)
    if grad_out.stride(2) != 1:
        grad_out = grad_out.contiguous()
    gx = torch.empty(B, N, P, dtype=x.dtype, device=x.device)
    gc = torch.empty(P, k, dtype=coeff.dtype, device=x.device)
    dt = dtype_code(x)
    ws = workspace(x.device, lib.pom_features_workspace_size(dt, B, N, P, k))
    xv, gv, dv = view3(x), view3(grad_out), view3(gx)
    with _Span("features_bwd"):
        rc = lib.pom_features_bwd(dt, _pdt(coeff), B, N, P, k, ctypes.byref(xv), coeff.data_ptr(),
                                  ctypes.byref(gv), ctypes.byref(dv), gc.data_ptr(), ws.data_ptr(), ws.numel(),
                                  stream_handle(x.device))
    check(rc, "pom_features_bwd")
    return gx, gc


def gate_heads_forward(ys: torch.Tensor, bias: Optional[torch.Tensor], hagg: torch.Tensor, heads: int,
                       rope: Optional[RopeSpec] = None, out_t: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-head gating (n_sel_heads = heads > 1) via pom_gate_heads_fwd:
    sh[b, n, c] = R hardsigmoid(ys + bias)[b, n, c // (P / heads)] * hagg[b, group(n), c].
    ys (B, N, heads) view; hagg (B, G, P); rope over the heads gate channels;
    with out_t (P, B*N), also the channel-major copy of sh."""
    lib = _lib.load()
    B, N, H = ys.shape
    if H != heads:
        raise ValueError(f"y_s has {H} channels, expected n_sel_heads = {heads}")
    hagg = _hagg(hagg, ys)
    G, P = hagg.shape[1], hagg.shape[2]
    sh = torch.empty(B, N, P, dtype=ys.dtype, device=ys.device)
    yv, sv = view3(ys), view3(sh)

    def call(tv):
        with _Span("gate_heads_fwd"):
            return lib.pom_gate_heads_fwd(dtype_code(ys), _pdt(bias), B, N, P, H, ctypes.byref(yv), ptr(bias),
                                          hagg.data_ptr(), G, rope_ptr(rope), ctypes.byref(sv), tv,
                                          stream_handle(ys.device))
    _with_copy(call, out_t, sh.view(B * N, P) if out_t is not None else None, "transpose_sh",
               "pom_gate_heads_fwd", B, N)
    return sh


def gate_heads_backward(ys: torch.Tensor, bias: Optional[torch.Tensor], hagg: torch.Tensor,
                        grad_sh: torch.Tensor, heads: int, rope: Optional[RopeSpec] = None,
                        want_bias: bool = True, grad_ys: Optional[torch.Tensor] = None):
    """Returns (grad_ys (B, N, heads) in ys.dtype — written into ``grad_ys``
    when given, e.g. the gate slice of dY — grad_hagg (B, G, P) fp32,
    grad_bias (heads,) in bias.dtype or None) via pom_gate_heads_bwd."""
    lib = _lib.load()
    B, N, H = ys.shape
    hagg = _hagg(hagg, ys)
    G, P = hagg.shape[1], hagg.shape[2]
    if grad_sh.dtype != ys.dtype:
        grad_sh = grad_sh.to(ys.dtype)
    if grad_sh.stride(2) != 1:
        grad_sh = grad_sh.contiguous()
    dt = dtype_code(ys)
    gys = torch.empty(B, N, H, dtype=ys.dtype, device=ys.device) if grad_ys is None else grad_ys
    gh = torch.empty(B, G, P, dtype=torch.float32, device=ys.device)
    gb = torch.empty(H, dtype=bias.dtype if bias is not None else torch.float32,
                     device=ys.device) if want_bias else None
    ws = workspace(ys.device, lib.pom_gate_heads_workspace_size(dt, B, N, P, H, G))
    yv, gv, dv = view3(ys), view3(grad_sh), view3(gys)
    with _Span("gate_heads_bwd"):
        rc = lib.pom_gate_heads_bwd(dt, _pdt(bias if bias is not None else gb), B, N, P, H, ctypes.byref(yv),
                                    ptr(bias), hagg.data_ptr(), G, rope_ptr(rope), ctypes.byref(gv),
                                    ctypes.byref(dv), gh.data_ptr(), ptr(gb), ws.data_ptr(), ws.numel(),
                                    stream_handle(ys.device))
    check(rc, "pom_gate_heads_bwd")
    return gys, gh, gb


# ---------------------------------------------------------------------------
# Kernel-level autograd operators (drop-ins for the Triton entry points)
# ---------------------------------------------------------------------------

class _PolyAgg(torch.autograd.Function):
    """Aggregation with every mode of pom_agg_fwd / pom_agg_bwd."""

    @staticmethod
    def forward(ctx, x, coeff, k, frame_len, mask32, rope, carry, n_past):
        _lib.require_device(x)
        B, N, P = x.shape
        c32 = _coeff_param(coeff, P, k)
        out, count = agg_forward(x, c32, k, frame_len, mask32, carry, n_past, rope)
        ctx.save_for_backward(x, c32, mask32, count)
        ctx.k, ctx.frame_len, ctx.rope, ctx.n_past = k, frame_len, rope, n_past
        ctx.coeff_dtype = coeff.dtype
        ctx.has_carry = carry is not None
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, c32, mask32, count = ctx.saved_tensors
        go32 = grad_out.float().contiguous()
        gx = torch.empty_like(x, memory_format=torch.contiguous_format)
        gc = agg_backward(x, c32, ctx.k, ctx.frame_len, go32, gx, mask32, count, ctx.n_past, ctx.rope)
        g_carry = None
        if ctx.has_carry and ctx.needs_input_grad[6]:
            nf = go32.shape[1]
            w = ctx.n_past / (ctx.n_past + torch.arange(nf, device=x.device, dtype=torch.float32) + 1.0)
            g_carry = (go32 * w.view(1, nf, 1)).sum(dim=1, keepdim=True).to(x.dtype)
        return gx, gc.to(ctx.coeff_dtype), None, None, None, None, g_carry, None


def _mask32(mask: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    B, N, _ = x.shape
    if mask.shape != (B, N):
        raise ValueError(f"mask must have shape ({B}, {N}), got {tuple(mask.shape)}")
    return mask.to(device=x.device, dtype=torch.float32).contiguous()


class _Features(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, coeff, k):
        _lib.require_device(x)
        c = _coeff_param(coeff, x.shape[2], k)
        ctx.save_for_backward(x, c)
        ctx.k, ctx.coeff_dtype = k, coeff.dtype
        return features_forward(x, c, k)

    @staticmethod
    def backward(ctx, grad_out):
        x, c = ctx.saved_tensors
        gx, gc = features_backward(x, c, ctx.k, grad_out)
        return gx, gc.to(ctx.coeff_dtype), None


def poly_features_hip(x: torch.Tensor, coeff: torch.Tensor, k: int) -> torch.Tensor:
    """(B, N, P) -> (B, N, P) per-token p(act(x)) — pom/pom.py:83-88 — on the
    HIP kernels (the dense-mask route's operand)."""
    _check_degree(k)
    return _Features.apply(x, coeff, k)


def poly_agg_mean_hip(x: torch.Tensor, coeff: torch.Tensor, k: int) -> torch.Tensor:
    """(B, N, D) -> (B, 1, D) mean of p(act(x)) in x.dtype."""
    _check_degree(k)
    return _PolyAgg.apply(x, coeff, k, x.shape[1], None, None, None, 0)


def poly_agg_masked_hip(x: torch.Tensor, mask: torch.Tensor, coeff: torch.Tensor, k: int,
                        rope: Optional[RopeSpec] = None) -> torch.Tensor:
    """(B, N, D), (B, N) weights -> (B, 1, D) weighted mean (all-zero row -> 0);
    with rope, of the rotated features (pom/pom_rope.py:511-515)."""
    _check_degree(k)
    return _PolyAgg.apply(x, coeff, k, x.shape[1], _mask32(mask, x), rope, None, 0)


def poly_agg_block_causal_hip(x: torch.Tensor, coeff: torch.Tensor, k: int, frame_len: int) -> torch.Tensor:
    """(B, N, D) -> (B, N/frame_len, D): row f = mean over frames 0..f."""
    _check_degree(k)
    if frame_len <= 0 or x.shape[1] % frame_len:
        raise ValueError(f"frame_len {frame_len} must divide the sequence length {x.shape[1]}")
    return _PolyAgg.apply(x, coeff, k, frame_len, None, None, None, 0)


def poly_agg_causal_hip(x: torch.Tensor, coeff: torch.Tensor, k: int) -> torch.Tensor:
    """(B, N, D) -> (B, N, D) token-causal prefix mean."""
    _check_degree(k)
    return _PolyAgg.apply(x, coeff, k, 1, None, None, None, 0)


def _rope1d(x: torch.Tensor, freqs_cos, freqs_sin, positions) -> RopeSpec:
    B, N, D = x.shape
    if D % 2 != 0:
        raise ValueError(f"D must be even for RoPE (got {D})")
    n_max = None
    if positions is None:
        positions, n_max = torch.arange(N, device=x.device, dtype=torch.int64), N
    if freqs_cos.shape[1] < D // 2:
        raise ValueError("RoPE tables are narrower than D/2")
    return RopeSpec(_lib.ROPE_1D, [freqs_cos, freqs_sin], positions, x.device, n_max)


def poly_agg_rope_mean_hip(x, coeff, k, freqs_cos, freqs_sin, positions=None):
    """Fused act + poly + 1-D RoPE + mean: (B, N, D) -> (B, 1, D)."""
    _check_degree(k)
    return _PolyAgg.apply(x, coeff, k, x.shape[1], None, _rope1d(x, freqs_cos, freqs_sin, positions), None, 0)


def poly_agg_rope_causal_hip(x, coeff, k, freqs_cos, freqs_sin, positions=None):
    """Fused act + poly + 1-D RoPE + causal prefix mean: (B, N, D) -> (B, N, D)."""
    _check_degree(k)
    return _PolyAgg.apply(x, coeff, k, 1, None, _rope1d(x, freqs_cos, freqs_sin, positions), None, 0)


def poly_agg_rope_hip(x, coeff, k, rope: RopeSpec, frame_len: Optional[int] = None):
    """Aggregation of rotated features for an arbitrary RopeSpec (1-D or 2-D)."""
    _check_degree(k)
    return _PolyAgg.apply(x, coeff, k, x.shape[1] if frame_len is None else frame_len, None, rope, None, 0)


def poly_agg_state_hip(x, coeff, k, carry: Optional[torch.Tensor], n_past: int) -> torch.Tensor:
    """One PoM.state_forward aggregation step: (n_past*carry + mean)/(n_past+1)."""
    _check_degree(k)
    return _PolyAgg.apply(x, coeff, k, x.shape[1], None, None, carry, n_past if carry is not None else 0)


class _Gate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ys, bias, hagg, rope):
        _lib.require_device(ys, hagg)
        B, N, P = ys.shape
        b32 = None if bias is None else _param(bias)
        h = _hagg(hagg.detach(), ys)
        sh = gate_forward(ys, b32, h, rope)
        ctx.save_for_backward(ys, b32, h)
        ctx.rope = rope
        ctx.bias_dtype = None if bias is None else bias.dtype
        ctx.hagg_dtype = hagg.dtype
        return sh

    @staticmethod
    def backward(ctx, grad_sh):
        ys, b32, h = ctx.saved_tensors
        gys = torch.empty_like(ys, memory_format=torch.contiguous_format)
        gh, gb = gate_backward(ys, b32, h, grad_sh, gys, ctx.rope, want_bias=b32 is not None)
        return (gys, None if gb is None else gb.to(ctx.bias_dtype), gh.to(ctx.hagg_dtype), None)


def gate_hip(ys: torch.Tensor, bias: Optional[torch.Tensor], hagg: torch.Tensor,
             rope: Optional[RopeSpec] = None) -> torch.Tensor:
    """R(pos) hardsigmoid(ys + bias) * hagg, hagg (B, G, P) broadcast over N/G tokens per group."""
    return _Gate.apply(ys, bias, hagg, rope)


class _GateHeads(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ys, bias, hagg, heads, rope):
        _lib.require_device(ys, hagg)
        b32 = None if bias is None else _param(bias)
        h = _hagg(hagg.detach(), ys)
        sh = gate_heads_forward(ys, b32, h, heads, rope)
        ctx.save_for_backward(ys, b32, h)
        ctx.heads, ctx.rope = heads, rope
        ctx.bias_dtype = None if bias is None else bias.dtype
        ctx.hagg_dtype = hagg.dtype
        return sh

    @staticmethod
    def backward(ctx, grad_sh):
        ys, b32, h = ctx.saved_tensors
        gys, gh, gb = gate_heads_backward(ys, b32, h, grad_sh, ctx.heads, ctx.rope, want_bias=b32 is not None)
        return (gys, None if gb is None else gb.to(ctx.bias_dtype), gh.to(ctx.hagg_dtype), None, None)


def gate_heads_hip(ys: torch.Tensor, bias: Optional[torch.Tensor], hagg: torch.Tensor, heads: int,
                   rope: Optional[RopeSpec] = None) -> torch.Tensor:
    """Per-head gate (n_sel_heads = heads > 1): R(pos) hardsigmoid(ys + bias), one
    scalar per head and token, times hagg (B, G, P) broadcast over N/G tokens
    per group — pom/pom.py:118-122 with :207 (and pom/pom_rope.py:417-437)."""
    return _GateHeads.apply(ys, bias, hagg, heads, rope)


# ---------------------------------------------------------------------------
# Fused PoM layer: qc_proj GEMM -> aggregation -> gating -> ag_proj GEMM
# ---------------------------------------------------------------------------

# The layer's launch sequence in C++ (pom_layer_fwd / pom_layer_bwd: one C
# call per direction, library GEMMs with the tuned table's solutions) for bf16
# with the default GEMM options; POM_AMD_NATIVE_LAYER=0 keeps the Python one.
# A shape the C path does not cover (no registered GEMM solution) falls back
# to the Python sequence before anything is launched.
_NATIVE_LAYER = os.environ.get("POM_AMD_NATIVE_LAYER", "1") != "0"
native_layer_calls = [0, 0]   # forward, backward calls that took the C sequence


def _native_layer_usable(dt: torch.dtype, c32: torch.Tensor, b32: torch.Tensor) -> bool:
    return (_NATIVE_LAYER and dt == torch.bfloat16 and _NT_GEMMS and _NT_COPIES == "fused" and not _OVERLAP_GEMMS
            and not _SIDE_WGRAD and _HIP_GEMMS == frozenset(("gemm_ag_wgrad", "gemm_qc_wgrad"))
            and c32.dtype == b32.dtype and gemm_select.native_ready())


def _pom_gemm_fits(M: int, N: int, T: int) -> bool:
    """A weight gradient (M x N over T tokens, token-major operands) that pom_gemm takes."""
    t, s = ctypes.c_int(-1), ctypes.c_int(0)
    return _lib.load().pom_gemm_plan(M, N, T, 1, 1, ctypes.byref(t), ctypes.byref(s)) == 0


def _layer_args(B, N, D, P, S, W, heads, k, frame_len, n_past, c32, b32, keep) -> "_lib.PomLayerArgs":
    a = _lib.PomLayerArgs()
    a.B, a.N, a.D, a.P, a.S, a.W, a.heads, a.K = B, N, D, P, S, W, heads, k
    a.param_dtype = dtype_code(c32)
    a.frame_len, a.n_past = frame_len, n_past
    a.coeff, a.se_bias = c32.data_ptr(), b32.data_ptr()
    keep.extend((c32, b32))
    return a


def _set_rope(a, rope_h, rope_s, keep) -> None:
    for name, spec in (("rope_h", rope_h), ("rope_s", rope_s)):
        if spec is not None:
            r = spec.struct()
            keep.append(r)
            setattr(a, name, ctypes.pointer(r))


def _native_layer_forward(x2, wq, wa, b_ag, b32, c32, k, frame_len, mask, carry, n_past, rope_h, rope_s, heads,
                          B, N, D, P, S, W, want_xt, want_sht):
    """One pom_layer_fwd call; None when the C path does not cover the shapes
    (nothing launched)."""
    lib = _lib.load()
    dev, dt, T = x2.device, x2.dtype, B * N
    keep = []
    a = _layer_args(B, N, D, P, S, W, heads, k, frame_len, n_past, c32, b32, keep)
    y = torch.empty(T, W, dtype=dt, device=dev)
    hagg = torch.empty(B, N // frame_len, P, dtype=dt, device=dev)
    count = torch.empty(B, dtype=torch.float32, device=dev) if mask is not None else None
    sh = torch.empty(T, P, dtype=dt, device=dev)
    out = torch.empty(T, D, dtype=dt, device=dev)
    xt = torch.empty(D, T, dtype=dt, device=dev) if want_xt else None
    sht = torch.empty(P, T, dtype=dt, device=dev) if want_sht else None
    a.wq, a.wa, a.x, a.y, a.hagg, a.sh, a.out = (wq.data_ptr(), wa.data_ptr(), x2.data_ptr(), y.data_ptr(),
                                                 hagg.data_ptr(), sh.data_ptr(), out.data_ptr())
    a.xt, a.sht, a.count = ptr(xt), ptr(sht), ptr(count)
    if b_ag is not None:
        a.b_ag, a.bias_ag_dtype = b_ag.data_ptr(), dtype_code(b_ag)
        keep.append(b_ag)
    if mask is not None:
        a.mask, a.mask_stride_b, a.mask_stride_n = mask.data_ptr(), mask.stride(0), mask.stride(1)
    if carry is not None:
        carry = carry.reshape(B, P).to(dt).contiguous()
        a.carry = carry.data_ptr()
        keep.append(carry)
    _set_rope(a, rope_h, rope_s, keep)
    ws = workspace(dev, lib.pom_layer_workspace_size(ctypes.byref(a), 0))
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    with _Span("layer_fwd"):
        rc = lib.pom_layer_fwd(ctypes.byref(a), stream_handle(dev))
    if rc == _lib.POM_ERR_UNSUPPORTED:
        return None
    check(rc, "pom_layer_fwd")
    native_layer_calls[0] += 1
    return y, hagg, count, sh, out, xt, sht


def _native_layer_backward(ctx, grad_out, grad_hagg):
    x, xt, y, sh, sht, hagg, c32, b32, wq, wa, mask, count = ctx.saved_tensors
    k, frame_len, rope_h, rope_s, n_past, has_carry, has_bias, heads = ctx.meta
    B, N, D = ctx.shape
    dev, dt = y.device, y.dtype
    P = c32.shape[0]
    S = heads if heads > 1 else P
    W = _padded_width(P, S)
    T = B * N
    need_x, need_wq, need_wa = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[4]
    tq, tb, tc, ta, tab = ctx.dtypes
    if grad_out is None:
        grad_out = torch.zeros(B, N, D, dtype=dt, device=dev)
    g2 = grad_out.reshape(T, D)
    if g2.dtype != dt:
        g2 = g2.to(dt)
    if not g2.is_contiguous():
        g2 = g2.contiguous()
    lib = _lib.load()
    keep = [g2]
    a = _layer_args(B, N, D, P, S, W, heads, k, frame_len, n_past, c32, b32, keep)
    G = N // frame_len
    wq_fits, wa_fits = _pom_gemm_fits(W, D, T), _pom_gemm_fits(D, P, T)
    dsh = torch.empty(T, P, dtype=dt, device=dev)
    dy = torch.empty(T, W, dtype=dt, device=dev)
    gt = torch.empty(D, T, dtype=dt, device=dev) if need_wa and not wa_fits else None
    dyt = torch.empty(W, T, dtype=dt, device=dev) if need_wq and not wq_fits else None
    dx = torch.empty(T, D, dtype=dt, device=dev) if need_x else None
    dwq = torch.empty(W, D, dtype=_wgrad_dtype(tq) if wq_fits else dt, device=dev) if need_wq else None
    dwa = torch.empty(D, P, dtype=_wgrad_dtype(ta) if wa_fits else dt, device=dev) if need_wa else None
    dbias = torch.empty(S, dtype=b32.dtype, device=dev)
    dcoeff = torch.empty(P, k, dtype=c32.dtype, device=dev)
    db_ag = torch.empty(D, dtype=torch.float32, device=dev) if has_bias else None
    dh = torch.empty(B, G, P, dtype=torch.float32, device=dev)
    gh = grad_hagg.float().contiguous() if grad_hagg is not None else None
    wq_t = _weight_t(wq) if need_x else None
    wa_t = _weight_t(wa)
    keep.extend((wq_t, wa_t, gh))
    a.wq, a.wq_t, a.wa, a.wa_t = wq.data_ptr(), ptr(wq_t), wa.data_ptr(), wa_t.data_ptr()
    a.x, a.xt, a.y, a.hagg, a.count, a.sh, a.sht = (ptr(x), ptr(xt), y.data_ptr(), hagg.data_ptr(), ptr(count),
                                                    sh.data_ptr(), ptr(sht))
    if mask is not None:
        a.mask, a.mask_stride_b, a.mask_stride_n = mask.data_ptr(), mask.stride(0), mask.stride(1)
    _set_rope(a, rope_h, rope_s, keep)
    a.g, a.gt, a.dsh, a.dy, a.dyt, a.dx = g2.data_ptr(), ptr(gt), dsh.data_ptr(), dy.data_ptr(), ptr(dyt), ptr(dx)
    if dwq is not None:
        a.dwq, a.dwq_dtype = dwq.data_ptr(), dtype_code(dwq)
    if dwa is not None:
        a.dwa, a.dwa_dtype = dwa.data_ptr(), dtype_code(dwa)
    a.dse_bias, a.dcoeff, a.db_ag, a.dh, a.grad_hagg = (dbias.data_ptr(), dcoeff.data_ptr(), ptr(db_ag),
                                                        dh.data_ptr(), ptr(gh))
    ws = workspace(dev, lib.pom_layer_workspace_size(ctypes.byref(a), 1))
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    with _Span("layer_bwd"):
        check(lib.pom_layer_bwd(ctypes.byref(a), stream_handle(dev)), "pom_layer_bwd")
    native_layer_calls[1] += 1
    g_carry = None
    if has_carry:
        w = n_past / (n_past + torch.arange(G, device=dev, dtype=torch.float32) + 1.0)
        g_carry = (dh * w.view(1, G, 1)).sum(dim=1, keepdim=True).to(dt)
    if dwq is not None and dwq.shape[0] != P + S:
        dwq = dwq[:P + S]   # the padding rows' gradient is not a parameter's
    return (None if dx is None else dx.view(B, N, D), None if dwq is None else dwq.to(tq),
            dbias.to(tb), dcoeff.to(tc), None if dwa is None else dwa.to(ta),
            None if db_ag is None else db_ag.to(tab), None, None, None, None, None, g_carry, None, None, None)


class _PoMLayer(torch.autograd.Function):
    """Self-mixing PoM layer (n_groups == 1) — pom/pom.py:216-231 composed with
    _get_h_s (:204-207), pom() (:125-135) and, for RoPE, pom/pom_rope.py:476-526.

    Memory plan (T = B*N tokens, S = P gate channels, or H = n_sel_heads):
      forward : Y = x W_qc^T (T, P+S) -> hagg (B, G, P) -> sh (T, P) -> out (T, D)
      backward: dsh = g W_ag (T, P); dY (T, P+S) is filled in two parts by the
                gate (s-part) and aggregation (h-part) kernels, then
                dx = dY W_qc and dW_qc = dY^T x.
    In 16-bit training (_NT_GEMMS) the weight gradients are dW_ag = g^T sh
    and dW_qc = dY^T x on token-contiguous copies (gt, sht, dyt, xt) and the
    data gradients use transposed weights, so every backward GEMM has both
    operands contiguous in K.  The copies of inputs (x, g) are made on a
    second stream while the current one runs the GEMM that does not need
    them; sh^T and dY^T likewise ("side") or inside the producing kernels
    ("fused").
    Saved: Y, hagg, the fp32 coefficient/bias copies, and x, sh (or x^T, sh^T).
    Returns (out, hagg) — hagg in x.dtype, differentiable (state_forward's carry).
    """

    @staticmethod
    def forward(ctx, x, w_qc, se_bias, coeff, w_ag, b_ag, k, frame_len, mask, rope_h, rope_s, carry, n_past,
                training, heads):
        _lib.require_device(x)
        B, N, D = x.shape
        P = coeff.shape[0]
        S = heads if heads > 1 else P
        W = _padded_width(P, S)   # Y's row width (zero columns past P + S)
        T = B * N
        dt = x.dtype
        dev = x.device
        x2 = x.reshape(T, D)
        nt = training and _NT_GEMMS and dt != torch.float32
        # weight gradients on pom_gemm read x and sh in place; hipBLASLt gets token-contiguous copies
        hip_wq = training and ctx.needs_input_grad[1] and hip_gemm_fits("gemm_qc_wgrad", W, D, T, dt)
        hip_wa = training and ctx.needs_input_grad[4] and hip_gemm_fits("gemm_ag_wgrad", D, P, T, dt)
        want_xt = nt and ctx.needs_input_grad[1] and not hip_wq
        want_sht = nt and ctx.needs_input_grad[4] and not hip_wa
        wq = _qc_weight(w_qc, dt, W)                                # (W, D), zero rows past P + S
        c32 = _coeff_param(coeff, P, k)
        b32 = _param(se_bias)
        wa = w_ag if w_ag.dtype == dt else w_ag.to(dt)
        res = None
        if _native_layer_usable(dt, c32, b32):
            need_q = training and ctx.needs_input_grad[1]
            need_a = training and ctx.needs_input_grad[4]
            res = _native_layer_forward(x2, wq, wa, b_ag, b32, c32, k, frame_len, mask, carry, n_past, rope_h,
                                        rope_s, heads, B, N, D, P, S, W,
                                        need_q and not _pom_gemm_fits(W, D, T),
                                        need_a and not _pom_gemm_fits(D, P, T))
        if res is not None:
            y, hagg, count, sh, out, xt, sht = res
            ctx.native = True
            ctx.save_for_backward(x, xt, y, sh, sht, hagg, c32, b32, wq, wa, mask, count)
            ctx.shape = (B, N, D)
            ctx.set_materialize_grads(False)
            ctx.meta = (k, frame_len, rope_h, rope_s, n_past, carry is not None, b_ag is not None, heads)
            ctx.dtypes = (w_qc.dtype, se_bias.dtype, coeff.dtype, w_ag.dtype,
                          None if b_ag is None else b_ag.dtype)
            return out.view(B, N, D), hagg
        ctx.native = False
        cur = torch.cuda.current_stream(dev)
        side = _copy_stream(dev) if (want_xt or want_sht) else None
        xt = sht = None
        if want_xt:
            side.wait_stream(cur)
            with torch.cuda.stream(side):
                xt = transpose(x2, "transpose_x")                  # (D, T), overlaps qc_fwd
        with _Span("gemm_qc_fwd"), tuned_gemms():
            y = torch.mm(x2, wq.t())                                # (T, W)
        y3 = y.view(B, N, W)
        h_view, s_view = y3[..., :P], y3[..., P:P + S]
        hagg, count = agg_forward(h_view, c32, k, frame_len, mask, carry, n_past, rope_h)
        fused = want_sht and _NT_COPIES == "fused"
        if fused:
            sht = torch.empty(P, T, dtype=dt, device=dev)
        if heads > 1:
            sh = gate_heads_forward(s_view, b32, hagg, heads, rope_s, out_t=sht if fused else None)   # (B, N, P)
        else:
            sh = gate_forward(s_view, b32, hagg, rope_s, out_t=sht if fused else None)   # (B, N, P)
        if want_sht and not fused:
            side.wait_stream(cur)
            with torch.cuda.stream(side):
                sht = transpose(sh.view(T, P), "transpose_sh")      # (P, T), overlaps ag_fwd
        with _Span("gemm_ag_fwd"), tuned_gemms():
            out = torch.mm(sh.view(T, P), wa.t())
        if b_ag is not None:
            out = out + b_ag.to(dt)
        if side is not None:
            # join before x or sh can be freed; the copies live on the current stream
            cur.wait_stream(side)
            if xt is not None:
                xt.record_stream(cur)
            if sht is not None and not fused:
                sht.record_stream(cur)
        ctx.nt = nt
        ctx.hip_w = (hip_wq, hip_wa)
        ctx.save_for_backward(None if want_xt else x, xt, y, None if want_sht else sh, sht,
                              hagg, c32, b32, wq, wa, mask, count)
        ctx.shape = (B, N, D)
        ctx.set_materialize_grads(False)   # the aggregate output is usually unused
        ctx.meta = (k, frame_len, rope_h, rope_s, n_past, carry is not None, b_ag is not None, heads)
        ctx.dtypes = (w_qc.dtype, se_bias.dtype, coeff.dtype, w_ag.dtype,
                      None if b_ag is None else b_ag.dtype)
        return out.view(B, N, D), hagg

    @staticmethod
    def backward(ctx, grad_out, grad_hagg):
        if ctx.native:
            return _native_layer_backward(ctx, grad_out, grad_hagg)
        x, xt, y, sh, sht, hagg, c32, b32, wq, wa, mask, count = ctx.saved_tensors
        k, frame_len, rope_h, rope_s, n_past, has_carry, has_bias, heads = ctx.meta
        B, N, D = ctx.shape
        dev = y.device
        dt = y.dtype
        if grad_out is None:   # only the aggregate was used downstream
            grad_out = torch.zeros(B, N, D, dtype=dt, device=dev)
        P = c32.shape[0]
        S = heads if heads > 1 else P
        W = _padded_width(P, S)
        T = B * N
        need_x, need_wq, need_wa = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[4]
        nt_a = xt is not None or sht is not None   # token-contiguous weight gradients
        nt = ctx.nt
        g2 = grad_out.reshape(T, D)
        if g2.dtype != dt:
            g2 = g2.to(dt)
        if nt and not g2.is_contiguous():
            g2 = g2.contiguous()
        cur = torch.cuda.current_stream(dev)
        side = _copy_stream(dev) if nt_a else None
        gt = None
        if need_wa and sht is not None:
            side.wait_stream(cur)
            with torch.cuda.stream(side):
                gt = transpose(g2, "transpose_g")                  # (D, T), overlaps ag_dgrad
        wa_k = _weight_t(wa).t() if nt else wa                      # (D, P), K-contiguous when nt
        with _Span("gemm_ag_dgrad"), tuned_gemms():
            dsh = torch.mm(g2, wa_k)                                # (T, P)
        dw_ag = None
        over = _OVERLAP_GEMMS and side is not None
        hip_wq, hip_wa = ctx.hip_w
        tq, tb, tc, ta, tab = ctx.dtypes
        side_wa = None
        if need_wa and hip_wa:
            if not g2.is_contiguous():
                g2 = g2.contiguous()
            if _SIDE_WGRAD and _COPY_STREAM:
                side_wa = _copy_stream(dev)
                side_wa.wait_stream(cur)
                with torch.cuda.stream(side_wa):
                    dw_ag = hip_gemm(g2, True, sh.view(T, P), True, _wgrad_dtype(ta), "gemm_ag_wgrad")   # (D, P)
            else:
                dw_ag = hip_gemm(g2, True, sh.view(T, P), True, _wgrad_dtype(ta), "gemm_ag_wgrad")   # (D, P)
        elif need_wa:
            if gt is not None and over:
                with torch.cuda.stream(side), _Span("gemm_ag_wgrad"), tuned_gemms():
                    dw_ag = torch.mm(gt, sht.t())                   # (D, P), on the second stream
                del gt
            elif gt is not None:
                cur.wait_stream(side)
                gt.record_stream(cur)
                with _Span("gemm_ag_wgrad"), tuned_gemms():
                    dw_ag = torch.mm(gt, sht.t())                   # (D, P)
                del gt
            else:
                with _Span("gemm_ag_wgrad"), tuned_gemms():
                    dw_ag = torch.mm(g2.t(), sh.view(T, P))         # (D, P)
        db_ag = g2.float().sum(0) if has_bias else None
        y3 = y.view(B, N, W)
        dy = torch.empty(T, W, dtype=dt, device=dev)
        dy3 = dy.view(B, N, W)
        if W > P + S:
            dy[:, P + S:].zero_()   # the padding columns meet W_qc's zero rows in dx = dY W_qc
        want_dyt = need_wq and xt is not None
        fused = want_dyt and _NT_COPIES == "fused"
        dyt = torch.empty(W, T, dtype=dt, device=dev) if fused else None
        if heads > 1:
            _, dh, dbias = gate_heads_backward(y3[..., P:P + S], b32, hagg, dsh.view(B, N, P), heads, rope_s,
                                               grad_ys=dy3[..., P:P + S])
            if dyt is not None:   # the gate part of dY^T (with the padding rows) from the transpose kernel
                _transpose_into(dy[:, P:], dyt[P:], "transpose_dy")
        else:
            dh, dbias = gate_backward(y3[..., P:P + S], b32, hagg, dsh.view(B, N, P), dy3[..., P:P + S], rope_s,
                                      grad_ys_t=None if dyt is None else dyt[P:P + S],
                                      grad_ys_rows=dy[:, P:P + S])
        if grad_hagg is not None:
            dh = dh + grad_hagg.float()
        dcoeff = agg_backward(y3[..., :P], c32, k, frame_len, dh, dy3[..., :P], mask, count, n_past, rope_h,
                              grad_x_t=None if dyt is None else dyt[:P], grad_x_rows=dy[:, :P])
        if want_dyt and not fused:
            side.wait_stream(cur)
            with torch.cuda.stream(side):
                dyt = transpose(dy, "transpose_dy")                # (P+S, T), overlaps qc_dgrad
        dw_qc = None
        if need_wq and want_dyt and over:
            side.wait_stream(cur)                                   # dY^T is complete
            with torch.cuda.stream(side), _Span("gemm_qc_wgrad"), tuned_gemms():
                dw_qc = torch.mm(dyt, xt.t())                       # (P+S, D), on the second stream
        dx = None
        if need_x:
            wq_k = _weight_t(wq).t() if nt else wq                  # (P+S, D), K-contiguous when nt
            with _Span("gemm_qc_dgrad"), tuned_gemms():
                dx = torch.mm(dy, wq_k)                             # (T, D)
        if need_wq and dw_qc is None and hip_wq:
            dw_qc = hip_gemm(dy, True, x.reshape(T, D), True, _wgrad_dtype(tq), "gemm_qc_wgrad")   # (W, D)
        elif need_wq and dw_qc is None:
            if want_dyt:
                if not fused:
                    cur.wait_stream(side)
                    dyt.record_stream(cur)
                with _Span("gemm_qc_wgrad"), tuned_gemms():
                    dw_qc = torch.mm(dyt, xt.t())                   # (P+S, D)
            else:
                with _Span("gemm_qc_wgrad"), tuned_gemms():
                    dw_qc = torch.mm(dy.t(), x.reshape(T, D))       # (P+S, D)
        if side_wa is not None:
            cur.wait_stream(side_wa)   # join before g2 or sh can be freed
            dw_ag.record_stream(cur)
        if side is not None:
            cur.wait_stream(side)   # join before g2 or dy can be freed
            if over:
                for t in (dw_ag, dw_qc):
                    if t is not None:
                        t.record_stream(cur)
        g_carry = None
        if has_carry:
            nf = dh.shape[1]
            w = n_past / (n_past + torch.arange(nf, device=dev, dtype=torch.float32) + 1.0)
            g_carry = (dh * w.view(1, nf, 1)).sum(dim=1, keepdim=True).to(dt)
        if dw_qc is not None and dw_qc.shape[0] != P + S:
            dw_qc = dw_qc[:P + S]   # the padding rows' gradient is not a parameter's
        return (None if dx is None else dx.view(B, N, D), None if dw_qc is None else dw_qc.to(tq),
                dbias.to(tb), dcoeff.to(tc), None if dw_ag is None else dw_ag.to(ta),
                None if db_ag is None else db_ag.to(tab), None, None, None, None, None, g_carry, None, None, None)


def pom_layer(x, w_qc, se_bias, coeff, w_ag, b_ag, k: int, frame_len: Optional[int] = None,
              mask: Optional[torch.Tensor] = None, rope_h: Optional[RopeSpec] = None,
              rope_s: Optional[RopeSpec] = None, carry: Optional[torch.Tensor] = None,
              n_past: int = 0, heads: int = 1) -> Tuple[torch.Tensor, torch.Tensor]:
    """Run the fused layer; returns (out (B, N, D), hagg (B, G, P)).  heads > 1:
    per-head gating (n_sel_heads), w_qc (P + heads, D), rope_s over the heads."""
    _check_degree(k)
    if not x.is_contiguous():
        x = x.contiguous()
    B, N, _ = x.shape
    frame_len = N if frame_len is None else frame_len
    if frame_len <= 0 or N % frame_len:
        raise ValueError(f"frame_len {frame_len} must divide the sequence length {N}")
    m32 = None if mask is None else _mask32(mask, x)
    return _PoMLayer.apply(x, w_qc, se_bias, coeff, w_ag, b_ag, k, frame_len, m32, rope_h, rope_s,
                           carry, n_past if carry is not None else 0, torch.is_grad_enabled(), heads)
