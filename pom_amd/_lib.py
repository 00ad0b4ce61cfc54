"""ctypes binding of libpom_amd.so, the C ABI declared in include/pom_amd.h.

The shared library is built in-tree (``python pom_amd/csrc/build.py``) and
loaded lazily on first use.  There is no fallback: if the library is missing
or fails to load, every entry point raises.  torch is imported first so that
the library binds to the HIP runtime torch already loaded.
"""
from __future__ import annotations

import ctypes
import os
import threading
import weakref
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("POM_AMD_LIB", os.path.join(_HERE, "libpom_amd.so"))

POM_OK = 0
POM_ERR_INVALID = 1
POM_ERR_UNSUPPORTED = 2
POM_ERR_WORKSPACE = 3
POM_ERR_DEVICE = 4

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
ROPE_NONE, ROPE_1D, ROPE_2D = 0, 1, 2
MAX_DEGREE = 16
ABI_VERSION = 10
NOALLOC_SCRATCH_BYTES = 16 << 20

# Every symbol include/pom_amd.h declares, with its ctypes signature.
_c_i64 = ctypes.c_int64
_c_vp = ctypes.c_void_p
_c_int = ctypes.c_int
_c_size = ctypes.c_size_t


class PomView(ctypes.Structure):
    _fields_ = [("data", _c_vp), ("stride_b", _c_i64), ("stride_n", _c_i64)]


class PomRope(ctypes.Structure):
    _fields_ = [("kind", _c_int), ("cos0", _c_vp), ("sin0", _c_vp), ("cos1", _c_vp), ("sin1", _c_vp),
                ("table_stride", _c_i64), ("rows0", _c_i64), ("rows1", _c_i64), ("pos", _c_vp),
                ("pos_stride", _c_i64)]


class PomTView(ctypes.Structure):
    _fields_ = [("data", _c_vp), ("stride_c", _c_i64), ("stride_b", _c_i64)]


class PomLayerArgs(ctypes.Structure):
    """pom_layer_args (include/pom_amd.h), field for field; load() checks its size."""
    _fields_ = [("B", _c_i64), ("N", _c_i64), ("D", _c_i64), ("P", _c_i64), ("S", _c_i64), ("W", _c_i64),
                ("heads", _c_i64), ("K", _c_int), ("param_dtype", _c_int), ("bias_ag_dtype", _c_int),
                ("frame_len", _c_i64), ("n_past", _c_i64),
                ("wq", _c_vp), ("wq_t", _c_vp), ("wa", _c_vp), ("wa_t", _c_vp), ("se_bias", _c_vp), ("coeff", _c_vp),
                ("b_ag", _c_vp), ("mask", _c_vp), ("mask_stride_b", _c_i64), ("mask_stride_n", _c_i64),
                ("carry", _c_vp), ("rope_h", ctypes.POINTER(PomRope)), ("rope_s", ctypes.POINTER(PomRope)),
                ("x", _c_vp), ("xt", _c_vp), ("y", _c_vp), ("hagg", _c_vp), ("count", _c_vp), ("sh", _c_vp),
                ("sht", _c_vp), ("out", _c_vp),
                ("g", _c_vp), ("gt", _c_vp), ("dsh", _c_vp), ("dy", _c_vp), ("dyt", _c_vp), ("dx", _c_vp),
                ("dwq", _c_vp), ("dwq_dtype", _c_int), ("dwa", _c_vp), ("dwa_dtype", _c_int),
                ("dse_bias", _c_vp), ("dcoeff", _c_vp), ("db_ag", _c_vp), ("dh", _c_vp), ("grad_hagg", _c_vp),
                ("workspace", _c_vp), ("workspace_bytes", _c_size)]


_PV = ctypes.POINTER(PomView)
_PR = ctypes.POINTER(PomRope)
_PT = ctypes.POINTER(PomTView)

SIGNATURES = {
    "pom_abi_version": (_c_int, []),
    "pom_last_error": (ctypes.c_char_p, []),
    "pom_agg_workspace_size": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_i64, _c_int, _c_int]),
    "pom_agg_fwd": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _PV, _c_vp, _c_vp, _c_i64, _c_i64,
                             _c_i64, _c_vp, _c_i64, _PR, _c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
    "pom_agg_fwd_noalloc": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _PV, _c_vp, _c_vp, _c_i64,
                                     _c_i64, _c_i64, _c_vp, _c_i64, _PR, _c_vp, _c_vp, _c_vp]),
    "pom_agg_bwd": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _PV, _c_vp, _c_vp, _c_i64, _c_i64,
                             _c_vp, _c_i64, _c_i64, _PR, _c_vp, _PV, _PT, _c_vp, _c_vp, _c_size, _c_vp]),
    "pom_gate_workspace_size": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int]),
    "pom_gate_fwd": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _PV, _c_vp, _c_vp, _c_i64, _PR, _PV, _PT, _c_vp]),
    "pom_gate_bwd": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _PV, _c_vp, _c_vp, _c_i64, _PR, _PV, _PV, _PT,
                              _c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
    "pom_gate_heads_workspace_size": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "pom_gate_heads_fwd": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _PV, _c_vp, _c_vp, _c_i64, _PR,
                                    _PV, _PT, _c_vp]),
    "pom_gate_heads_bwd": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _PV, _c_vp, _c_vp, _c_i64, _PR,
                                    _PV, _PV, _c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
    "pom_features_workspace_size": (_c_size, [_c_int, _c_i64, _c_i64, _c_i64, _c_int]),
    "pom_features_fwd": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _PV, _c_vp, _PV, _c_vp]),
    "pom_features_bwd": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _PV, _c_vp, _PV, _PV, _c_vp,
                                  _c_vp, _c_size, _c_vp]),
    "pom_transpose": (_c_int, [_c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp]),
    "pom_gemm_plan": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int, _c_int, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int)]),
    "pom_gemm_workspace_size": (_c_size, [_c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "pom_gemm": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_vp, _c_i64,
                          _c_int, _c_int, _c_vp, _c_size, _c_vp]),
    "pom_blas_set_solution": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "pom_blas_has_solution": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "pom_blas_gemm": (_c_int, [_c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_size,
                               _c_vp]),
    "pom_blas_library": (ctypes.c_char_p, [_c_int]),
    "pom_layer_args_size": (_c_size, []),
    "pom_layer_workspace_size": (_c_size, [ctypes.POINTER(PomLayerArgs), _c_int]),
    "pom_layer_fwd": (_c_int, [ctypes.POINTER(PomLayerArgs), _c_vp]),
    "pom_layer_bwd": (_c_int, [ctypes.POINTER(PomLayerArgs), _c_vp]),
}
BLAS_ROCBLAS, BLAS_HIPBLASLT = 1, 2
GEMM_STREAM_K = 256   # pom_gemm's `splits` value for the stream-K schedule

_lib: Optional[ctypes.CDLL] = None
_lib_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load libpom_amd.so (once) and bind every declared symbol; raise if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"pom_amd: HIP library not found at {LIB_PATH}; build it with "
                "`python pom_amd/csrc/build.py` (there is no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.pom_abi_version() != ABI_VERSION:
            raise RuntimeError("pom_amd: ABI version mismatch; rebuild libpom_amd.so")
        if lib.pom_layer_args_size() != ctypes.sizeof(PomLayerArgs):
            raise RuntimeError("pom_amd: pom_layer_args layout differs from PomLayerArgs; rebuild libpom_amd.so")
        _lib = lib
    return _lib


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def check(rc: int, what: str) -> None:
    """Map a pom_status to a Python exception carrying pom_last_error()."""
    if rc == POM_OK:
        return
    msg = f"{what}: {load().pom_last_error().decode(errors='replace')}"
    if rc == POM_ERR_INVALID:
        raise ValueError(msg)
    if rc == POM_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"pom_amd: unsupported dtype {t.dtype}; expected float32, bfloat16 or float16")


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("pom_amd runs on ROCm devices only (got a CPU tensor); "
                               "move the module and inputs to a GPU")


def tview(t: Optional["torch.Tensor"], B: int, N: int):
    """Channel-major copy target: a (C, B*N) tensor with unit token stride, as
    a PomTView (element (b, n, c) at c * stride_c + b * N + n), or None."""
    if t is None:
        return None
    if t.dim() != 2 or t.shape[1] != B * N or t.stride(1) != 1:
        raise ValueError(f"channel-major copy must be (C, {B * N}) with unit token stride, got "
                         f"{tuple(t.shape)} strides {t.stride()}")
    return ctypes.byref(PomTView(t.data_ptr(), t.stride(0), N))


def view3(t: torch.Tensor) -> PomView:
    """(B, N, C) tensor with unit last-axis stride -> PomView."""
    if t.dim() != 3:
        raise ValueError(f"expected a 3-D (B, N, C) tensor, got shape {tuple(t.shape)}")
    if t.shape[2] > 1 and t.stride(2) != 1:
        raise ValueError("the channel axis must have unit stride")
    return PomView(t.data_ptr(), t.stride(0), t.stride(1))


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_ws_cache: dict = {}
_ws_lock = threading.Lock()


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch workspace for one (device, stream); contents need no initialisation.

    Calls on one stream run in order, so they share the buffer; a larger
    request replaces it with a bigger one (the caching allocator keeps the old
    block alive until the queued kernels that use it have run).
    """
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream)
    with _ws_lock:
        buf = _ws_cache.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _ws_cache[key] = buf
        return buf


# Parameter-derived copies (fp32 coefficient / bias copies, transposed and
# padded weights, fp32 RoPE tables) are rebuilt on every call by default.  A
# cache keyed on the tensor's identity, storage pointer and version counter is
# opt-in (set_derived_cache(True) or POM_AMD_CACHE_DERIVED=1): an in-place
# write through ``p.data`` does not bump the version counter, so with the
# cache on, such writes (EMA swaps, clamps through .data) must be followed by
# invalidate_derived().
_cache_on = os.environ.get("POM_AMD_CACHE_DERIVED", "0") == "1"
_derived_caches: list = []


def set_derived_cache(enabled: bool) -> None:
    """Turn the parameter-derived copy cache on or off (dropping its entries)."""
    global _cache_on
    _cache_on = bool(enabled)
    invalidate_derived()


def derived_cache_enabled() -> bool:
    return _cache_on


def invalidate_derived() -> None:
    """Drop every cached parameter-derived copy."""
    for c in _derived_caches:
        c.clear()


def derived(cache: dict, t: "torch.Tensor", make, always: bool = False):
    """``make(t)``: a copy derived from parameter ``t``.  With the cache on
    (set_derived_cache), the copy is kept while that same tensor object is
    alive and unchanged by identity, storage pointer and version counter;
    keyed by object identity, so a freed tensor's address or id reused by a
    new tensor can never hit a stale copy.  Under stream capture the copy is
    always rebuilt, so a captured graph recomputes it on every replay (a replay
    runs no Python and would otherwise keep the capture-time copy).
    ``always``: cache even with the cache off (tensors that are not trained,
    e.g. RoPE tables, whose version only moves when they are rewritten)."""
    if not (_cache_on or always) or (t.is_cuda and torch.cuda.is_current_stream_capturing()):
        return make(t)
    if not any(c is cache for c in _derived_caches):
        _derived_caches.append(cache)
    hit = cache.get(id(t))
    if hit is not None:
        ref, version, ptr, c = hit
        if ref() is t and version == t._version and ptr == t.data_ptr():
            return c
    c = make(t)
    if len(cache) > 64:
        for k in [k for k, v in cache.items() if v[0]() is None]:
            del cache[k]
        if len(cache) > 64:
            cache.clear()
    cache[id(t)] = (weakref.ref(t), t._version, t.data_ptr(), c)
    return c


_table_cache: dict = {}


def _f32_table(t: torch.Tensor) -> torch.Tensor:
    """fp32 contiguous view or cached copy of a RoPE table (a module buffer,
    bf16 in a bf16 model): converted once per table version, not per call,
    whether or not the parameter cache is on (tables are not trained)."""
    if t.dtype == torch.float32 and t.is_contiguous():
        return t
    return derived(_table_cache, t, lambda u: u.detach().float().contiguous(), always=True)


# POM_AMD_CHECK_POSITIONS=1: also range-check RoPE positions that live on the
# device (one device-to-host synchronisation per RopeSpec).
_CHECK_DEVICE_POSITIONS = os.environ.get("POM_AMD_CHECK_POSITIONS", "0") == "1"


def _check_positions(pos: torch.Tensor, rows) -> None:
    """Raise IndexError for positions outside [-rows, rows), the range torch's
    indexing of the tables accepts (pom/pom_rope.py:173-174, :211-212)."""
    if pos.numel() == 0:
        return
    cols = pos.view(-1, 1) if pos.dim() == 1 else pos
    for j, r in enumerate(rows):
        lo, hi = int(cols[:, j].min()), int(cols[:, j].max())
        if lo < -r or hi >= r:
            raise IndexError(f"RoPE position out of range for a table of {r} rows "
                             f"(positions span [{lo}, {hi}])")


class RopeSpec:
    """Device-side RoPE description: fp32 tables and int64 positions kept alive
    for as long as the kernels may read them.

    Positions in [-rows, 0) select row p + rows (torch's indexing, done in the
    kernels' table lookup).  Positions outside [-rows, rows) raise IndexError
    when they are checked: positions given as a host tensor always are (before
    the copy to the device), device positions under POM_AMD_CHECK_POSITIONS=1;
    unchecked ones are clamped to the table by the kernels.  ``n_max``: the
    positions are known to be arange(n_max) (checked on the host for free).
    """

    def __init__(self, kind: int, tables, pos: torch.Tensor, device=None, n_max: Optional[int] = None):
        self.kind = kind
        self.tables = [_f32_table(t) for t in tables]
        width = self.tables[0].shape[1]
        for t in self.tables:
            if t.shape[1] != width:
                raise ValueError("RoPE tables must share their width")
        self.width = width
        rows = [self.tables[0].shape[0]] if kind == ROPE_1D else [self.tables[0].shape[0], self.tables[2].shape[0]]
        if n_max is not None:
            if n_max > min(rows):
                raise IndexError(f"sequence of {n_max} tokens is longer than the RoPE table ({min(rows)} rows)")
        elif not pos.is_cuda or _CHECK_DEVICE_POSITIONS:
            _check_positions(pos, rows)
        dev = self.tables[0].device if device is None else device
        self.pos = pos.to(device=dev, dtype=torch.int64).contiguous()

    def struct(self) -> PomRope:
        t = self.tables
        if self.kind == ROPE_1D:
            return PomRope(ROPE_1D, t[0].data_ptr(), t[1].data_ptr(), None, None, t[0].stride(0),
                           t[0].shape[0], 0, self.pos.data_ptr(), 1)
        return PomRope(ROPE_2D, t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), t[3].data_ptr(),
                       t[0].stride(0), t[0].shape[0], t[2].shape[0], self.pos.data_ptr(), 2)


def rope_ptr(spec: Optional[RopeSpec]):
    return None if spec is None else ctypes.byref(spec.struct())
