"""Offline-tuned algorithm selection for the projection GEMMs.

The projections are plain bf16 GEMMs on hipBLASLt / rocBLAS.  Their default
heuristic picks are 21-43 % of the MI355X bf16 peak on the PoM shapes; an
exhaustive search over the libraries' solutions (PyTorch TunableOp) finds
kernels that are up to 1.8x faster.  The search results for the baseline
configurations ship in ``tuned/gemm_gfx950.csv``.

``tuned_gemms()`` makes torch's GEMMs look their shapes up in that table for
the duration of a ``with`` block, with tuning itself switched off, so nothing is
benchmarked or written at run time.  Shapes missing from the table use the
default heuristic.  The table is rejected by torch (and the default used) when
the PyTorch, ROCm, hipBLASLt or rocBLAS versions differ from the ones it was
made with.  The caller's TunableOp settings are restored on exit.  Set
POM_AMD_TUNED_GEMMS=0 to disable, or POM_AMD_GEMM_TABLE to the path of another
table in the same format.
"""
from __future__ import annotations

import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
TABLE = os.environ.get("POM_AMD_GEMM_TABLE") or os.path.join(_HERE, "tuned", "gemm_gfx950.csv")

_lock = threading.Lock()
_loaded = None   # None: not tried; True/False: table usable


def _ready() -> bool:
    global _loaded
    if _loaded is not None:
        return _loaded
    with _lock:
        if _loaded is None:
            ok = False
            if os.environ.get("POM_AMD_TUNED_GEMMS", "1") != "0" and os.path.exists(TABLE):
                try:
                    tun = torch.cuda.tunable
                    ok = bool(tun.read_file(TABLE))
                except (AttributeError, RuntimeError):
                    ok = False
            _loaded = ok
    return _loaded


class tuned_gemms:
    """Context manager: GEMMs inside use the shipped selection table."""

    __slots__ = ("_prev",)

    def __init__(self):
        self._prev = None

    def __enter__(self):
        if _ready():
            tun = torch.cuda.tunable
            self._prev = (tun.is_enabled(), tun.tuning_is_enabled())
            tun.tuning_enable(False)
            tun.enable(True)
        return self

    def __exit__(self, *exc):
        if self._prev is not None:
            tun = torch.cuda.tunable
            tun.enable(self._prev[0])
            tun.tuning_enable(self._prev[1])
        return False


_native_lock = threading.Lock()
_native = None   # None: not tried; True/False: the C library's GEMMs use the table


def table_entries():
    """The table's bf16 "tn" entries with a library solution:
    [((m, n, k, lda, ldb, ldc), lib, index)], lib 1 = rocBLAS, 2 = hipBLASLt
    (entries whose pick is torch's default path are left out)."""
    out = []
    if not os.path.exists(TABLE):
        return out
    with open(TABLE) as f:
        for line in f:
            parts = line.strip().split(",")
            if len(parts) < 3 or parts[0] != "GemmTunableOp_BFloat16_TN" or not parts[1].startswith("tn_"):
                continue
            dims = parts[1].split("_")            # tn, m, n, k, ld, lda, ldb, ldc
            if len(dims) != 8 or dims[4] != "ld":
                continue
            m, n, k, lda, ldb, ldc = (int(v) for v in dims[1:4] + dims[5:8])
            sol = parts[2]
            if sol.startswith("Gemm_Rocblas_"):
                out.append(((m, n, k, lda, ldb, ldc), 1, int(sol[len("Gemm_Rocblas_"):])))
            elif sol.startswith("Gemm_Hipblaslt_"):
                out.append(((m, n, k, lda, ldb, ldc), 2, int(sol[len("Gemm_Hipblaslt_"):])))
    return out


def native_ready() -> bool:
    """Register the table's solutions with the C library's GEMM entry point
    (pom_blas_gemm), once; True when it did.  Only when torch accepted the
    table (its validators match the libraries torch runs) and the C library's
    rocBLAS and hipBLASLt calls resolve to those same loaded files, so that a
    solution index names the same kernel on both routes."""
    global _native
    if _native is not None:
        return _native
    with _native_lock:
        if _native is None:
            ok = False
            if _ready():
                from . import _lib
                lib = _lib.load()
                tdir = os.path.realpath(os.path.join(os.path.dirname(torch.__file__), "lib"))
                files = [os.path.realpath(lib.pom_blas_library(k).decode() or "/") for k in (1, 2)]
                if all(os.path.dirname(f) == tdir for f in files):
                    ok = True
                    for (m, n, k, lda, ldb, ldc), which, idx in table_entries():
                        ok = ok and lib.pom_blas_set_solution(m, n, k, lda, ldb, ldc, which, idx) == 0
            _native = ok
    return _native
