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
POM_AMD_TUNED_GEMMS=0 to disable.
"""
from __future__ import annotations

import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
TABLE = os.path.join(_HERE, "tuned", "gemm_gfx950.csv")

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
