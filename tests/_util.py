"""Shared helpers of the parity tests."""
from __future__ import annotations

import torch

# Elementwise tolerances of the reference's own kernel tests
# (test_triton_correctness.py:92-95, test_triton_rope_correctness.py:92-95):
# |a - b| <= atol + rtol * |b|.
KERNEL_TOLS = {
    torch.float32: dict(atol=1e-4, rtol=1e-3),
    torch.bfloat16: dict(atol=1e-3, rtol=5e-3),
    torch.float16: dict(atol=1e-3, rtol=5e-3),
}
ROPE_TOLS = {
    torch.float32: dict(atol=1e-4, rtol=1e-3),
    torch.bfloat16: dict(atol=1e-2, rtol=1e-2),
    torch.float16: dict(atol=1e-2, rtol=1e-2),
}
# Norm-wise relative bound of the build's contract, against the fp32/fp64
# reference computed from the same (quantised) inputs.
REL_TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """||a - b|| / ||b|| in fp64 (0 when both are zero)."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    nb = b.norm().item()
    d = (a - b).norm().item()
    return d if nb == 0 else d / nb


def assert_close(got: torch.Tensor, ref: torch.Tensor, dtype, tols=KERNEL_TOLS, what: str = ""):
    t = tols[dtype]
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert g.shape == r.shape, f"{what}: shape {tuple(g.shape)} vs {tuple(r.shape)}"
    diff = (g - r).abs()
    thr = t["atol"] + t["rtol"] * r.abs()
    bad = ~(diff <= thr)
    if bad.any():
        i = int(bad.flatten().nonzero()[0])
        raise AssertionError(f"{what}: {int(bad.sum())}/{diff.numel()} elements off; first at flat {i}: "
                             f"got {g.flatten()[i]:.6g} ref {r.flatten()[i]:.6g}; max abs {diff.max():.3g}")


def assert_rel(got, ref, dtype, what: str = "", tol=None):
    e = rel_err(got, ref)
    bound = REL_TOL[dtype] if tol is None else tol
    assert e <= bound, f"{what}: relative error {e:.3g} > {bound:g}"
    return e


def oracle_params(module, dtype=torch.float64):
    """OracleParams holding a copy of a pom_amd PoM / PoMRoPE module's weights."""
    from oracle import pom_oracle as O
    cv = lambda t: None if t is None else t.detach().to("cpu", dtype)
    rope = None
    if hasattr(module, "rope_2d"):
        if module.rope_2d:
            rope = {"rope_2d": True, "row_cos": cv(module.row_cos), "row_sin": cv(module.row_sin),
                    "col_cos": cv(module.col_cos), "col_sin": cv(module.col_sin)}
        else:
            rope = {"rope_2d": False, "freqs_cos": cv(module.freqs_cos), "freqs_sin": cv(module.freqs_sin)}
    return O.OracleParams(module.dim, module.order, module.order_expand, module.n_sel_heads,
                          cv(module.qc_proj.weight), cv(module.se_bias), cv(module.po_coeff),
                          cv(module.ag_proj.weight), cv(module.ag_proj.bias), rope)


def oracle_grads(prm, names=("w_qc", "se_bias", "po_coeff", "w_ag", "b_ag")):
    out = {}
    for n in names:
        t = getattr(prm, n)
        if t is not None:
            out[n] = t.grad
    return out


def requires_grad_params(prm, names=("w_qc", "se_bias", "po_coeff", "w_ag", "b_ag")):
    for n in names:
        t = getattr(prm, n)
        if t is not None:
            t.requires_grad_(True)
    return prm


MODULE_GRADS = {"w_qc": "qc_proj.weight", "se_bias": "se_bias", "po_coeff": "po_coeff",
                "w_ag": "ag_proj.weight", "b_ag": "ag_proj.bias"}
