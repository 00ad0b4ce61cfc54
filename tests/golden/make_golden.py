"""Write the golden fixtures of the PoM module composition from the reference.

Run in the build container only (the reference is not on the GPU box):
    POM_DISABLE_TRITON=1 python tests/golden/make_golden.py [/root/reference]

The fixtures pin what no closed form or brute-force check pins: the module
composition of the reference (parameter draw order of PoM.__init__, the
[h | s] split of qc_proj, se_bias + hardsigmoid, the pom(s, h) argument order,
the ag_proj output, state_forward's carry semantics, PoMRoPE's 1-D / 2-D
rotations including the strided tables of the n_sel_heads > 1 gate, masks).

Every case runs the reference's own module on CPU tensors (its PyTorch
route, pom/pom.py:82-100 and pom/pom_rope.py:511-515) and stores inputs,
parameters, outputs and gradients as float64 arrays in one .npz per case
(numpy, no pickle).  Sizes are tiny; the files are data, not source.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _np(t):
    return t.detach().double().cpu().numpy()



def _save(name, summary=False, **arrays):
    """One .npz per case.  summary=True keeps, per array, its sum, its L2 norm
    and 4096 evenly strided values instead of the whole array."""
    path = os.path.join(HERE, f"{name}.npz")
    out = {}
    for k, v in arrays.items():
        v = np.asarray(v)
        if summary and v.size > 4096 and v.dtype.kind == "f":
            flat = v.reshape(-1)
            idx = np.linspace(0, flat.size - 1, 4096).astype(np.int64)
            out[k + ".sum"] = flat.sum()
            out[k + ".l2"] = np.sqrt((flat * flat).sum())
            out[k + ".sample"] = flat[idx]
            out[k + ".sample_idx"] = idx
            out[k + ".shape"] = np.array(v.shape)
        else:
            out[k] = v
    np.savez_compressed(path, **out)
    print("wrote", os.path.relpath(path))


def _params(m):
    return {f"param.{k}": _np(v) for k, v in m.named_parameters()}


def _grads(m):
    return {f"grad.{k}": _np(v.grad) for k, v in m.named_parameters() if v.grad is not None}


def _buffers(m):
    return {f"buffer.{k}": _np(v) for k, v in m.named_buffers()}


def pom_case(P, name, dim, degree, expand, n_sel_heads, B, N, mask_kind=None, bias=False, n_groups=1,
             dtype=torch.float32, coeff_std=None, summary=False):
    torch.manual_seed(0)
    m = P.PoM(dim, degree, expand, n_groups, n_sel_heads, bias)
    if coeff_std is not None:
        with torch.no_grad():
            m.po_coeff.copy_(torch.randn(m.po_coeff.shape, generator=torch.Generator().manual_seed(11)) * coeff_std)
    m = m.to(dtype)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, N, dim, generator=g).to(dtype)
    mask = None
    extra = {}
    if mask_kind == "padding":
        lens = torch.tensor([N, max(1, N // 3)] + [N // 2] * (B - 2))[:B]
        mask = torch.arange(N).view(1, N) < lens.view(B, 1)
        extra["mask"] = mask.numpy().astype(np.float64)
    elif mask_kind == "causal":
        mask = "causal"
    elif mask_kind == "block3d":
        L = N // 4
        f = torch.arange(N) // L
        mask = (f.view(N, 1) >= f.view(1, N)).to(dtype).unsqueeze(0).expand(B, N, N).contiguous()
        extra["mask3d"] = _np(mask)
        extra["frame_len"] = np.array(L)
    xr = x.clone().requires_grad_(True)
    out = m(xr, mask=mask)
    go = torch.randn(out.shape, generator=torch.Generator().manual_seed(2)).to(dtype)
    out.backward(go)
    _save(name, summary, x=_np(x), out=_np(out), go=_np(go), grad_x=_np(xr.grad), **_params(m), **_grads(m),
          **extra, meta=np.array([dim, degree, expand, n_groups, n_sel_heads, int(bias)]))


def state_case(P, name, dim, degree, expand, B, L, F, dtype):
    torch.manual_seed(0)
    m = P.PoM(dim, degree, expand, 1, 1, False)
    with torch.no_grad():
        m.po_coeff.copy_(torch.randn(m.po_coeff.shape, generator=torch.Generator().manual_seed(11)) * 0.1)
    m = m.to(dtype)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, F * L, dim, generator=g).to(dtype)
    state = None
    outs, hs, ns = [], [], []
    with torch.no_grad():
        for f in range(F):
            xf = x[:, f * L:(f + 1) * L]
            o, state = m.state_forward(xf, xf, state)
            outs.append(_np(o))
            hs.append(_np(state["h"]))
            ns.append(state["n"])
            assert state["h"].dtype == dtype
    _save(name, x=_np(x), out=np.stack(outs, 1), h=np.stack(hs, 1), n=np.array(ns), **_params(m),
          meta=np.array([dim, degree, expand, L, F]), dtype=np.array(str(dtype)))


def rope_case(P, name, dim, degree, expand, n_sel_heads, B, H, W, rope_2d, mask_kind=None, positions=None):
    torch.manual_seed(0)
    m = P.PoMRoPE(dim, degree, expand, 1, n_sel_heads, False, max_seq_len=64, max_h=H + 2, max_w=W + 2,
                  rope_base=100.0, rope_2d=rope_2d)
    with torch.no_grad():
        m.po_coeff.copy_(torch.randn(m.po_coeff.shape, generator=torch.Generator().manual_seed(11)) * 0.1)
        m.se_bias.copy_(torch.randn(m.se_bias.shape, generator=torch.Generator().manual_seed(12)) * 0.5)
    N = H * W
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, N, dim, generator=g)
    kw = {}
    extra = {}
    if rope_2d:
        pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
        kw["positions_hw"] = pos
        extra["positions_hw"] = pos.numpy().astype(np.float64)
    elif positions is not None:
        kw["positions"] = positions
        extra["positions"] = positions.numpy().astype(np.float64)
    mask = None
    if mask_kind == "causal":
        mask = "causal"
    elif mask_kind == "padding":
        lens = torch.tensor([N, N // 3] + [N // 2] * (B - 2))[:B]
        mask = torch.arange(N).view(1, N) < lens.view(B, 1)
        extra["mask"] = mask.numpy().astype(np.float64)
    xr = x.clone().requires_grad_(True)
    out = m(xr, mask=mask, **kw)
    go = torch.randn(out.shape, generator=torch.Generator().manual_seed(2))
    out.backward(go)
    _save(name, x=_np(x), out=_np(out), go=_np(go), grad_x=_np(xr.grad), **_params(m), **_grads(m),
          **_buffers(m), **extra, meta=np.array([dim, degree, expand, n_sel_heads, int(rope_2d), H, W]))


def ar_case(P, name, dim, degree, expand, n_sel_heads, n_groups, B, T):
    """PoM.ar_forward twice from a fresh state, then reset (pom/pom.py:264-280):
    the per-token gate times the raw projected context, 'n' advancing by T
    per call, 'max_len' passed through."""
    torch.manual_seed(0)
    m = P.PoM(dim, degree, expand, n_groups, n_sel_heads, False)
    with torch.no_grad():
        if n_groups == 1:
            m.se_bias.copy_(torch.randn(m.se_bias.shape, generator=torch.Generator().manual_seed(12)) * 0.5)
    g = torch.Generator().manual_seed(1)
    x1 = torch.randn(B, T, dim, generator=g)
    x2 = torch.randn(B, T, dim, generator=g)
    state = {"max_len": 64, "h": 0., "n": 0}
    out1, st1 = m.ar_forward(x1, state)
    out2, st2 = m.ar_forward(x2, st1)
    assert st2["max_len"] == 64
    after = m.reset(dict(st2))
    _save(name, x1=_np(x1), x2=_np(x2), out1=_np(out1), out2=_np(out2), h1=_np(st1["h"]), h2=_np(st2["h"]),
          n=np.array([st1["n"], st2["n"]]), reset_n=np.array(after["n"]), reset_h=np.array(float(after["h"])),
          **_params(m), meta=np.array([dim, degree, expand, n_groups, n_sel_heads, 0]))


CASES = [
    # PoM composition: init order, projections, gating, mean aggregation
    (pom_case, "pom_mean_f32", (32, 2, 2, 1, 2, 16), {}),
    (pom_case, "pom_mean_k3_coeff", (32, 3, 2, 1, 2, 16), dict(coeff_std=0.1)),
    (pom_case, "pom_mean_bias", (24, 2, 3, 1, 2, 12), dict(bias=True, coeff_std=0.1)),
    (pom_case, "pom_masked", (32, 2, 2, 1, 3, 16), dict(mask_kind="padding", coeff_std=0.1)),
    (pom_case, "pom_causal", (32, 2, 2, 1, 2, 16), dict(mask_kind="causal", coeff_std=0.1)),
    (pom_case, "pom_block3d", (32, 2, 2, 1, 2, 16), dict(mask_kind="block3d", coeff_std=0.1)),
    (pom_case, "pom_heads", (32, 2, 2, 4, 2, 16), dict(coeff_std=0.1)),
    (pom_case, "pom_groups", (32, 2, 2, 1, 2, 16), dict(n_groups=4, coeff_std=0.1)),
    # config 1 at its real size (B2 N256 D256 degree 2 expand 2 fp32), seed-0 init
    (pom_case, "pom_c1", (256, 2, 2, 1, 2, 256), dict(summary=True)),
    # state_forward: 'n' counts calls, 'h' carried in the input dtype
    (state_case, "state_f32", (32, 2, 2, 2, 8, 4, torch.float32), {}),
    (state_case, "state_bf16", (32, 2, 2, 2, 8, 4, torch.bfloat16), {}),
    # PoMRoPE
    (rope_case, "rope2d", (16, 2, 2, 1, 2, 4, 4, True), {}),
    (rope_case, "rope2d_heads", (16, 2, 2, 4, 2, 4, 4, True), {}),
    (rope_case, "rope1d", (16, 2, 2, 1, 2, 4, 4, False), {}),
    (rope_case, "rope1d_pos", (16, 2, 2, 1, 2, 4, 4, False),
     dict(positions=torch.tensor([3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5, 8, 9, 7, 9, 3]))),
    (rope_case, "rope1d_heads", (16, 2, 2, 4, 2, 4, 4, False), {}),
    (rope_case, "rope1d_causal", (16, 2, 2, 1, 2, 4, 4, False), dict(mask_kind="causal")),
    (rope_case, "rope2d_masked", (16, 2, 2, 1, 3, 4, 4, True), dict(mask_kind="padding")),
    # ar_forward / reset: plain, per-head gate, grouped projection
    (ar_case, "ar_plain", (32, 2, 2, 1, 1, 2, 8), {}),
    (ar_case, "ar_heads", (32, 2, 2, 4, 1, 2, 8), {}),
    (ar_case, "ar_groups", (32, 2, 2, 1, 4, 2, 8), {}),
]


def main():
    """Usage: make_golden.py [reference_dir] [--only=<name prefix> ...]"""
    args = [a for a in sys.argv[1:] if not a.startswith("--only=")]
    only = [a[len("--only="):] for a in sys.argv[1:] if a.startswith("--only=")]
    ref = args[0] if args else "/root/reference"
    os.environ.setdefault("POM_DISABLE_TRITON", "1")
    sys.path.insert(0, ref)
    import pom as P   # the reference package (pure PyTorch route on CPU tensors)
    torch.set_num_threads(4)
    for fn, name, a, kw in CASES:
        if not only or any(name.startswith(o) for o in only):
            fn(P, name, *a, **kw)


if __name__ == "__main__":
    main()
