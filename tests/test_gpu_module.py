"""End-to-end parity of PoM / PoMRoPE (forward + every gradient) with the oracle.

fp32 modules must match the fp64 oracle to 1e-5 (norm-wise relative); bf16
modules to 2e-2 against the oracle run on the bf16-quantised weights and
inputs, the bar stated for this build.
"""
import pytest
import torch

from oracle import pom_oracle as O
from _util import MODULE_GRADS, assert_rel, oracle_params, requires_grad_params

pytestmark = pytest.mark.gpu

import pom_amd  # noqa: E402


def _inputs(B, N, D, dtype, seed=1):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, N, D, generator=g).to(dtype)
    go = torch.randn(B, N, D, generator=torch.Generator().manual_seed(seed + 1)).to(dtype)
    return x, go


def _check_module(device, module, x, go, dtype, oracle_fn, module_fn, tol=None, what=""):
    prm = requires_grad_params(oracle_params(module))
    xr = x.double().requires_grad_(True)
    ref = oracle_fn(prm, xr)
    ref.backward(go.double())

    m = module.to(device)
    xd = x.to(device).requires_grad_(True)
    out = module_fn(m, xd)
    assert out.dtype == dtype and out.shape == ref.shape
    out.backward(go.to(device))
    errs = {"out": assert_rel(out, ref, dtype, f"{what} out", tol)}
    errs["x"] = assert_rel(xd.grad, xr.grad, dtype, f"{what} grad x", tol)
    for oname, mname in MODULE_GRADS.items():
        t = getattr(prm, oname)
        if t is None:
            continue
        p = dict(m.named_parameters())[mname]
        errs[mname] = assert_rel(p.grad, t.grad, dtype, f"{what} grad {mname}", tol)
    return errs


def _pom(dim, degree, expand, dtype, seed=0, coeff_std=None, bias=False, heads=1):
    torch.manual_seed(seed)
    m = pom_amd.PoM(dim, degree, expand, 1, heads, bias)
    if coeff_std is not None:
        with torch.no_grad():
            m.po_coeff.copy_(torch.randn(m.po_coeff.shape, generator=torch.Generator().manual_seed(11)) * coeff_std)
            m.se_bias.copy_(torch.randn(m.se_bias.shape, generator=torch.Generator().manual_seed(12)) * 0.5)
    return m.to(dtype)


def test_c1_fp32(device):
    """Config 1: B2 N256 D256 degree 2 expand 2 fp32, nn.Linear init from seed 0."""
    x, go = _inputs(2, 256, 256, torch.float32)
    m = _pom(256, 2, 2, torch.float32)
    _check_module(device, m, x, go, torch.float32, lambda p, xr: O.pom_forward(p, xr), lambda m, xd: m(xd))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,D,K,E", [(2, 256, 128, 2, 2), (2, 128, 96, 3, 2), (1, 64, 64, 4, 1)])
def test_mean_module(device, B, N, D, K, E, dtype):
    x, go = _inputs(B, N, D, dtype)
    m = _pom(D, K, E, dtype, coeff_std=0.1, bias=True)
    _check_module(device, m, x, go, dtype, lambda p, xr: O.pom_forward(p, xr), lambda m, xd: m(xd))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_module(device, dtype):
    B, N, D = 4, 256, 64
    x, go = _inputs(B, N, D, dtype)
    L = torch.tensor([256, 17, 100, 200])
    mask = torch.arange(N).view(1, N) < L.view(B, 1)
    m = _pom(D, 3, 2, dtype, coeff_std=0.1)
    _check_module(device, m, x, go, dtype, lambda p, xr: O.pom_forward(p, xr, mask=mask),
                  lambda m, xd: m(xd, mask=mask.to(device)))


def test_masked_padding_does_not_leak(device):
    """Config 3 contract: padded tokens' values never change valid outputs."""
    B, N, D = 3, 512, 64
    x, _ = _inputs(B, N, D, torch.bfloat16)
    L = torch.tensor([300, 512, 1])
    mask = torch.arange(N).view(1, N) < L.view(B, 1)
    x2 = x.clone()
    x2[~mask] = (torch.randn(int((~mask).sum()), D) * 3).to(torch.bfloat16)
    m = _pom(D, 3, 2, torch.bfloat16, coeff_std=0.1).to(device)
    with torch.no_grad():
        a = m(x.to(device), mask=mask.to(device))
        b = m(x2.to(device), mask=mask.to(device))
    md = mask.to(device)
    assert torch.equal(a[md], b[md])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_causal_module(device, dtype):
    B, F, L, D = 2, 4, 64, 64
    x, go = _inputs(B, F * L, D, dtype)
    m = _pom(D, 2, 4, dtype, coeff_std=0.1)
    dense = O.block_causal_dense_mask(B, F * L, L, torch.float64)
    _check_module(device, m, x, go, dtype, lambda p, xr: O.pom_forward(p, xr, mask=dense),
                  lambda m, xd: m(xd, mask=pom_amd.block_causal(L)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_state_forward_loop_matches_full(device, dtype):
    """Config 4 contract: the frame-by-frame state_forward loop reproduces the
    full-sequence block-causal pass (README.md:46-61 loop)."""
    B, F, L, D = 2, 4, 128, 64
    x, go = _inputs(B, F * L, D, dtype)
    m = _pom(D, 2, 4, dtype, coeff_std=0.1).to(device)
    xd = x.to(device)
    with torch.no_grad():
        full = m(xd, mask=pom_amd.block_causal(L))
        state, outs = None, []
        for f in range(F):
            o, state = m.state_forward(xd[:, f * L:(f + 1) * L], state=state)
            outs.append(o)
        loop = torch.cat(outs, dim=1)
    assert state["n"] == F and state["h"].shape == (B, 1, 2 * 0 + m._po_dim) and state["h"].dtype == dtype
    assert_rel(loop, full, dtype, "loop vs full", 1e-5 if dtype == torch.float32 else 1e-2)
    # and the loop matches the reference's own state_forward semantics
    prm = oracle_params(m)
    st, ref_outs = None, []
    for f in range(F):
        o, st = O.state_forward(prm, x[:, f * L:(f + 1) * L].double(), state=st)
        ref_outs.append(o)
    assert_rel(loop, torch.cat(ref_outs, 1), dtype, "loop vs oracle state_forward")


def test_state_forward_grad(device):
    """Gradients flow through the carry across calls as in the reference."""
    B, L, D = 2, 64, 32
    x, go = _inputs(B, 2 * L, D, torch.float32)
    m = _pom(D, 2, 2, torch.float32, coeff_std=0.1)
    prm = requires_grad_params(oracle_params(m))
    xr = x.double().requires_grad_(True)
    o1, st = O.state_forward(prm, xr[:, :L])
    o2, st = O.state_forward(prm, xr[:, L:], state=st)
    (torch.cat([o1, o2], 1) * go.double()).sum().backward()
    m = m.to(device)
    xd = x.to(device).requires_grad_(True)
    p1, s = m.state_forward(xd[:, :L])
    p2, s = m.state_forward(xd[:, L:], state=s)
    (torch.cat([p1, p2], 1) * go.to(device)).sum().backward()
    assert_rel(xd.grad, xr.grad, torch.float32, "grad x")
    assert_rel(m.po_coeff.grad, prm.po_coeff.grad, torch.float32, "grad coeff")
    assert_rel(m.qc_proj.weight.grad, prm.w_qc.grad, torch.float32, "grad w_qc")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_causal_module(device, dtype):
    x, go = _inputs(2, 64, 32, dtype)
    m = _pom(32, 2, 2, dtype, coeff_std=0.1)
    _check_module(device, m, x, go, dtype, lambda p, xr: O.pom_forward(p, xr, mask="causal"),
                  lambda m, xd: m(xd, mask="causal"))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cross_mixing(device, dtype):
    """xq is not xc: two projections on weight slices (pom/pom.py:208-213)."""
    B, T, N, D = 2, 48, 96, 64
    xq, go = _inputs(B, T, D, dtype)
    xc, _ = _inputs(B, N, D, dtype, seed=5)
    m = _pom(D, 2, 2, dtype, coeff_std=0.1)
    xcd = xc.to(device)
    _check_module(device, m, xq, go, dtype, lambda p, xr: O.pom_forward(p, xr, xc.double()),
                  lambda m, xd: m(xd, xcd))


def _rope_module(dim, degree, expand, dtype, rope_2d, seed=0, heads=1, **kw):
    torch.manual_seed(seed)
    m = pom_amd.PoMRoPE(dim, degree, expand, 1, heads, False, rope_2d=rope_2d, **kw)
    with torch.no_grad():
        m.po_coeff.copy_(torch.randn(m.po_coeff.shape, generator=torch.Generator().manual_seed(11)) * 0.1)
    return m.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope2d_module(device, dtype):
    """Config 5 in miniature: axial 2-D RoPE on a 16x16 grid."""
    H = W = 16
    pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
    x, go = _inputs(2, H * W, 64, dtype)
    m = _rope_module(64, 2, 2, dtype, True, max_h=H, max_w=W)
    _check_module(device, m, x, go, dtype, lambda p, xr: O.rope_forward(p, xr, positions_hw=pos),
                  lambda m, xd: m(xd, positions_hw=pos.to(device)))


@pytest.mark.parametrize("mask", [None, "causal"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope1d_module(device, dtype, mask):
    x, go = _inputs(2, 64, 48, dtype)
    m = _rope_module(48, 2, 2, dtype, False, max_seq_len=128)
    pos = torch.arange(64) + 3
    _check_module(device, m, x, go, dtype, lambda p, xr: O.rope_forward(p, xr, mask=mask, positions=pos),
                  lambda m, xd: m(xd, mask=mask, positions=pos.to(device)))


def test_layer_deterministic(device):
    x, go = _inputs(4, 512, 128, torch.bfloat16)
    m = _pom(128, 2, 2, torch.bfloat16, coeff_std=0.1).to(device)
    res = []
    for _ in range(2):
        m.zero_grad(set_to_none=True)
        xd = x.to(device).requires_grad_(True)
        out = m(xd)
        out.backward(go.to(device))
        res.append([out.detach().clone(), xd.grad.clone()] + [p.grad.clone() for p in m.parameters()])
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("mask", [None, "causal", "padding", "frames"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_heads_module(device, dtype, mask):
    """n_sel_heads = 8 through the fused layer (per-head gate kernels; in 16-bit
    training the gate part of dY^T comes from the transpose kernel)."""
    B, N, D = 2, 128, 64
    x, go = _inputs(B, N, D, dtype)
    m = _pom(D, 2, 2, dtype, coeff_std=0.1, bias=True, heads=8)
    if mask == "padding":
        mk = torch.arange(N).view(1, N) < torch.tensor([128, 37]).view(B, 1)
        omask, dmask = mk, mk.to(device)
    elif mask == "frames":
        omask, dmask = ("block_causal", 32), pom_amd.block_causal(32)
    else:
        omask = dmask = mask
    _check_module(device, m, x, go, dtype, lambda p, xr: O.pom_forward(p, xr, mask=omask),
                  lambda m, xd: m(xd, mask=dmask))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rope_2d", [False, True])
def test_heads_rope_module(device, dtype, rope_2d):
    """PoMRoPE with n_sel_heads = 8 and a padding mask: masked RoPE aggregation
    and the per-head rotated gate, fused."""
    H = W = 8
    B, N, D = 2, H * W, 64
    x, go = _inputs(B, N, D, dtype)
    mk = torch.arange(N).view(1, N) < torch.tensor([N, 23]).view(B, 1)
    if rope_2d:
        pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
        m = _rope_module(D, 2, 2, dtype, True, heads=8, max_h=H, max_w=W)
        _check_module(device, m, x, go, dtype, lambda p, xr: O.rope_forward(p, xr, mask=mk, positions_hw=pos),
                      lambda m, xd: m(xd, mask=mk.to(device), positions_hw=pos.to(device)))
    else:
        pos = torch.randperm(2 * N, generator=torch.Generator().manual_seed(4))[:N]
        m = _rope_module(D, 2, 2, dtype, False, heads=8, max_seq_len=2 * N)
        _check_module(device, m, x, go, dtype, lambda p, xr: O.rope_forward(p, xr, mask=mk, positions=pos),
                      lambda m, xd: m(xd, mask=mk.to(device), positions=pos.to(device)))
