"""End-to-end GPU parity against the golden fixtures written by the
reference's own modules (tests/golden/make_golden.py): the fixture's
parameters are loaded into a pom_amd module, the same input runs on the GPU
in fp32, and the output and every gradient are compared with the reference's.

Covers the module composition of every variant the fixtures hold: mean,
(B, N) padding mask, token-causal, dense (B, N, N) block mask, n_sel_heads = 4,
n_groups = 4, config 1 at full size, state_forward carries, and PoMRoPE 1-D /
2-D with positions, heads, causal and padding masks.
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

import pom_amd  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-4   # fp32 on the GPU vs fp32 on the reference's CPU route


def _load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _rel(a, b):
    a = torch.as_tensor(a).double().cpu()
    b = torch.as_tensor(np.asarray(b)).double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _load_params(m, z):
    with torch.no_grad():
        for name, p in m.named_parameters():
            p.copy_(torch.from_numpy(z["param." + name]).to(p.dtype))
        for name, b in m.named_buffers():
            if "buffer." + name in z:
                b.copy_(torch.from_numpy(z["buffer." + name]).to(b.dtype))


def _check(device, m, z, call):
    m = m.to(device)
    x = torch.from_numpy(z["x"]).float().to(device).requires_grad_(True)
    out = call(m, x)
    assert out.shape == z["out"].shape
    assert _rel(out, z["out"]) < TOL, f"out {_rel(out, z['out']):.3g}"
    out.backward(torch.from_numpy(z["go"]).float().to(device))
    assert _rel(x.grad, z["grad_x"]) < TOL, f"grad_x {_rel(x.grad, z['grad_x']):.3g}"
    for name, p in m.named_parameters():
        key = "grad." + name
        if key in z:
            assert _rel(p.grad, z[key]) < TOL, f"{key} {_rel(p.grad, z[key]):.3g}"


@pytest.mark.parametrize("name,mask", [("pom_mean_f32", None), ("pom_mean_k3_coeff", None),
                                       ("pom_mean_bias", None), ("pom_masked", "padding"),
                                       ("pom_causal", "causal"), ("pom_block3d", "block3d"),
                                       ("pom_heads", None), ("pom_groups", None)])
def test_golden_module(device, name, mask):
    z = _load(name)
    dim, degree, expand, n_groups, n_sel, bias = [int(v) for v in z["meta"]]
    m = pom_amd.PoM(dim, degree, expand, n_groups, n_sel, bool(bias))
    _load_params(m, z)
    if mask == "padding":
        mk = torch.from_numpy(z["mask"]).bool().to(device)
    elif mask == "block3d":
        mk = torch.from_numpy(z["mask3d"]).float().to(device)
    else:
        mk = mask
    _check(device, m, z, lambda m, x: m(x, mask=mk))
    if mask == "block3d":
        # the O(N) frame-causal descriptor gives the dense mask's result
        L = int(z["frame_len"])
        x = torch.from_numpy(z["x"]).float().to(device)
        with torch.no_grad():
            assert _rel(m(x, mask=pom_amd.block_causal(L)), z["out"]) < TOL


@pytest.mark.parametrize("name", ["rope2d", "rope2d_heads", "rope1d", "rope1d_pos", "rope1d_heads",
                                  "rope1d_causal", "rope2d_masked"])
def test_golden_rope_module(device, name):
    z = _load(name)
    dim, degree, expand, n_sel, r2d, H, W = [int(v) for v in z["meta"]]
    m = pom_amd.PoMRoPE(dim, degree, expand, 1, n_sel, False, max_seq_len=64, max_h=H + 2, max_w=W + 2,
                        rope_base=100.0, rope_2d=bool(r2d))
    _load_params(m, z)
    kw = {}
    if "positions_hw" in z:
        kw["positions_hw"] = torch.from_numpy(z["positions_hw"]).long().to(device)
    if "positions" in z:
        kw["positions"] = torch.from_numpy(z["positions"]).long().to(device)
    mask = "causal" if name.endswith("causal") else (
        torch.from_numpy(z["mask"]).bool().to(device) if "mask" in z else None)
    _check(device, m, z, lambda m, x: m(x, mask=mask, **kw))


def test_golden_c1(device):
    """Config 1 (B2 N256 D256 degree 2 expand 2 fp32, seed-0 init) against the
    reference's checksums and 4096-value samples."""
    z = _load("pom_c1")
    torch.manual_seed(0)
    m = pom_amd.PoM(256, 2, 2).to(device)
    x = torch.randn(2, 256, 256, generator=torch.Generator().manual_seed(1)).to(device).requires_grad_(True)
    out = m(x)
    go = torch.randn(out.shape, generator=torch.Generator().manual_seed(2)).to(device)
    out.backward(go)
    for key, t in [("out", out), ("grad_x", x.grad), ("grad.qc_proj.weight", m.qc_proj.weight.grad),
                   ("grad.po_coeff", m.po_coeff.grad), ("grad.ag_proj.weight", m.ag_proj.weight.grad)]:
        flat = t.detach().double().cpu().reshape(-1).numpy()
        if key + ".sample" in z:   # large arrays are stored as checksums + a strided sample
            idx, ref = z[key + ".sample_idx"], z[key + ".sample"]
            assert abs(np.linalg.norm(flat) - z[key + ".l2"]) <= TOL * z[key + ".l2"], key
        else:
            idx, ref = np.arange(flat.size), z[key].reshape(-1)
        assert np.linalg.norm(flat[idx] - ref) <= TOL * np.linalg.norm(ref), key


@pytest.mark.parametrize("name,dtype", [("state_f32", torch.float32), ("state_bf16", torch.bfloat16)])
def test_golden_state_forward(device, name, dtype):
    z = _load(name)
    dim, degree, expand, L, F = [int(v) for v in z["meta"]]
    m = pom_amd.PoM(dim, degree, expand)
    _load_params(m, z)
    m = m.to(device, dtype)
    x = torch.from_numpy(z["x"]).to(dtype).to(device)
    state = None
    with torch.no_grad():
        for f in range(F):
            o, state = m.state_forward(x[:, f * L:(f + 1) * L], state=state)
            assert state["n"] == int(z["n"][f]) and state["h"].dtype == dtype
            tol = 1e-5 if dtype == torch.float32 else 2e-2
            assert _rel(state["h"], z["h"][:, f]) < tol
            assert _rel(o, z["out"][:, f]) < tol


def test_heads_state_and_masks(device):
    """n_sel_heads > 1 through state_forward, the frame-causal descriptor and a
    random (B, M, N) cross mask, against the oracle."""
    from oracle import pom_oracle as O
    from _util import oracle_params
    torch.manual_seed(0)
    m = pom_amd.PoM(32, 2, 2, 1, 8)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.2)
        m.se_bias.normal_(0, 0.5)
    m = m.to(device)
    prm = oracle_params(m)
    x = torch.randn(2, 24, 32, generator=torch.Generator().manual_seed(1))
    xd = x.to(device)
    with torch.no_grad():
        got = m(xd, mask=pom_amd.block_causal(8))
    ref = O.pom_forward(prm, x.double(), mask=("block_causal", 8))
    assert _rel(got, ref.numpy()) < TOL
    xc = torch.randn(2, 20, 32, generator=torch.Generator().manual_seed(2))
    mask3 = (torch.rand(2, 24, 20, generator=torch.Generator().manual_seed(3)) < 0.6).float()
    mask3[..., 0] = 1
    with torch.no_grad():
        got = m(xd, xc.to(device), mask=mask3.to(device))
    ref = O.pom_forward(prm, x.double(), xc.double(), mask=mask3.double())
    assert _rel(got, ref.numpy()) < TOL
    st, so = None, None
    with torch.no_grad():
        for f in range(3):
            o, st = m.state_forward(xd[:, f * 8:(f + 1) * 8], state=st)
            r, so = O.state_forward(prm, x[:, f * 8:(f + 1) * 8].double(), state=so)
            assert _rel(o, r.numpy()) < TOL
