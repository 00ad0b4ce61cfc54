"""GPU parity of the functional API and the less common module entry points.

  polynomial_aggregation_ (pom/pom.py:52-100) for every mask form it takes:
      None, "causal", (B, N), (B, M, N) and the block_causal(L) descriptor
  polynomial_selection_ (pom/pom.py:103-122) and pom() (:125-135) with
      n_sel_heads 1 and > 1
  PoM.ar_forward / reset (pom/pom.py:264-280) against the golden fixtures the
      reference wrote (tests/golden/make_golden.py) and the oracle
  PoMRoPE with mask="causal" (1-D and 2-D) and with block_causal(L)
      (pom/pom_rope.py:282-285, :406-416)

Each result (and its gradients) is compared with the fp64 oracle on the same
inputs: fp32 to 1e-5 norm-wise relative, bf16 to 2e-2 (the build's bar).
"""
import os

import numpy as np
import pytest
import torch

from oracle import pom_oracle as O
from _util import MODULE_GRADS, assert_rel, oracle_params, requires_grad_params

pytestmark = pytest.mark.gpu

import pom_amd  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _x(shape, dtype, seed, scale=1.0):
    return (torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale).to(dtype)


def _mask(kind, B, N):
    """(kernel-side mask, oracle-side mask) for one mask form."""
    if kind == "none":
        return None, None
    if kind == "causal":
        return "causal", "causal"
    if kind == "padding":
        lens = torch.tensor([N, N // 3, 1][:B])
        m = torch.arange(N).view(1, N) < lens.view(B, 1)
        return m, m.double()
    if kind == "dense3d":
        m = torch.rand(B, N, N, generator=torch.Generator().manual_seed(9)) < 0.4
        m |= torch.eye(N, dtype=torch.bool).unsqueeze(0)   # no empty query row
        return m, m.double()
    if kind == "block_causal":
        return pom_amd.block_causal(N // 4), ("block_causal", N // 4)
    raise AssertionError(kind)


def _dev(m, device):
    return m.to(device) if torch.is_tensor(m) else m


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["none", "causal", "padding", "dense3d", "block_causal"])
def test_polynomial_aggregation_every_mask_form(device, kind, dtype):
    B, N, P, K = 3, 64, 96, 3
    x = _x((B, N, P), dtype, 1, 0.8)
    c = _x((P, K), torch.float32, 2, 0.2)
    mk, mo = _mask(kind, B, N)
    xr, cr = x.double().requires_grad_(True), c.double().requires_grad_(True)
    ref = O.aggregate(O.poly_features(xr, cr, K), mo)
    xd, cd = x.to(device).requires_grad_(True), c.to(device).requires_grad_(True)
    got = pom_amd.polynomial_aggregation_(xd, cd, K, _dev(mk, device))
    assert got.shape == ref.shape and got.dtype == dtype
    assert_rel(got, ref, dtype, f"{kind} forward")
    go = _x(ref.shape, dtype, 3)
    ref.backward(go.double())
    got.backward(go.to(device))
    assert_rel(xd.grad, xr.grad, dtype, f"{kind} grad x")
    assert_rel(cd.grad, cr.grad, dtype, f"{kind} grad coeff")


@pytest.mark.parametrize("heads", [1, 4])
@pytest.mark.parametrize("G", [1, 16])
def test_polynomial_selection(device, heads, G):
    B, T, P = 2, 16, 64
    s = _x((B, T, P if heads == 1 else heads), torch.float32, 4)
    h = _x((B, G, P), torch.float32, 5)
    got = pom_amd.polynomial_selection_(s.to(device), h.to(device), heads)
    ref = O.selection(s.double(), h.double(), heads)
    assert got.shape == ref.shape == (B, T, P)
    assert_rel(got, ref, torch.float32, "selection")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("heads", [1, 4])
@pytest.mark.parametrize("kind", ["none", "causal", "padding", "dense3d"])
def test_pom_functional(device, kind, heads, dtype):
    """pom(s, h, coeff, k, n_sel_heads, mask): the gate first, the context second
    (pom/pom.py:125-135, called as pom(s, h, ...) at :230)."""
    B, N, P, K = 3, 64, 96, 2
    s = _x((B, N, P if heads == 1 else heads), dtype, 6, 0.5)
    h = _x((B, N, P), dtype, 7, 0.8)
    c = _x((P, K), torch.float32, 8, 0.2)
    mk, mo = _mask(kind, B, N)
    sr, hr, cr = (t.double().requires_grad_(True) for t in (s, h, c))
    ref = O.selection(sr, O.aggregate(O.poly_features(hr, cr, K), mo), heads)
    sd, hd, cd = (t.to(device).requires_grad_(True) for t in (s, h, c))
    got = pom_amd.pom(sd, hd, cd, K, heads, _dev(mk, device))
    assert got.shape == ref.shape
    assert_rel(got, ref, dtype, f"pom {kind}")
    go = _x(ref.shape, dtype, 9)
    ref.backward(go.double())
    got.backward(go.to(device))
    for a, b, n in ((sd, sr, "s"), (hd, hr, "h"), (cd, cr, "coeff")):
        assert_rel(a.grad, b.grad, dtype, f"pom {kind} grad {n}")


def _load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", ["ar_plain", "ar_heads", "ar_groups"])
def test_ar_forward_and_reset_golden(device, name):
    """PoM.ar_forward twice from a fresh state, then reset: outputs, carried h
    and 'n' against what the reference wrote (fp32)."""
    z = _load(name)
    dim, degree, expand, n_groups, heads, _ = [int(v) for v in z["meta"]]
    m = pom_amd.PoM(dim, degree, expand, n_groups, heads, False)
    with torch.no_grad():
        for n, p in m.named_parameters():
            p.copy_(torch.from_numpy(z["param." + n]).float())
    m = m.to(device)
    state = {"max_len": 64, "h": 0., "n": 0}
    out1, st1 = m.ar_forward(torch.from_numpy(z["x1"]).float().to(device), state)
    out2, st2 = m.ar_forward(torch.from_numpy(z["x2"]).float().to(device), st1)
    for got, key in ((out1, "out1"), (out2, "out2"), (st1["h"], "h1"), (st2["h"], "h2")):
        assert tuple(got.shape) == z[key].shape, key
        assert_rel(got, torch.from_numpy(z[key]), torch.float32, key, 1e-5)
    assert [st1["n"], st2["n"]] == [int(v) for v in z["n"]]
    assert st2["max_len"] == 64
    after = m.reset(st2)
    assert after is st2 and after["n"] == int(z["reset_n"]) == 0 and after["h"] == float(z["reset_h"]) == 0.0
    # the oracle's restatement agrees on the same parameters
    prm = oracle_params(m) if n_groups == 1 else None
    if prm is not None:
        ref, _ = O.ar_forward(prm, torch.from_numpy(z["x1"]), {"max_len": 64, "h": 0., "n": 0})
        assert_rel(out1, ref, torch.float32, "oracle out1", 1e-5)


@pytest.mark.parametrize("heads", [1, 4])
def test_ar_forward_bf16(device, heads):
    torch.manual_seed(0)
    m = pom_amd.PoM(64, 2, 2, 1, heads).to(device, torch.bfloat16)
    with torch.no_grad():
        m.se_bias.normal_(0, 0.5)
    x = _x((2, 16, 64), torch.bfloat16, 1)
    out, st = m.ar_forward(x.to(device), {"max_len": 16, "h": 0., "n": 5})
    ref, rst = O.ar_forward(oracle_params(m), x.double(), {"max_len": 16, "h": 0., "n": 5})
    assert st["n"] == rst["n"] == 21
    assert_rel(out, ref, torch.bfloat16, "ar out")
    assert_rel(st["h"], rst["h"], torch.bfloat16, "ar h")


def _rope_module(device, dtype, rope_2d, heads, H, W, D=32):
    torch.manual_seed(0)
    m = pom_amd.PoMRoPE(D, 2, 2, 1, heads, False, max_seq_len=H * W, max_h=H, max_w=W, rope_base=100.0,
                        rope_2d=rope_2d)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.1)
        m.se_bias.normal_(0, 0.5)
    return m.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("heads", [1, 4])
@pytest.mark.parametrize("rope_2d", [False, True])
@pytest.mark.parametrize("kind", ["causal", "block_causal"])
def test_rope_module_causal_forms(device, kind, rope_2d, heads, dtype):
    """PoMRoPE with the token-causal mask and with frame-causal frames, 1-D and
    2-D, full-width and per-head gates: output and every gradient."""
    B, H, W, D = 2, 8, 8, 32
    N = H * W
    m = _rope_module(device, dtype, rope_2d, heads, H, W, D)
    pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
    kw_o = {"positions_hw": pos} if rope_2d else {}
    kw = {"positions_hw": pos.to(device)} if rope_2d else {}
    mk, mo = _mask(kind, B, N)
    x = _x((B, N, D), dtype, 1)
    go = _x((B, N, D), dtype, 2)
    prm = requires_grad_params(oracle_params(m))
    xr = x.double().requires_grad_(True)
    ref = O.rope_forward(prm, xr, mask=mo, **kw_o)
    ref.backward(go.double())
    m = m.to(device)
    xd = x.to(device).requires_grad_(True)
    out = m(xd, mask=mk, **kw)
    out.backward(go.to(device))
    assert_rel(out, ref, dtype, f"{kind} out")
    assert_rel(xd.grad, xr.grad, dtype, f"{kind} grad x")
    params = dict(m.named_parameters())
    for oname, mname in MODULE_GRADS.items():
        t = getattr(prm, oname)
        if t is not None:
            assert_rel(params[mname].grad, t.grad, dtype, f"{kind} grad {mname}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_module_negative_positions(device, dtype):
    """1-D positions in [-rows, rows) on the host: negatives select row p + rows
    as the reference's table indexing does."""
    B, N, D = 2, 32, 32
    m = _rope_module(device, dtype, False, 1, 8, 8, D)   # 64-row table
    pos = torch.randint(-64, 64, (N,), generator=torch.Generator().manual_seed(3))
    x = _x((B, N, D), dtype, 1)
    ref = O.rope_forward(oracle_params(m), x.double(), positions=pos)
    m = m.to(device)
    assert_rel(m(x.to(device), positions=pos), ref, dtype, "host positions")
    assert_rel(m(x.to(device), positions=pos.to(device)), ref, dtype, "device positions")
    with pytest.raises(IndexError):
        m(x.to(device), positions=torch.full((N,), 64))
    with pytest.raises(IndexError):
        m(x.to(device), positions=torch.full((N,), -65))
