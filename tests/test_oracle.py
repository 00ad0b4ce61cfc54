"""CPU tests that pin the oracle (oracle/pom_oracle.py) before it is trusted.

Three kinds of checks, chosen so that a dropped term, a wrong sign or index or
a transposed operand fails at least one:
  * golden fixtures written by the reference's own modules
    (tests/golden/make_golden.py): module composition, init order, state
    carry, RoPE conventions, masks, multi-head gating, grouped projection;
  * brute-force Python loops on tiny inputs and closed forms
    (activation points, polynomial, every aggregation, rotations);
  * invariants the mathematics fixes (dense mask == mean, causal last row ==
    mean, frame_len N == mean, frame_len 1 == causal, frame loop == full
    block-causal, rotation orthogonality) and fp64 gradchecks.
"""
import glob
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import pom_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _t(a):
    return torch.from_numpy(np.asarray(a)).double()


def _params_from(z, rope=None):
    meta = [int(v) for v in z["meta"]]
    dim, degree, expand, n_groups, n_sel, bias = meta[:6] if len(meta) >= 6 else meta + [0] * (6 - len(meta))
    g = lambda k: _t(z[k]) if k in z else None
    if n_groups > 1:
        return O.OracleParams(dim, degree, expand, n_sel, None, None, g("param.po_coeff"),
                              g("param.ag_proj.weight"), g("param.ag_proj.bias"), rope, n_groups,
                              g("param.po_proj.weight"), g("param.po_proj.bias"),
                              g("param.se_proj.weight"), g("param.se_proj.bias"))
    return O.OracleParams(dim, degree, expand, n_sel, g("param.qc_proj.weight"), g("param.se_bias"),
                          g("param.po_coeff"), g("param.ag_proj.weight"), g("param.ag_proj.bias"), rope)


def _rel(a, b):
    a, b = torch.as_tensor(a).double(), torch.as_tensor(b).double()
    nb = b.norm().item()
    return (a - b).norm().item() / (nb if nb else 1.0)


GRAD_KEYS = [("w_qc", "grad.qc_proj.weight"), ("se_bias", "grad.se_bias"), ("po_coeff", "grad.po_coeff"),
             ("w_ag", "grad.ag_proj.weight"), ("b_ag", "grad.ag_proj.bias"), ("po_w", "grad.po_proj.weight"),
             ("po_b", "grad.po_proj.bias"), ("se_w", "grad.se_proj.weight"), ("se_b", "grad.se_proj.bias")]


def _check_grads(prm, z, tol=1e-5):
    for attr, key in GRAD_KEYS:
        t = getattr(prm, attr)
        if t is None or key not in z:
            continue
        assert _rel(t.grad, z[key]) < tol, f"{key}: rel {_rel(t.grad, z[key]):.3g}"


def _requires_grad(prm):
    for attr, _ in GRAD_KEYS:
        t = getattr(prm, attr)
        if t is not None:
            t.requires_grad_(True)
    return prm


# ---------------------------------------------------------------------------
# Golden fixtures from the reference modules
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name,mask", [("pom_mean_f32", None), ("pom_mean_k3_coeff", None),
                                       ("pom_mean_bias", None), ("pom_masked", "padding"),
                                       ("pom_causal", "causal"), ("pom_block3d", "block3d"),
                                       ("pom_heads", None), ("pom_groups", None)])
def test_golden_pom(name, mask):
    z = _load(name)
    prm = _requires_grad(_params_from(z))
    x = _t(z["x"]).requires_grad_(True)
    m = None
    if mask == "padding":
        m = _t(z["mask"])
    elif mask == "causal":
        m = "causal"
    elif mask == "block3d":
        m = _t(z["mask3d"])
    out = O.pom_forward(prm, x, mask=m)
    assert out.shape == z["out"].shape
    assert _rel(out, z["out"]) < 1e-5, _rel(out, z["out"])
    out.backward(_t(z["go"]))
    assert _rel(x.grad, z["grad_x"]) < 1e-5
    _check_grads(prm, z)


def test_golden_block3d_equals_compact():
    """The reference's dense block-lower-triangular 3-D mask == the compact
    frame-causal mean expanded per frame."""
    z = _load("pom_block3d")
    prm = _params_from(z)
    L = int(z["frame_len"])
    out = O.pom_forward(prm, _t(z["x"]), mask=("block_causal", L))
    assert _rel(out, z["out"]) < 1e-6


def test_golden_c1_checksums():
    """Config 1 (B2 N256 D256 degree 2 expand 2 fp32), parameters drawn by the
    oracle's init_params from torch.manual_seed(0) in the reference's order."""
    z = _load("pom_c1")
    torch.manual_seed(0)
    prm = _requires_grad(O.init_params(256, 2, 2).to(torch.float64))
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 256, 256, generator=g).double().requires_grad_(True)
    out = O.pom_forward(prm, x)
    go = torch.randn(out.shape, generator=torch.Generator().manual_seed(2)).double()
    out.backward(go)
    for key, t in [("out", out), ("grad_x", x.grad), ("grad.qc_proj.weight", prm.w_qc.grad),
                   ("grad.po_coeff", prm.po_coeff.grad), ("grad.ag_proj.weight", prm.w_ag.grad),
                   ("param.qc_proj.weight", prm.w_qc), ("param.ag_proj.weight", prm.w_ag)]:
        # the reference ran in fp32, the oracle in fp64: elementwise bound
        # relative to the array's scale
        flat = t.detach().reshape(-1).numpy()
        if key + ".sample" in z:
            idx = z[key + ".sample_idx"]
            ref = z[key + ".sample"]
            assert abs(np.sqrt((flat * flat).sum()) - z[key + ".l2"]) <= 1e-5 * z[key + ".l2"], key
        else:
            idx = np.arange(flat.size)
            ref = z[key].reshape(-1)
        np.testing.assert_allclose(flat[idx], ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max(), err_msg=key)
    # se_bias starts at zero, po_coeff saturates to +-1e-3 almost everywhere
    assert torch.all(prm.se_bias == 0)
    sat = prm.po_coeff.detach().float().abs() == torch.tensor(1e-3, dtype=torch.float32)
    assert sat.float().mean() > 0.99


@pytest.mark.parametrize("name,dtype", [("state_f32", torch.float32), ("state_bf16", torch.bfloat16)])
def test_golden_state_forward(name, dtype):
    """'n' counts calls and 'h' is the running mean of per-call means, kept in
    the input dtype (pom/pom.py:252-262)."""
    z = _load(name)
    dim, degree, expand, L, F_ = [int(v) for v in z["meta"]]
    prm = O.OracleParams(dim, degree, expand, 1, _t(z["param.qc_proj.weight"]).to(dtype),
                         _t(z["param.se_bias"]).to(dtype), _t(z["param.po_coeff"]).to(dtype),
                         _t(z["param.ag_proj.weight"]).to(dtype), None)
    x = _t(z["x"]).to(dtype)
    state = None
    for f in range(F_):
        xf = x[:, f * L:(f + 1) * L]
        out, state = O.state_forward(prm, xf, xf, state)
        assert state["n"] == z["n"][f] == f + 1
        assert state["h"].dtype == dtype
        if dtype == torch.float32:
            assert _rel(state["h"], z["h"][:, f]) < 1e-6
            assert _rel(out, z["out"][:, f]) < 1e-6
        else:
            # same torch ops on the same bf16 tensors
            assert torch.equal(state["h"].double(), _t(z["h"][:, f]))
            assert _rel(out, z["out"][:, f]) < 1e-2


@pytest.mark.parametrize("name", ["rope2d", "rope2d_heads", "rope1d", "rope1d_pos", "rope1d_heads",
                                  "rope1d_causal", "rope2d_masked"])
def test_golden_rope(name):
    z = _load(name)
    dim, degree, expand, n_sel, r2d, H, W = [int(v) for v in z["meta"]]
    if r2d:
        rope = {"rope_2d": True, "row_cos": _t(z["buffer.row_cos"]), "row_sin": _t(z["buffer.row_sin"]),
                "col_cos": _t(z["buffer.col_cos"]), "col_sin": _t(z["buffer.col_sin"])}
    else:
        rope = {"rope_2d": False, "freqs_cos": _t(z["buffer.freqs_cos"]), "freqs_sin": _t(z["buffer.freqs_sin"])}
    prm = _requires_grad(O.OracleParams(dim, degree, expand, n_sel, _t(z["param.qc_proj.weight"]),
                                        _t(z["param.se_bias"]), _t(z["param.po_coeff"]),
                                        _t(z["param.ag_proj.weight"]), None, rope))
    kw = {}
    if "positions_hw" in z:
        kw["positions_hw"] = torch.from_numpy(z["positions_hw"]).long()
    if "positions" in z:
        kw["positions"] = torch.from_numpy(z["positions"]).long()
    mask = "causal" if name.endswith("causal") else (_t(z["mask"]) if "mask" in z else None)
    x = _t(z["x"]).requires_grad_(True)
    out = O.rope_forward(prm, x, mask=mask, **kw)
    assert _rel(out, z["out"]) < 1e-5
    out.backward(_t(z["go"]))
    assert _rel(x.grad, z["grad_x"]) < 1e-5
    _check_grads(prm, z)
    # the oracle's own tables equal the reference's buffers
    P = dim * expand
    if r2d:
        rc, rs, cc, cs = O.precompute_freqs_2d(P, H + 2, W + 2, 100.0)
        assert torch.allclose(rc.double(), rope["row_cos"]) and torch.allclose(cs.double(), rope["col_sin"])
    else:
        fc, fs = O.precompute_freqs_1d(P, 64, 100.0)
        assert torch.allclose(fc.double(), rope["freqs_cos"]) and torch.allclose(fs.double(), rope["freqs_sin"])


@pytest.mark.parametrize("name", ["ar_plain", "ar_heads", "ar_groups"])
def test_golden_ar_forward(name):
    """PoM.ar_forward twice, then reset (pom/pom.py:264-280)."""
    z = _load(name)
    prm = _params_from(z)
    state = {"max_len": 64, "h": 0., "n": 0}
    out1, st1 = O.ar_forward(prm, _t(z["x1"]), state)
    out2, st2 = O.ar_forward(prm, _t(z["x2"]), st1)
    assert _rel(out1, z["out1"]) < 1e-6 and _rel(out2, z["out2"]) < 1e-6
    assert _rel(st1["h"], z["h1"]) < 1e-6 and _rel(st2["h"], z["h2"]) < 1e-6
    assert [st1["n"], st2["n"]] == [int(v) for v in z["n"]] == [8, 16]
    assert st2["max_len"] == 64
    assert int(z["reset_n"]) == 0 and float(z["reset_h"]) == 0.0


def test_golden_files_all_used():
    names = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "*.npz")))
    assert len(names) == 21, names


# ---------------------------------------------------------------------------
# Closed forms and brute force
# ---------------------------------------------------------------------------

def test_activation_points():
    x = torch.tensor([-20.0, -10.0, -5.0, -0.5, 0.0, 0.5, 3.0, 6.0, 7.0], dtype=torch.float64)
    want = torch.tensor([-0.1, -0.1, -0.05, -0.005, 0.0, 0.5, 3.0, 6.0, 6.0], dtype=torch.float64)
    assert torch.allclose(O.activation(x), want)
    # torch autograd conventions the kernels follow: slope 0.01 at x == 0,
    # clamp passes the gradient on its closed bounds
    xr = x.clone().requires_grad_(True)
    O.activation(xr).sum().backward()
    g = torch.tensor([0.0, 0.01, 0.01, 0.01, 0.01, 1.0, 1.0, 1.0, 0.0], dtype=torch.float64)
    assert torch.allclose(xr.grad, g), xr.grad


def test_hardsigmoid_points():
    z = torch.tensor([-4.0, -3.0, 0.0, 1.5, 3.0, 4.0], dtype=torch.float64, requires_grad=True)
    s = O.hardsigmoid(z)
    assert torch.allclose(s, torch.tensor([0.0, 0.0, 0.5, 0.75, 1.0, 1.0], dtype=torch.float64))
    s.sum().backward()
    assert torch.allclose(z.grad, torch.tensor([0, 0, 1 / 6, 1 / 6, 0, 0], dtype=torch.float64))


def _brute_poly(x, c, k):
    B, N, D = x.shape
    out = torch.zeros(B, N, D, dtype=torch.float64)
    for b in range(B):
        for n in range(N):
            for d in range(D):
                v = float(x[b, n, d])
                h = min(max(v if v > 0 else 0.01 * v, -0.1), 6.0)
                out[b, n, d] = sum(float(c[d, j]) * h ** (j + 1) for j in range(k))
    return out


@pytest.mark.parametrize("k", [1, 2, 3, 5])
def test_poly_features_brute(k):
    g = torch.Generator().manual_seed(k)
    x = torch.randn(2, 5, 3, generator=g, dtype=torch.float64) * 3
    c = torch.randn(3, k, generator=g, dtype=torch.float64)
    assert torch.allclose(O.poly_features(x, c, k), _brute_poly(x, c, k))


def test_aggregations_brute():
    g = torch.Generator().manual_seed(3)
    B, N, D, L = 2, 12, 3, 4
    h = torch.randn(B, N, D, generator=g, dtype=torch.float64)
    m = (torch.rand(B, N, generator=g) < 0.5).double()
    m[:, 0] = 1
    mean = torch.stack([sum(h[:, n] for n in range(N)) / N], 1)
    assert torch.allclose(O.agg_mean(h), mean)
    masked = torch.stack([sum(m[:, n, None] * h[:, n] for n in range(N)) / m.sum(1, keepdim=True)], 1)
    assert torch.allclose(O.agg_masked(h, m), masked)
    causal = torch.stack([sum(h[:, j] for j in range(n + 1)) / (n + 1) for n in range(N)], 1)
    assert torch.allclose(O.agg_causal(h), causal)
    block = torch.stack([sum(h[:, j] for j in range((f + 1) * L)) / ((f + 1) * L) for f in range(N // L)], 1)
    assert torch.allclose(O.agg_block_causal(h, L), block)
    # invariants
    assert torch.allclose(O.agg_masked(h, torch.ones(B, N, dtype=torch.float64)), O.agg_mean(h))
    assert torch.allclose(O.agg_causal(h)[:, -1:], O.agg_mean(h))
    assert torch.allclose(O.agg_block_causal(h, N), O.agg_mean(h))
    assert torch.allclose(O.agg_block_causal(h, 1), O.agg_causal(h))
    dense = O.block_causal_dense_mask(B, N, L, torch.float64)
    assert torch.allclose(O.agg_full_mask(h, dense), O.agg_block_causal(h, L).repeat_interleave(L, 1))
    tril = torch.tril(torch.ones(N, N, dtype=torch.float64)).expand(B, N, N)
    assert torch.allclose(O.agg_full_mask(h, tril), O.agg_causal(h))


def test_masked_empty_row_conventions():
    h = torch.randn(2, 5, 3, dtype=torch.float64)
    m = torch.ones(2, 5, dtype=torch.float64)
    m[1] = 0
    assert torch.all(O.agg_masked(h, m)[1] == 0)                          # GPU kernels' convention
    assert torch.isnan(O.agg_masked(h, m, empty_is_zero=False)[1]).all()   # CPU fallback's 0/0


def test_frame_loop_equals_block_causal():
    """state_forward's recurrence over equal frames == the full frame-causal mean (fp64)."""
    g = torch.Generator().manual_seed(4)
    B, L, Fn, D = 2, 6, 5, 4
    h = torch.randn(B, L * Fn, D, generator=g, dtype=torch.float64)
    full = O.agg_block_causal(h, L)
    means = h.view(B, Fn, L, D).mean(2)
    loop = O.running_mean_frames(means, torch.float64)
    assert torch.allclose(loop, full)
    # carry continuation: frames [0, 2) then [2, 5) with n_past = 2
    head = O.running_mean_frames(means[:, :2], torch.float64)
    tail = O.running_mean_frames(means[:, 2:], torch.float64, carry=head[:, -1], n_past=2)
    assert torch.allclose(torch.cat([head, tail], 1), full)


def test_running_mean_rounding_matches_reference_formula():
    """running_mean_frames on bf16 == the reference's expression evaluated by
    torch on bf16 CPU tensors, up to CPU's true division (the GPU kernels
    multiply by the fp32 reciprocal): at most one bf16 ulp apart, rarely."""
    g = torch.Generator().manual_seed(5)
    means = torch.randn(4, 12, 256, generator=g)
    emu = O.running_mean_frames(means, torch.bfloat16)
    h = means[:, 0].to(torch.bfloat16)
    ref = [h]
    for f in range(1, 12):
        h = (f * h + 1 * means[:, f].to(torch.bfloat16)) / (f + 1)
        ref.append(h)
    ref = torch.stack(ref, 1)
    diff = (emu.float() - ref.float()).abs()
    ulp = ref.float().abs() * 2.0 ** -7 + 1e-30
    assert torch.all(diff <= ulp)
    assert (diff == 0).float().mean() > 0.98


def test_rope_closed_form():
    P, S = 8, 10
    fc, fs = O.precompute_freqs_1d(P, S, 10000.0)
    # theta_i = 10000^(-i / (P/2)); table[n, i] = cos / sin(n theta_i)
    for n in (0, 3, 9):
        for i in range(P // 2):
            th = n * 10000.0 ** (-i / (P // 2))
            assert abs(fc[n, i].item() - math.cos(th)) < 1e-6 and abs(fs[n, i].item() - math.sin(th)) < 1e-6
    x = torch.randn(1, S, P, dtype=torch.float64)
    pos = torch.arange(S)
    r = O.apply_rope_1d(x, pos, fc.double(), fs.double())
    # pair (i, i + P/2) rotates by +theta: [a cos - b sin, b cos + a sin]
    a, b = x[0, 3, 1].item(), x[0, 3, 1 + P // 2].item()
    th = 3 * 10000.0 ** (-1 / (P // 2))
    assert abs(r[0, 3, 1].item() - (a * math.cos(th) - b * math.sin(th))) < 1e-6
    assert abs(r[0, 3, 1 + P // 2].item() - (b * math.cos(th) + a * math.sin(th))) < 1e-6
    # position 0 is the identity; pair norms are preserved
    assert torch.allclose(O.apply_rope_1d(x, torch.zeros(S, dtype=torch.long), fc.double(), fs.double()), x)
    n1 = x[..., :P // 2] ** 2 + x[..., P // 2:] ** 2
    n2 = r[..., :P // 2] ** 2 + r[..., P // 2:] ** 2
    assert torch.allclose(n1, n2)


def test_rope2d_quarters():
    P, H, W = 16, 3, 4
    rc, rs, cc, cs = [t.double() for t in O.precompute_freqs_2d(P, H, W, 10000.0)]
    pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
    x = torch.randn(1, H * W, P, dtype=torch.float64)
    r = O.apply_rope_2d(x, pos, rc, rs, cc, cs)
    q = P // 4
    n = 7   # row 1, column 3
    i = 2
    th_r = 1 * 10000.0 ** (-i / q)
    th_c = 3 * 10000.0 ** (-i / q)
    a, b = x[0, n, i].item(), x[0, n, q + i].item()
    assert abs(r[0, n, i].item() - (a * math.cos(th_r) - b * math.sin(th_r))) < 1e-6
    c1, c2 = x[0, n, 2 * q + i].item(), x[0, n, 3 * q + i].item()
    assert abs(r[0, n, 3 * q + i].item() - (c2 * math.cos(th_c) + c1 * math.sin(th_c))) < 1e-6
    zero = torch.zeros(H * W, 2, dtype=torch.long)
    assert torch.allclose(O.apply_rope_2d(x, zero, rc, rs, cc, cs), x)


def test_gradcheck_composition():
    torch.manual_seed(0)
    prm = O.init_params(6, 3, 2).to(torch.float64)
    with torch.no_grad():
        prm.po_coeff.normal_(0, 0.3)
        prm.se_bias.normal_(0, 0.5)
    x = (torch.randn(2, 5, 6, dtype=torch.float64) * 2).requires_grad_(True)
    for mask in (None, "causal", ("block_causal", 1)):
        assert torch.autograd.gradcheck(lambda t: O.pom_forward(prm, t, mask=mask), (x,), eps=1e-6, atol=1e-5)
