"""GPU tests at the baseline configurations' full sizes, and bit-exact
checks of the frame recurrence against the reference's state_forward
arithmetic evaluated by torch on the GPU.

Full sizes are checked through properties that do not depend on size
(bitwise determinism, padding independence, dense mask == mean, frame loop
== full sequence, zero positions == no rotation) and against the fp64
oracle on one batch row (rows are independent in the forward pass and in
grad_x).  The ``test_*_rows_all_grads`` tests run the module on one or two
batch rows at the configuration's full N, D, degree and expand (the real
per-row workload) and compare the output, grad_x and every parameter
gradient with the fp64 oracle on the same rows.
"""
import pytest
import torch

from oracle import pom_oracle as O
from _util import MODULE_GRADS, assert_rel, oracle_params, requires_grad_params

pytestmark = pytest.mark.gpu

import pom_amd  # noqa: E402
from pom_amd import ops  # noqa: E402


def _x(B, N, D, dtype, seed=1, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, N, D, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_frame_recurrence_bitwise_vs_torch_formula(device, dtype):
    """Full-sequence frame-causal output == the reference's state_forward
    update (pom/pom.py:255-259) run by torch on GPU tensors of `dtype`, fed the
    per-frame means of single-frame calls: identical bits."""
    B, L, F, P, K = 3, 256, 7, 384, 2
    x = _x(B, L * F, P, dtype, scale=0.7).to(device)
    c = (torch.randn(P, K, generator=torch.Generator().manual_seed(3)) * 0.2).to(device)
    full = pom_amd.poly_agg_block_causal_hip(x, c, K, L)
    means = [pom_amd.poly_agg_mean_hip(x[:, f * L:(f + 1) * L], c, K) for f in range(F)]
    h, ref = None, []
    for f, m in enumerate(means):
        if h is None:
            h, n_past = m, 0
        else:
            n_past = f
            h = (n_past * h + 1 * m) / (n_past + 1)
        ref.append(h)
    ref = torch.cat(ref, 1)
    assert full.dtype == dtype
    assert torch.equal(full, ref)
    # the chained single-frame calls with the carry give the same bits too
    carry, loop = None, []
    for f in range(F):
        hh = ops.poly_agg_state_hip(x[:, f * L:(f + 1) * L], c, K, carry, f)
        loop.append(hh)
        carry = hh
    assert torch.equal(torch.cat(loop, 1), full)


def test_state_forward_h_bitwise_equals_full_sequence(device):
    """Module level, config-4 shape in miniature: every state_forward carry
    equals the matching row of the full-sequence frame-causal aggregate."""
    B, F, L, D = 2, 5, 256, 128
    torch.manual_seed(0)
    m = pom_amd.PoM(D, 2, 4).to(device, torch.bfloat16)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.1)
    x = _x(B, F * L, D, torch.bfloat16).to(device)
    with torch.no_grad():
        _, hagg = ops.pom_layer(x, m.qc_proj.weight, m.se_bias, m.po_coeff, m.ag_proj.weight, None, 2, L)
        state = None
        for f in range(F):
            _, state = m.state_forward(x[:, f * L:(f + 1) * L], state=state)
            assert torch.equal(state["h"][:, 0], hagg[:, f]), f"frame {f}"
            assert state["n"] == f + 1


def _layer_row_check(device, m, x, go, fwd, ofwd, row=0, tol=2e-2):
    """Run the full batch on the GPU; compare output and grad_x of one batch row
    with the fp64 oracle on that row alone."""
    xd = x.to(device).requires_grad_(True)
    out = fwd(m, xd)
    out.backward(go.to(device))
    prm = oracle_params(m)
    xr = x[row:row + 1].double().requires_grad_(True)
    ref = ofwd(prm, xr)
    ref.backward(go[row:row + 1].double())
    assert_rel(out[row:row + 1], ref, x.dtype, "out row", tol)
    assert_rel(xd.grad[row:row + 1], xr.grad, x.dtype, "grad x row", tol)
    return out, xd.grad


def test_c2_full_size(device):
    """Config 2: B16 N1024 D1152 degree 2 expand 2 bf16 — oracle on one row,
    bitwise determinism over two runs."""
    torch.manual_seed(0)
    m = pom_amd.PoM(1152, 2, 2).to(device, torch.bfloat16)
    x = _x(16, 1024, 1152, torch.bfloat16)
    go = _x(16, 1024, 1152, torch.bfloat16, seed=2)
    out1, gx1 = _layer_row_check(device, m, x, go, lambda m, t: m(t), lambda p, t: O.pom_forward(p, t), row=5)
    g1 = [p.grad.clone() for p in m.parameters()]
    m.zero_grad(set_to_none=True)
    xd = x.to(device).requires_grad_(True)
    out2 = m(xd)
    out2.backward(go.to(device))
    assert torch.equal(out1, out2) and torch.equal(gx1, xd.grad)
    for a, p in zip(g1, m.parameters()):
        assert torch.equal(a, p.grad)


def test_c3_full_size_masked(device):
    """Config 3: B32 N2048 D1024 degree 3 expand 2 bf16, key-padding mask with
    valid lengths U[256, 2048]: padding noise never reaches the outputs or
    the parameter gradients; one row against the oracle."""
    B, N, D = 32, 2048, 1024
    torch.manual_seed(0)
    m = pom_amd.PoM(D, 3, 2).to(device, torch.bfloat16)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.05)
    lens = torch.randint(256, N + 1, (B,), generator=torch.Generator().manual_seed(3))
    mask = torch.arange(N).view(1, N) < lens.view(B, 1)
    x = _x(B, N, D, torch.bfloat16)
    go = _x(B, N, D, torch.bfloat16, seed=2)
    md = mask.to(device)
    row = int(torch.argmin(lens))
    _layer_row_check(device, m, x, go, lambda m, t: m(t, mask=md),
                     lambda p, t: O.pom_forward(p, t, mask=mask[row:row + 1].double()), row=row)
    # the aggregate does not see padded tokens: replace them with large noise
    h = (x.to(device).float() @ m.qc_proj.weight.float().t()).to(torch.bfloat16)[..., :2 * D]
    a = pom_amd.poly_agg_masked_hip(h, md, m.po_coeff, 3)
    h2 = h.clone()
    h2[~md] = torch.randn(int((~md).sum()), 2 * D, device=device).to(torch.bfloat16) * 100
    b = pom_amd.poly_agg_masked_hip(h2, md, m.po_coeff, 3)
    assert torch.equal(a, b)
    # dense mask == unmasked mean at this size
    ones = torch.ones(B, N, device=device)
    assert torch.equal(pom_amd.poly_agg_masked_hip(h, ones, m.po_coeff, 3),
                       pom_amd.poly_agg_masked_hip(h, ones.bool(), m.po_coeff, 3))
    d = pom_amd.poly_agg_masked_hip(h, ones, m.po_coeff, 3).float()
    e = pom_amd.poly_agg_mean_hip(h, m.po_coeff, 3).float()
    assert (d - e).abs().max().item() <= 1e-2 * e.abs().max().item()


def test_c4_full_size_block_causal(device):
    """Config 4: B4, 16 frames x 1024 tokens, D1024, degree 2, expand 4, bf16:
    the state_forward loop's carries equal the full-sequence aggregate bit for
    bit; the aggregate of one row against the oracle."""
    B, F, L, D, E = 4, 16, 1024, 1024, 4
    P = D * E
    x = _x(B, F * L, P, torch.bfloat16, scale=0.7).to(device)
    c = (torch.randn(P, 2, generator=torch.Generator().manual_seed(3)) * 0.1).to(device)
    full = pom_amd.poly_agg_block_causal_hip(x, c, 2, L)
    carry = None
    for f in range(F):
        hh = ops.poly_agg_state_hip(x[:, f * L:(f + 1) * L], c, 2, carry, f)
        assert torch.equal(hh[:, 0], full[:, f]), f"frame {f}"
        carry = hh
    ref = O.agg_block_causal(O.poly_features(x[1:2].double().cpu(), c.double().cpu(), 2), L)
    assert_rel(full[1:2], ref, torch.bfloat16, "frame means row 1", 1e-2)
    # token-causal at this length: last row == plain mean
    xc = x[:1, :4096]
    tc = pom_amd.poly_agg_causal_hip(xc, c, 2)
    assert_rel(tc[:, -1:], pom_amd.poly_agg_mean_hip(xc, c, 2), torch.bfloat16, "causal last row", 1e-2)


def test_c5_full_size_rope2d(device):
    """Config 5: B8 N4096 (64x64 grid) D1536 degree 2 expand 2 bf16, axial 2-D
    RoPE: one row against the oracle; all-zero positions == no rotation."""
    B, H, W, D = 8, 64, 64, 1536
    torch.manual_seed(0)
    m = pom_amd.PoMRoPE(D, 2, 2, 1, 1, False, max_h=H, max_w=W, rope_2d=True).to(device, torch.bfloat16)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.05)
    pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
    x = _x(B, H * W, D, torch.bfloat16)
    go = _x(B, H * W, D, torch.bfloat16, seed=2)
    pd = pos.to(device)
    _layer_row_check(device, m, x, go, lambda m, t: m(t, positions_hw=pd),
                     lambda p, t: O.rope_forward(p, t, positions_hw=pos), row=3)
    h = x.to(device)[..., :D].repeat(1, 1, 2)
    zero = torch.zeros_like(pd)
    spec = pom_amd._lib.RopeSpec(pom_amd._lib.ROPE_2D, [m.row_cos, m.row_sin, m.col_cos, m.col_sin], zero)
    a = ops.poly_agg_rope_hip(h, m.po_coeff, 2, spec)
    b = pom_amd.poly_agg_mean_hip(h, m.po_coeff, 2)
    assert_rel(a, b, torch.bfloat16, "zero positions", 1e-2)


def _rows_all_grads(device, m, x, go, fwd, ofwd, what, tol=2e-2):
    """Module on these rows vs the fp64 oracle: out, grad_x, every parameter grad."""
    prm = requires_grad_params(oracle_params(m))
    xr = x.double().requires_grad_(True)
    ref = ofwd(prm, xr)
    ref.backward(go.double())
    m.zero_grad(set_to_none=True)
    xd = x.to(device).requires_grad_(True)
    out = fwd(m, xd)
    out.backward(go.to(device))
    errs = {"out": assert_rel(out, ref, x.dtype, f"{what} out", tol),
            "x": assert_rel(xd.grad, xr.grad, x.dtype, f"{what} grad x", tol)}
    params = dict(m.named_parameters())
    for oname, mname in MODULE_GRADS.items():
        t = getattr(prm, oname)
        if t is not None:
            errs[mname] = assert_rel(params[mname].grad, t.grad, x.dtype, f"{what} grad {mname}", tol)
    print(what, {k: f"{v:.2e}" for k, v in errs.items()})
    return out


@pytest.mark.parametrize("heads", [1, 16])
def test_c2_rows_all_grads(device, heads):
    """Config 2 (B16 N1024 D1152 degree 2 expand 2 bf16) on one row; heads=16 is
    the reference benches' n_sel_heads."""
    torch.manual_seed(0)
    m = pom_amd.PoM(1152, 2, 2, 1, heads).to(device, torch.bfloat16)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.05)
        m.se_bias.normal_(0, 0.5)
    x = _x(16, 1024, 1152, torch.bfloat16)[5:6]
    go = _x(16, 1024, 1152, torch.bfloat16, seed=2)[5:6]
    _rows_all_grads(device, m, x, go, lambda m, t: m(t), lambda p, t: O.pom_forward(p, t), f"c2 heads={heads}")


def test_c3_rows_all_grads(device):
    """Config 3 (B32 N2048 D1024 degree 3 expand 2 bf16, padding mask) on its
    longest and its shortest valid row together."""
    B, N, D = 32, 2048, 1024
    torch.manual_seed(0)
    m = pom_amd.PoM(D, 3, 2).to(device, torch.bfloat16)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.05)
        m.se_bias.normal_(0, 0.5)
    lens = torch.randint(256, N + 1, (B,), generator=torch.Generator().manual_seed(3))
    rows = [int(torch.argmax(lens)), int(torch.argmin(lens))]
    mask = (torch.arange(N).view(1, N) < lens.view(B, 1))[rows]
    assert int(mask[0].sum()) > 1900 and int(mask[1].sum()) < 400
    x = _x(B, N, D, torch.bfloat16)[rows]
    go = _x(B, N, D, torch.bfloat16, seed=2)[rows]
    md = mask.to(device)
    _rows_all_grads(device, m, x, go, lambda m, t: m(t, mask=md),
                    lambda p, t: O.pom_forward(p, t, mask=mask.double()), "c3 longest+shortest")


def test_c4_rows_all_grads_block_causal(device):
    """Config 4 (16 frames x 1024 tokens, D1024, degree 2, expand 4, bf16) on one
    row: the module forward and backward with block_causal(1024) at N=16384."""
    F, L, D = 16, 1024, 1024
    torch.manual_seed(0)
    m = pom_amd.PoM(D, 2, 4).to(device, torch.bfloat16)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.05)
        m.se_bias.normal_(0, 0.5)
    x = _x(1, F * L, D, torch.bfloat16)
    go = _x(1, F * L, D, torch.bfloat16, seed=2)
    _rows_all_grads(device, m, x, go, lambda m, t: m(t, mask=pom_amd.block_causal(L)),
                    lambda p, t: O.pom_forward(p, t, mask=("block_causal", L)), "c4 block-causal")


def test_c4_state_forward_loop_outputs_equal_full_pass(device):
    """Config 4 at full size (B4, 16 frames x 1024 tokens): the module's 16-call
    state_forward loop gives the full block-causal pass's outputs frame by
    frame (carries bit for bit; outputs up to the projections' accumulation
    order, the GEMM shapes differ)."""
    B, F, L, D = 4, 16, 1024, 1024
    torch.manual_seed(0)
    m = pom_amd.PoM(D, 2, 4).to(device, torch.bfloat16)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.05)
        m.se_bias.normal_(0, 0.5)
    x = _x(B, F * L, D, torch.bfloat16).to(device)
    with torch.no_grad():
        full = m(x, mask=pom_amd.block_causal(L))
        _, hagg = ops.pom_layer(x, m.qc_proj.weight, m.se_bias, m.po_coeff, m.ag_proj.weight, None, 2, L)
        state, worst = None, 0.0
        for f in range(F):
            out, state = m.state_forward(x[:, f * L:(f + 1) * L], state=state)
            assert state["n"] == f + 1
            assert torch.equal(state["h"][:, 0], hagg[:, f]), f"carry of frame {f}"
            worst = max(worst, assert_rel(out, full[:, f * L:(f + 1) * L], torch.bfloat16, f"frame {f}", 1e-2))
    print(f"c4 loop vs full: worst frame rel {worst:.2e}")


def test_c5_rows_all_grads_rope2d(device):
    """Config 5 (B8 N4096 on a 64x64 grid, D1536, degree 2, expand 2, bf16,
    axial 2-D RoPE) on one row."""
    H, W, D = 64, 64, 1536
    torch.manual_seed(0)
    m = pom_amd.PoMRoPE(D, 2, 2, 1, 1, False, max_h=H, max_w=W, rope_2d=True).to(device, torch.bfloat16)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.05)
        m.se_bias.normal_(0, 0.5)
    pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
    x = _x(8, H * W, D, torch.bfloat16)[3:4]
    go = _x(8, H * W, D, torch.bfloat16, seed=2)[3:4]
    pd = pos.to(device)
    _rows_all_grads(device, m, x, go, lambda m, t: m(t, positions_hw=pd),
                    lambda p, t: O.rope_forward(p, t, positions_hw=pos), "c5 rope2d")
