"""The kernels read the polynomial coefficients and the gate bias in the
parameters' own dtype and write their gradients in it (pom_* param_dtype).
A bf16 / fp16 parameter gives bit for bit the results of its fp32 copy, and
gradients equal to the fp32 gradients rounded to the parameter's dtype."""
import pytest
import torch

pytestmark = pytest.mark.gpu

from pom_amd import _lib, ops  # noqa: E402


def _rope1d(N, P, device):
    g = torch.Generator().manual_seed(5)
    fc, fs = torch.randn(N, P // 2, generator=g), torch.randn(N, P // 2, generator=g)
    return _lib.RopeSpec(_lib.ROPE_1D, [fc.to(device), fs.to(device)], torch.arange(N).to(device))


@pytest.mark.parametrize("pdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["mean", "masked", "frames", "causal", "rope"])
def test_aggregation_param_dtype(device, pdt, mode):
    g = torch.Generator().manual_seed(1)
    B, N, P, K = 2, 96, 64, 3
    x = (torch.randn(B, N, P, generator=g) * 2).to(device, torch.bfloat16)
    cp = (torch.randn(P, K, generator=g) * 0.3).to(device, pdt)
    c32 = cp.float()
    fl = {"frames": 32, "causal": 1}.get(mode, N)
    mask = count = None
    if mode == "masked":
        mask = (torch.arange(N).view(1, N) < torch.tensor([70, 33]).view(B, 1)).float().to(device)
    rope = _rope1d(N, P, device) if mode == "rope" else None
    o32, cnt = ops.agg_forward(x, c32, K, fl, mask, None, 0, rope)
    op, _ = ops.agg_forward(x, cp, K, fl, mask, None, 0, rope)
    assert torch.equal(o32, op)
    if mask is not None:
        count = cnt
    go = torch.randn(o32.shape, generator=g).to(device)
    gx32 = torch.empty_like(x)
    gxp = torch.empty_like(x)
    gc32 = ops.agg_backward(x, c32, K, fl, go, gx32, mask, count, 0, rope)
    gcp = ops.agg_backward(x, cp, K, fl, go, gxp, mask, count, 0, rope)
    assert gcp.dtype == pdt
    assert torch.equal(gx32, gxp)
    assert torch.equal(gcp, gc32.to(pdt))


@pytest.mark.parametrize("pdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("groups", [1, 4])
def test_gate_param_dtype(device, pdt, groups):
    g = torch.Generator().manual_seed(2)
    B, N, P = 2, 64, 128
    ys = (torch.randn(B, N, P, generator=g) * 2.5).to(device, torch.bfloat16)
    bp = (torch.randn(P, generator=g) * 0.5).to(device, pdt)
    b32 = bp.float()
    hagg = torch.randn(B, groups, P, generator=g).to(device, torch.bfloat16)
    assert torch.equal(ops.gate_forward(ys, b32, hagg), ops.gate_forward(ys, bp, hagg))
    gsh = torch.randn(B, N, P, generator=g).to(device, torch.bfloat16)
    d32, dp = torch.empty_like(ys), torch.empty_like(ys)
    gh32, gb32 = ops.gate_backward(ys, b32, hagg, gsh, d32)
    ghp, gbp = ops.gate_backward(ys, bp, hagg, gsh, dp)
    assert gbp.dtype == pdt
    assert torch.equal(d32, dp) and torch.equal(gh32, ghp)
    assert torch.equal(gbp, gb32.to(pdt))
