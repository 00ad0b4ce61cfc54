"""GPU parity of the per-token polynomial-feature kernels (the operand of the
dense (B, M, N) mask route, pom/pom.py:41-45 and :83-88) against the oracle
in fp64: forward, grad_x and grad_coeff, at every degree bound, with strided
and odd-width inputs."""
import pytest
import torch

from oracle import pom_oracle as O
from _util import KERNEL_TOLS, ROPE_TOLS, assert_close

pytestmark = pytest.mark.gpu

import pom_amd  # noqa: E402
from pom_amd import ops  # noqa: E402


def _case(device, B, N, P, K, dtype, strided=False, seed=11):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, N, P, generator=g) * 2.0).to(dtype)   # spans the activation's clamps
    c = (torch.randn(P, K, generator=g) * 0.3).to(dtype)
    go = torch.randn(B, N, P, generator=g).to(dtype)
    xr = x.double().requires_grad_(True)
    cr = c.double().requires_grad_(True)
    ref = O.poly_features(xr, cr, K)
    ref.backward(go.double())
    if strided:
        full = torch.zeros(B, N, 2 * P + 3, dtype=dtype)
        full[..., 3:P + 3] = x
        fd = full.to(device).requires_grad_(True)
        xin = fd[..., 3:P + 3]
    else:
        fd = x.to(device).requires_grad_(True)
        xin = fd
    cd = c.to(device).requires_grad_(True)
    got = ops.poly_features_hip(xin, cd, K)
    assert got.dtype == dtype
    assert_close(got, ref.to(dtype), dtype, KERNEL_TOLS, "features forward")
    got.backward(go.to(device))
    gx = fd.grad[..., 3:P + 3] if strided else fd.grad
    assert_close(gx, xr.grad.to(dtype), dtype, KERNEL_TOLS, "features grad_x")
    # grad_coeff sums over every token: compare at the reduction bound
    assert_close(cd.grad.float(), cr.grad.to(dtype).float(), dtype, ROPE_TOLS, "features grad_coeff")
    if strided:
        assert torch.all(fd.grad[..., :3] == 0) and torch.all(fd.grad[..., P + 3:] == 0)


@pytest.mark.parametrize("K", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_features_degrees(device, K, dtype):
    _case(device, 2, 64, 96, K, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,N,P,K", [(1, 17, 24, 2), (3, 256, 512, 3), (2, 1000, 64, 2), (2, 33, 13, 2)])
def test_features_shapes(device, B, N, P, K, dtype):
    _case(device, B, N, P, K, dtype, strided=True)


def test_dense_mask_route_uses_the_kernels(device):
    """The (B, M, N) mask route forms its features with pom_features_*."""
    seen = []
    orig = ops.poly_features_hip

    def spy(*a, **k):
        seen.append(a[2])
        return orig(*a, **k)

    ops.poly_features_hip = spy
    try:
        m = pom_amd.PoM(32, 3, 2).to(device)
        x = torch.randn(2, 12, 32, device=device)
        mask = (torch.rand(2, 12, 12, device=device) < 0.5).float()
        mask[..., 0] = 1
        m(x, mask=mask).sum().backward()
    finally:
        ops.poly_features_hip = orig
    assert seen == [3]
