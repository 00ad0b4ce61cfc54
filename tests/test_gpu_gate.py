"""GPU parity of the gating kernels (hardsigmoid + bias + RoPE + selection)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import pom_oracle as O
from _util import KERNEL_TOLS, ROPE_TOLS, assert_close

pytestmark = pytest.mark.gpu

import pom_amd  # noqa: E402
from pom_amd import _lib, ops  # noqa: E402


def _case(device, B, N, P, G, dtype, rope=None, bias=True, strided=True, seed=3):
    g = torch.Generator().manual_seed(seed)
    ys = (torch.randn(B, N, P, generator=g) * 2.5).to(dtype)       # spans the hardsigmoid knees
    b = (torch.randn(P, generator=g) * 0.5).to(dtype) if bias else None
    hagg = torch.randn(B, G, P, generator=g).to(dtype)
    go = torch.randn(B, N, P, generator=g).to(dtype)

    # oracle in fp64
    yr = ys.double().requires_grad_(True)
    br = b.double().requires_grad_(True) if bias else None
    hr = hagg.double().requires_grad_(True)
    s = F.hardsigmoid(yr + br) if bias else F.hardsigmoid(yr)
    if rope is not None:
        s = rope["apply"](s)
    ref = O.selection(s, hr, 1)
    ref.backward(go.double())

    if strided:
        full = torch.zeros(B, N, 2 * P, dtype=dtype)
        full[..., P:] = ys
        fd = full.to(device).requires_grad_(True)
        yin = fd[..., P:]
    else:
        fd = ys.to(device).requires_grad_(True)
        yin = fd
    bd = b.to(device).requires_grad_(True) if bias else None
    hd = hagg.to(device).requires_grad_(True)
    spec = rope["spec"](device) if rope is not None else None
    got = ops.gate_hip(yin, bd, hd, spec)
    tols = ROPE_TOLS if rope is not None else KERNEL_TOLS
    assert_close(got, ref.to(dtype), dtype, tols, "gate forward")
    got.backward(go.to(device))
    gy = fd.grad[..., P:] if strided else fd.grad
    assert_close(gy, yr.grad.to(dtype), dtype, tols, "grad y_s")
    # hagg / bias gradients are sums over tokens: compare norm-wise
    assert_close(hd.grad.float(), hr.grad.to(dtype).float(), dtype, ROPE_TOLS, "grad hagg")
    if bias:
        assert_close(bd.grad.float(), br.grad.to(dtype).float(), dtype, ROPE_TOLS, "grad bias")
    if strided:
        assert torch.all(fd.grad[..., :P] == 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,P,G", [(2, 64, 64, 1), (2, 256, 96, 1), (3, 128, 2304 // 4, 1),
                                     (2, 256, 64, 4), (2, 64, 32, 64), (1, 33, 24, 1)])
def test_gate_plain(device, B, N, P, G, dtype):
    _case(device, B, N, P, G, dtype)


def test_gate_no_bias(device):
    _case(device, 2, 128, 64, 1, torch.float32, bias=False, strided=False)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gate_rope1d(device, dtype):
    N, P = 128, 96
    fc, fs = O.precompute_freqs_1d(P, 256)
    pos = torch.arange(N) + 7
    rope = {"apply": lambda s: O.apply_rope_1d(s, pos, fc.double(), fs.double()),
            "spec": lambda dev: _lib.RopeSpec(_lib.ROPE_1D, [fc.to(dev), fs.to(dev)], pos.to(dev))}
    _case(device, 2, N, P, 1, dtype, rope=rope)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gate_rope2d(device, dtype):
    H = W = 8
    P = 128
    rc, rs, cc, cs = O.precompute_freqs_2d(P, 16, 16)
    pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
    rope = {"apply": lambda s: O.apply_rope_2d(s, pos, rc.double(), rs.double(), cc.double(), cs.double()),
            "spec": lambda dev: _lib.RopeSpec(_lib.ROPE_2D, [rc.to(dev), rs.to(dev), cc.to(dev), cs.to(dev)],
                                              pos.to(dev))}
    _case(device, 2, H * W, P, 1, dtype, rope=rope)
