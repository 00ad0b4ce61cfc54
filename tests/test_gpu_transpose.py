"""pom_transpose (the HIP operand-layout kernel) against torch's transpose:
bit-exact for every dtype, on tile-aligned, ragged, strided and unaligned
operands."""
import pytest
import torch

pytestmark = pytest.mark.gpu

from pom_amd import ops  # noqa: E402


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(64, 64), (16384, 1152), (1024, 2304), (1, 8), (8, 1), (7, 13), (200, 72),
                                   (129, 257)])
def test_transpose_matches_torch(device, dtype, shape):
    g = torch.Generator(device="cpu").manual_seed(shape[0] * 7 + shape[1])
    x = torch.randn(shape, generator=g).to(device, dtype)
    got = ops.transpose(x)
    assert got.shape == (shape[1], shape[0]) and got.is_contiguous()
    assert torch.equal(got, x.t().contiguous())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_transpose_strided_half(device, dtype):
    # the s-half of a fused projection output: row stride 2P
    y = torch.randn(300, 2 * 136).to(device, dtype)
    s = y[:, 136:]
    assert torch.equal(ops.transpose(s), s.t().contiguous())


def test_transpose_unaligned_uses_element_path(device):
    base = torch.randn(50 * 33 + 1).to(device, torch.bfloat16)
    x = base[1:].view(50, 33)   # 2-byte offset: not 16-byte aligned
    assert torch.equal(ops.transpose(x), x.t().contiguous())


def test_transpose_repeated_calls_identical(device):
    x = torch.randn(4096, 1152).to(device, torch.bfloat16)
    a = ops.transpose(x)
    b = ops.transpose(x)
    assert torch.equal(a, b)
