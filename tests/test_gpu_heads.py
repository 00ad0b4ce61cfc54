"""GPU parity of the per-head gating kernels (n_sel_heads = H > 1):
hardsigmoid(y_s + bias) per head and token, RoPE over the H gate channels
with the reference's strided tables, selection over head_dim channels, and
their backward — against the oracle in fp64 (pom/pom.py:103-122, :207;
pom/pom_rope.py:417-437)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import pom_oracle as O
from _util import KERNEL_TOLS, ROPE_TOLS, assert_close

pytestmark = pytest.mark.gpu

import pom_amd  # noqa: E402
from pom_amd import _lib, ops  # noqa: E402


def _case(device, B, N, P, H, G, dtype, rope=None, bias=True, strided=True, seed=5):
    g = torch.Generator().manual_seed(seed)
    ys = (torch.randn(B, N, H, generator=g) * 2.5).to(dtype)       # spans the hardsigmoid knees
    b = (torch.randn(H, generator=g) * 0.5).to(dtype) if bias else None
    hagg = torch.randn(B, G, P, generator=g).to(dtype)
    go = torch.randn(B, N, P, generator=g).to(dtype)

    yr = ys.double().requires_grad_(True)
    br = b.double().requires_grad_(True) if bias else None
    hr = hagg.double().requires_grad_(True)
    s = F.hardsigmoid(yr + br) if bias else F.hardsigmoid(yr)
    if rope is not None:
        s = rope["apply"](s)
    ref = O.selection(s, hr, H)
    ref.backward(go.double())

    if strided:   # y_s as the gate slice of a projection output [h | y_s]
        full = torch.zeros(B, N, P + H, dtype=dtype)
        full[..., P:] = ys
        fd = full.to(device).requires_grad_(True)
        yin = fd[..., P:]
    else:
        fd = ys.to(device).requires_grad_(True)
        yin = fd
    bd = b.to(device).requires_grad_(True) if bias else None
    hd = hagg.to(device).requires_grad_(True)
    spec = rope["spec"](device) if rope is not None else None
    got = ops.gate_heads_hip(yin, bd, hd, H, spec)
    tols = ROPE_TOLS if rope is not None else KERNEL_TOLS
    assert_close(got, ref.to(dtype), dtype, tols, "heads gate forward")
    got.backward(go.to(device))
    gy = fd.grad[..., P:] if strided else fd.grad
    # d y_s and d bias sum over head_dim channels / tokens: compare at the RoPE bound
    assert_close(gy.float(), yr.grad.to(dtype).float(), dtype, ROPE_TOLS, "grad y_s")
    assert_close(hd.grad.float(), hr.grad.to(dtype).float(), dtype, ROPE_TOLS, "grad hagg")
    if bias:
        assert_close(bd.grad.float(), br.grad.to(dtype).float(), dtype, ROPE_TOLS, "grad bias")
    if strided:
        assert torch.all(fd.grad[..., :P] == 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,N,P,H,G", [(2, 64, 64, 4, 1), (2, 128, 576, 16, 1), (2, 96, 96, 8, 3),
                                       (2, 40, 48, 4, 40), (1, 33, 24, 3, 1), (2, 50, 36, 4, 1),
                                       (2, 30, 60, 6, 5), (2, 256, 128, 8, 2), (2, 100, 40, 5, 1),
                                       (1, 64, 200, 25, 64)])
def test_heads_plain(device, B, N, P, H, G, dtype):
    # backward paths: row walk where head_dim % 8 == 0 and groups hold many tokens (head_dim 16
    # with one or two groups, 8 with 33 and 100 tokens: partial last walks); tile path for
    # head_dim 36, 12 and single-token groups (64-channel tiles touching up to 9 heads); general
    # path for 32-token frames of head_dim 12, head_dim 9 (scalar chunks) and 10 (pairs)
    _case(device, B, N, P, H, G, dtype)


@pytest.mark.parametrize("N,P,H", [(128, 576, 16), (64, 200, 25), (40, 64, 8), (264, 2304, 16)])
def test_heads_channel_major_copy(device, N, P, H):
    """sh and its channel-major copy (P, B*N) from one launch (bf16); shapes the
    kernels do not build the copy for fall back to the transpose kernel.  Without
    the copy, head_dim 8 and 144 run the forward row walk, whose sh must equal
    the tile kernel's."""
    g = torch.Generator().manual_seed(9)
    B = 2
    ys = (torch.randn(B, N, H, generator=g) * 2).to(device, torch.bfloat16)
    hagg = torch.randn(B, 1, P, generator=g).to(device, torch.bfloat16)
    bias = torch.randn(H, generator=g).to(device, torch.bfloat16)
    sht = torch.full((P, B * N), float("nan"), device=device, dtype=torch.bfloat16)
    sh = ops.gate_heads_forward(ys, bias, hagg, H, None, out_t=sht)
    ref = ops.gate_heads_forward(ys, bias, hagg, H, None)
    assert torch.equal(sh, ref)
    assert torch.equal(sht, sh.reshape(B * N, P).t())


def test_heads_no_bias_contiguous(device):
    _case(device, 2, 64, 128, 8, 1, torch.float32, bias=False, strided=False)


def _rope1d_case(device, N, P, H, G, dtype):
    hd = P // H
    fc, fs = O.precompute_freqs_1d(P, 256)
    tc, ts = fc[:, ::hd // 2][:, :H // 2], fs[:, ::hd // 2][:, :H // 2]   # pom/pom_rope.py:417-437
    pos = torch.arange(N) + 7
    rope = {"apply": lambda s: O.apply_rope_1d(s, pos, tc.double(), ts.double()),
            "spec": lambda dev: _lib.RopeSpec(_lib.ROPE_1D, [tc.contiguous().to(dev), ts.contiguous().to(dev)],
                                              pos.to(dev))}
    _case(device, 2, N, P, H, G, dtype, rope=rope)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("G", [1, 4])
def test_heads_rope1d(device, dtype, G):
    # head_dim 12: the tile backward
    _rope1d_case(device, 128, 96, 8, G, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("G", [1, 4])
def test_heads_rope1d_row_walk(device, dtype, G):
    # head_dim 16 and groups of 32 or 128 tokens: the row-walk backward
    _rope1d_case(device, 128, 128, 8, G, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_heads_rope2d(device, dtype):
    Hh = Wh = 8
    P, H = 128, 8
    hd = P // H
    rc, rs, cc, cs = O.precompute_freqs_2d(P, 16, 16)
    tabs = [t[:, ::hd][:, :H // 4] for t in (rc, rs, cc, cs)]
    pos = torch.stack(torch.meshgrid(torch.arange(Hh), torch.arange(Wh), indexing="ij"), -1).reshape(-1, 2)
    rope = {"apply": lambda s: O.apply_rope_2d(s, pos, *[t.double() for t in tabs]),
            "spec": lambda dev: _lib.RopeSpec(_lib.ROPE_2D, [t.contiguous().to(dev) for t in tabs], pos.to(dev))}
    _case(device, 2, Hh * Wh, P, H, 1, dtype, rope=rope)


def test_heads_c2_width(device):
    """The reference benches' configuration: n_sel_heads = 16 at D = 1152,
    expand 2 (P = 2304, head_dim 144), bf16."""
    _case(device, 2, 512, 2304, 16, 1, torch.bfloat16)


@pytest.mark.parametrize("B,N,P,H,G", [(64, 1024, 64, 4, 4), (16, 1024, 256, 4, 1)])
def test_heads_row_walk_lengths(device, B, N, P, H, G):
    """Row-walk backward at batch sizes that pick 128-token walks (two per
    256-token group) and 32-token walks (the c2h batch, one group)."""
    _case(device, B, N, P, H, G, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,P,H,G", [(1, 40, 8192, 8, 1), (1, 24, 8256, 8, 1), (2, 60, 64, 4, 5)])
def test_heads_row_walk_limits(device, B, N, P, H, G, dtype):
    """The row walk at its widest row (P = 8192: 1024 threads, 64 KB of LDS), a
    row of 1032 chunks (over one workgroup: the general backward), and head_dim
    16 with 12-token groups (no walk length divides the group: the general
    backward)."""
    _case(device, B, N, P, H, G, dtype)


def test_heads_modules_use_the_kernels(device):
    """PoM / PoMRoPE with n_sel_heads > 1 gate through pom_gate_heads_* (the
    fused layer and the unfused route both call gate_heads_forward)."""
    torch.manual_seed(0)
    seen = []
    orig = ops.gate_heads_forward

    def spy(*a, **k):
        seen.append(a[3])
        return orig(*a, **k)

    ops.gate_heads_forward = spy
    try:
        m = pom_amd.PoM(32, 2, 2, 1, 8).to(device)
        m(torch.randn(2, 16, 32, device=device)).sum().backward()
        r = pom_amd.PoMRoPE(32, 2, 2, 1, 8, rope_2d=True, max_h=4, max_w=4).to(device)
        hw = torch.stack(torch.meshgrid(torch.arange(4), torch.arange(4), indexing="ij"), -1).reshape(-1, 2)
        r(torch.randn(2, 16, 32, device=device), positions_hw=hw.to(device)).sum().backward()
    finally:
        ops.gate_heads_forward = orig
    assert seen == [8, 8]
