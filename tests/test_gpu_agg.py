"""GPU parity of the aggregation kernels against the CPU oracle.

Protocol of the reference's kernel tests (test_triton_correctness.py:98-216):
x = randn * 0.5, coeff = randn * 0.1 from seed 42; upstream gradient from
seed 7, round-tripped through the tensor dtype; masks from seed 99 with the
first token kept.  The oracle runs in fp64 on the dtype-quantised inputs.
"""
import itertools

import pytest
import torch

from oracle import pom_oracle as O
from _util import KERNEL_TOLS, ROPE_TOLS, assert_close, assert_rel

pytestmark = pytest.mark.gpu

import pom_amd  # noqa: E402
from pom_amd import ops  # noqa: E402


def make_inputs(B, N, D, K, dtype, strided=False, seed=42):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, N, D, generator=g) * 0.5).to(dtype)
    coeff = (torch.randn(D, K, generator=g) * 0.1).to(dtype)
    if strided:
        # the aggregation input is the h-half of the fused projection (B, N, 2D)
        full = torch.zeros(B, N, 2 * D, dtype=dtype)
        full[..., :D] = x
        full[..., D:] = (torch.randn(B, N, D, generator=g)).to(dtype)
        return full, x, coeff
    return None, x, coeff


def to_dev(t, device):
    return None if t is None else t.to(device)


def run_case(device, B, N, D, K, dtype, kind, strided=False, frame_len=None, keep=0.5, rope=None):
    full, x, coeff = make_inputs(B, N, D, K, dtype, strided)
    xd_full = to_dev(full, device)
    xd = xd_full[..., :D] if strided else x.to(device)
    xd = xd.detach().requires_grad_(True) if not strided else xd
    cd = coeff.to(device).detach().requires_grad_(True)
    mask = None
    if kind == "masked":
        gm = torch.Generator().manual_seed(99)
        mask = (torch.rand(B, N, generator=gm) < keep).float()
        mask[:, 0] = 1.0

    # oracle, fp64 on the quantised inputs
    xr = x.double().requires_grad_(True)
    cr = coeff.double().requires_grad_(True)
    h = O.poly_features(xr, cr, K)
    if rope is not None:
        h = rope["apply"](h)
    if kind == "mean":
        ref = O.agg_mean(h)
    elif kind == "masked":
        ref = O.agg_masked(h, mask.double())
    elif kind == "block":
        ref = O.agg_block_causal(h, frame_len)
    elif kind == "causal":
        ref = O.agg_causal(h)
    else:
        raise AssertionError(kind)

    if strided:
        xd_leaf = xd_full.detach().requires_grad_(True)
        xin = xd_leaf[..., :D]
    else:
        xd_leaf = xd
        xin = xd
    if rope is not None and kind == "masked":
        got = ops.poly_agg_masked_hip(xin, mask.to(device), cd, K, rope["spec"](device))
    elif rope is not None:
        spec = rope["spec"](device)
        fl = N if kind == "mean" else (1 if kind == "causal" else frame_len)
        got = ops.poly_agg_rope_hip(xin, cd, K, spec, fl)
    elif kind == "mean":
        got = pom_amd.poly_agg_mean_hip(xin, cd, K)
    elif kind == "masked":
        got = pom_amd.poly_agg_masked_hip(xin, mask.to(device).bool() if keep in (0.0, 1.0) else mask.to(device),
                                          cd, K)
    elif kind == "block":
        got = pom_amd.poly_agg_block_causal_hip(xin, cd, K, frame_len)
    else:
        got = pom_amd.poly_agg_causal_hip(xin, cd, K)
    assert got.dtype == dtype
    # frame outputs carry a per-frame rounding (the state_forward recurrence)
    tols = ROPE_TOLS if (rope is not None or kind == "block") and dtype != torch.float32 else KERNEL_TOLS
    assert_close(got, ref.to(dtype), dtype, tols, f"forward {kind}")

    gg = torch.Generator().manual_seed(7)
    go = torch.randn(ref.shape, generator=gg).to(dtype)
    ref.backward(go.double())
    got.backward(go.to(device))
    gx = xd_leaf.grad[..., :D] if strided else xd_leaf.grad
    assert_close(gx, xr.grad.to(dtype), dtype, tols, f"grad_x {kind}")
    assert_close(cd.grad.float(), cr.grad, dtype, tols, f"grad_coeff {kind}")
    if strided:
        assert torch.all(xd_leaf.grad[..., D:] == 0), "grad leaked into the other half"


GRID_F32 = list(itertools.product([1, 4], [16, 256, 1024], [32, 96, 512], [1, 2, 3, 4, 8, 16]))
GRID_BF16 = list(itertools.product([2], [64, 512], [64, 128], [2, 4]))


@pytest.mark.parametrize("B,N,D,K", GRID_F32)
def test_mean_f32(device, B, N, D, K):
    run_case(device, B, N, D, K, torch.float32, "mean")


@pytest.mark.parametrize("B,N,D,K", GRID_BF16)
def test_mean_bf16(device, B, N, D, K):
    run_case(device, B, N, D, K, torch.bfloat16, "mean")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,N,D,K", [(2, 1024, 2304 // 8, 2), (3, 200, 72, 3), (2, 64, 12, 2)])
def test_mean_strided(device, B, N, D, K, dtype):
    run_case(device, B, N, D, K, dtype, "mean", strided=True)


@pytest.mark.parametrize("keep", [1.0, 0.5, 0.25])
@pytest.mark.parametrize("B,N,D,K", [(1, 16, 32, 1), (4, 256, 96, 3), (4, 1024, 512, 2), (2, 64, 128, 16)])
def test_masked_f32(device, B, N, D, K, keep):
    run_case(device, B, N, D, K, torch.float32, "masked", keep=keep)


@pytest.mark.parametrize("B,N,D,K", GRID_BF16)
def test_masked_bf16(device, B, N, D, K):
    run_case(device, B, N, D, K, torch.bfloat16, "masked", strided=True)


def test_masked_dense_equals_mean(device):
    """Dense mask == unmasked mean (test_triton_masked_correctness.py:195-199)."""
    _, x, c = make_inputs(2, 256, 64, 2, torch.float32)
    xd, cd = x.to(device), c.to(device)
    m = torch.ones(2, 256, device=device)
    a = pom_amd.poly_agg_masked_hip(xd, m, cd, 2)
    b = pom_amd.poly_agg_mean_hip(xd, cd, 2)
    assert (a - b).abs().max().item() <= 1e-6


def test_masked_empty_row_is_zero(device):
    """An all-zero mask row aggregates to 0 (pom/pom_triton_masked.py:165-167)."""
    _, x, c = make_inputs(3, 128, 64, 2, torch.float32)
    m = torch.ones(3, 128)
    m[1] = 0
    out = pom_amd.poly_agg_masked_hip(x.to(device), m.to(device), c.to(device), 2)
    assert torch.all(out[1] == 0)
    assert torch.isfinite(out).all()


def test_masked_padding_noise_ignored(device):
    """Padded tokens never affect the output (config 3's contract)."""
    B, N, D = 4, 512, 128
    _, x, c = make_inputs(B, N, D, 3, torch.bfloat16)
    L = torch.tensor([100, 512, 256, 1])
    m = (torch.arange(N).view(1, N) < L.view(B, 1)).float()
    x2 = x.clone()
    x2[m == 0] = torch.randn(int((m == 0).sum()), D).to(torch.bfloat16) * 50
    a = pom_amd.poly_agg_masked_hip(x.to(device), m.to(device), c.to(device), 3)
    b = pom_amd.poly_agg_masked_hip(x2.to(device), m.to(device), c.to(device), 3)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,D,K,L", [(2, 256, 64, 2, 64), (2, 1024, 96, 3, 128), (1, 512, 32, 2, 512),
                                       (3, 96, 32, 2, 32), (2, 64, 16, 4, 8)])
def test_block_causal(device, B, N, D, K, L, dtype):
    run_case(device, B, N, D, K, dtype, "block", frame_len=L, strided=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,D,K", [(1, 16, 32, 2), (2, 64, 64, 3), (2, 256, 96, 2)])
def test_causal(device, B, N, D, K, dtype):
    run_case(device, B, N, D, K, dtype, "causal")


def _rope1d(D, N, seed=5, random_pos=False, negative=False):
    fc, fs = O.precompute_freqs_1d(D, 4 * N)
    if negative:
        # positions in [-rows, rows): torch's indexing of the tables wraps the
        # negative ones to p + rows (pom/pom_rope.py:173-174), so must the kernels
        pos = torch.randint(-4 * N, 4 * N, (N,), generator=torch.Generator().manual_seed(seed))
        pos[0], pos[-1] = -4 * N, -1
    elif random_pos:
        pos = torch.randperm(4 * N, generator=torch.Generator().manual_seed(seed))[:N]
    else:
        pos = torch.arange(N)
    return {
        "apply": lambda h: O.apply_rope_1d(h, pos, fc.double(), fs.double()),
        "spec": lambda dev: pom_amd._lib.RopeSpec(pom_amd._lib.ROPE_1D, [fc.to(dev), fs.to(dev)], pos.to(dev)),
    }


def _rope2d(D, H, W, seed=5):
    rc, rs, cc, cs = O.precompute_freqs_2d(D, H, W)
    pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
    return {
        "apply": lambda h: O.apply_rope_2d(h, pos, rc.double(), rs.double(), cc.double(), cs.double()),
        "spec": lambda dev: pom_amd._lib.RopeSpec(pom_amd._lib.ROPE_2D,
                                                  [rc.to(dev), rs.to(dev), cc.to(dev), cs.to(dev)], pos.to(dev)),
    }


@pytest.mark.parametrize("B,N,D,K", list(itertools.product([1, 4], [16, 256], [32, 96, 512], [1, 2, 4, 16])))
def test_rope1d_mean_f32(device, B, N, D, K):
    run_case(device, B, N, D, K, torch.float32, "mean", rope=_rope1d(D, N))


@pytest.mark.parametrize("B,N,D,K", GRID_BF16)
def test_rope1d_mean_bf16(device, B, N, D, K):
    run_case(device, B, N, D, K, torch.bfloat16, "mean", rope=_rope1d(D, N, random_pos=True), strided=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,D,K", [(1, 16, 32, 2), (2, 64, 64, 4)])
def test_rope1d_causal(device, B, N, D, K, dtype):
    run_case(device, B, N, D, K, dtype, "causal", rope=_rope1d(D, N))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["mean", "causal"])
def test_rope1d_negative_positions(device, kind, dtype):
    """Negative positions select table row p + rows, as the reference's
    freqs_cos[positions] does."""
    run_case(device, 2, 64, 64, 2, dtype, kind, rope=_rope1d(64, 64, negative=True))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,W,D,K", [(2, 8, 8, 64, 2), (1, 16, 16, 96, 3), (8, 8, 24, 64, 2)])
def test_rope2d_causal(device, B, H, W, D, K, dtype):
    """2-D RoPE with the token-causal prefix mean (pom/pom_rope.py:282-285 with
    the rotation of :406-416): the MODE_ROPE2D chunk sums, scan and backward."""
    run_case(device, B, H * W, D, K, dtype, "causal", rope=_rope2d(D, H, W))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rope", [False, True])
def test_causal_partial_scan_batch(device, dtype, rope):
    """B=8, N=192, D=64: the scan splits each row into 12 chunks of 16 tokens,
    so the chunk scan runs one full batch of eight chunks and then a partial
    one, and grad_coeff's finalize sums B * 12 = 96 chunk rows (four waves)."""
    run_case(device, 8, 192, 64, 2, dtype, "causal", rope=_rope1d(64, 192) if rope else None)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,W,D,K", [(2, 8, 8, 64, 2), (1, 16, 16, 96, 3), (2, 32, 32, 384, 2)])
def test_rope2d_mean(device, B, H, W, D, K, dtype):
    run_case(device, B, H * W, D, K, dtype, "mean", rope=_rope2d(D, H, W), strided=True)


@pytest.mark.parametrize("keep", [0.5, 0.25])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,N,D,K", [(2, 64, 64, 2), (3, 256, 96, 3), (2, 1024, 128, 2), (1, 33, 32, 16)])
def test_rope1d_masked(device, B, N, D, K, dtype, keep):
    """RoPE with a (B, N) padding mask: masked mean of the rotated features
    (pom/pom_rope.py:511-515)."""
    run_case(device, B, N, D, K, dtype, "masked", keep=keep, rope=_rope1d(D, N, random_pos=True),
             strided=dtype != torch.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,W,D,K", [(2, 8, 8, 64, 2), (2, 16, 16, 96, 3)])
def test_rope2d_masked(device, B, H, W, D, K, dtype):
    run_case(device, B, H * W, D, K, dtype, "masked", keep=0.5, rope=_rope2d(D, H, W), strided=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B", [1, 2, 3, 4, 6, 8])
def test_rope_backward_batch_groups(device, B, dtype):
    """The RoPE backward walks NB batch rows per workgroup (4, 2 or 1: the
    largest dividing B), one lane per half of a rotation pair, each table
    lookup shared by the NB rows.  Every NB, with groups of one and of several,
    1-D and 2-D, a degree that runs at three waves per SIMD (2) and one that
    does not (8), token counts whose chunks end in a partial step (200 and
    12 x 20), and frames (the per-frame weights of the block-causal mean)."""
    for K in (2, 8):
        run_case(device, B, 200, 64, K, dtype, "mean", rope=_rope1d(64, 200, random_pos=True),
                 strided=dtype != torch.float32)
        run_case(device, B, 12 * 20, 64, K, dtype, "mean", rope=_rope2d(64, 12, 20), strided=True)
    run_case(device, B, 256, 64, 3, dtype, "block", frame_len=64, rope=_rope1d(64, 256))


def test_rope_masked_invariants(device):
    """Masked RoPE: an all-ones mask gives the RoPE mean, an all-zero row gives
    0, padded tokens (even huge ones) never change the output or get a
    gradient."""
    B, N, D, K = 3, 256, 64, 2
    _, x, c = make_inputs(B, N, D, K, torch.float32)
    r = _rope1d(D, N, random_pos=True)
    spec = r["spec"](device)
    xd, cd = x.to(device), c.to(device)
    ones = torch.ones(B, N, device=device)
    a = ops.poly_agg_masked_hip(xd, ones, cd, K, spec)
    b = ops.poly_agg_rope_hip(xd, cd, K, spec, N)
    assert (a - b).abs().max().item() <= 1e-6
    m = (torch.arange(N).view(1, N) < torch.tensor([100, 256, 0]).view(B, 1)).float().to(device)
    x2 = x.clone()
    x2[(m == 0).cpu()] = torch.randn(int((m == 0).sum()), D) * 50
    x2d = x2.to(device).requires_grad_(True)
    o1 = ops.poly_agg_masked_hip(xd, m, cd, K, spec)
    o2 = ops.poly_agg_masked_hip(x2d, m, cd, K, spec)
    assert torch.equal(o1, o2)
    assert torch.all(o2[2] == 0) and torch.isfinite(o2).all()
    o2.sum().backward()
    assert torch.all(x2d.grad[m == 0] == 0)


def test_state_carry_matches_frames(device):
    """One call over F frames == F chained single-frame calls with the carry (bitwise)."""
    B, L, F, D, K = 2, 256, 4, 96, 2
    _, x, c = make_inputs(B, L * F, D, K, torch.bfloat16)
    xd, cd = x.to(device), c.to(device)
    full = pom_amd.poly_agg_block_causal_hip(xd, cd, K, L)
    carry, outs = None, []
    for f in range(F):
        h = ops.poly_agg_state_hip(xd[:, f * L:(f + 1) * L], cd, K, carry, f)
        outs.append(h)
        carry = h
    loop = torch.cat(outs, dim=1)
    assert torch.equal(full, loop)


def test_deterministic(device):
    _, x, c = make_inputs(4, 1024, 512, 3, torch.bfloat16)
    xd = x.to(device).requires_grad_(True)
    cd = c.to(device).requires_grad_(True)
    go = torch.randn(4, 1, 512).to(torch.bfloat16).to(device)
    res = []
    for _ in range(2):
        xd.grad = None
        cd.grad = None
        out = pom_amd.poly_agg_mean_hip(xd, cd, 3)
        out.backward(go)
        res.append((out.clone(), xd.grad.clone(), cd.grad.clone()))
    for a, b in zip(res[0], res[1]):
        assert torch.equal(a, b)
