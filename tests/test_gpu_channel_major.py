"""The channel-major ("transposed") copies that the gate and aggregation
kernels write beside their row-major outputs (sh^T in the gate forward, the
two halves of dY^T in the backward) equal the transpose of those outputs bit
for bit, for every mode, ragged token counts (groups of 8 tokens cut by the
chunk end), masked extents (zero-filled rows) and the per-token gate.  The
row-major outputs are unchanged by the extra copy."""
import pytest
import torch

pytestmark = pytest.mark.gpu

from pom_amd import _lib, ops  # noqa: E402

DT = torch.bfloat16


def _rope(kind, N, P, device, seed=11):
    g = torch.Generator().manual_seed(seed)
    if kind is None:
        return None
    if kind == "1d":
        fc, fs = torch.randn(N + 3, P // 2, generator=g), torch.randn(N + 3, P // 2, generator=g)
        pos = torch.randperm(N, generator=g)
        return _lib.RopeSpec(_lib.ROPE_1D, [fc.to(device), fs.to(device)], pos.to(device))
    H = W = int(round(N ** 0.5))
    assert H * W == N
    t = [torch.randn(H, P // 4, generator=g) for _ in range(4)]
    pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
    return _lib.RopeSpec(_lib.ROPE_2D, [u.to(device) for u in t], pos.to(device))


def _inputs(B, N, P, device, seed=3):
    g = torch.Generator().manual_seed(seed)
    y = (torch.randn(B, N, 2 * P, generator=g) * 2.5).to(device, DT)
    return y, g


@pytest.mark.parametrize("B,N,P,G,rope", [(2, 256, 128, 1, None), (2, 36, 64, 1, None), (3, 100, 128, 4, None),
                                          (2, 64, 64, 64, None), (4, 1024, 2304, 1, None),
                                          (2, 64, 128, 1, "1d"), (2, 64, 128, 1, "2d"), (2, 36, 64, 1, "2d")])
def test_gate_forward_copy(device, B, N, P, G, rope):
    y, g = _inputs(B, N, P, device)
    ys = y[..., P:]
    bias = torch.randn(P, generator=g).to(device)
    hagg = torch.randn(B, G, P, generator=g).to(device, DT)
    spec = _rope(rope, N, P, device)
    ref = ops.gate_forward(ys, bias, hagg, spec)
    sht = torch.full((P, B * N), float("nan"), dtype=DT, device=device)
    sh = ops.gate_forward(ys, bias, hagg, spec, out_t=sht)
    assert torch.equal(sh, ref)
    assert torch.equal(sht, sh.reshape(B * N, P).t())


@pytest.mark.parametrize("B,N,P,G,rope", [(2, 256, 128, 1, None), (2, 36, 64, 1, None), (3, 100, 128, 4, None),
                                          (2, 64, 64, 64, None), (4, 1024, 2304, 1, None),
                                          (2, 64, 128, 1, "1d"), (2, 36, 64, 1, "2d")])
def test_gate_backward_copy(device, B, N, P, G, rope):
    y, g = _inputs(B, N, P, device)
    ys = y[..., P:]
    bias = torch.randn(P, generator=g).to(device)
    hagg = torch.randn(B, G, P, generator=g).to(device, DT)
    gsh = torch.randn(B, N, P, generator=g).to(device, DT)
    spec = _rope(rope, N, P, device)
    d0 = torch.zeros(B, N, 2 * P, dtype=DT, device=device)
    gh0, gb0 = ops.gate_backward(ys, bias, hagg, gsh, d0[..., P:], spec)
    d1 = torch.zeros(B, N, 2 * P, dtype=DT, device=device)
    dyt = torch.full((2 * P, B * N), float("nan"), dtype=DT, device=device)
    gh1, gb1 = ops.gate_backward(ys, bias, hagg, gsh, d1[..., P:], spec, grad_ys_t=dyt[P:],
                                 grad_ys_rows=d1.view(B * N, 2 * P)[:, P:])
    assert torch.equal(d1, d0)
    assert torch.equal(dyt[P:], d1.view(B * N, 2 * P)[:, P:].t())
    assert torch.isnan(dyt[:P].float()).all()   # the other half is left alone
    # reductions: the copy changes which lane sums which tokens, not the result beyond rounding
    assert torch.allclose(gh1, gh0, rtol=1e-4, atol=1e-4)
    assert torch.allclose(gb1, gb0, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("B,N,P,K,frame_len,kind", [(2, 256, 128, 2, None, "mean"), (2, 36, 64, 3, None, "mean"),
                                                    (3, 128, 64, 2, 32, "mean"), (2, 200, 128, 2, None, "masked"),
                                                    (4, 1024, 2304, 2, None, "mean"), (2, 64, 128, 2, None, "1d"),
                                                    (2, 64, 128, 2, None, "2d"), (2, 36, 64, 2, None, "2d")])
def test_agg_backward_copy(device, B, N, P, K, frame_len, kind):
    y, g = _inputs(B, N, P, device)
    x = y[..., :P]
    coeff = (torch.randn(P, K, generator=g) * 0.3).to(device)
    fl = N if frame_len is None else frame_len
    F = N // fl
    go = torch.randn(B, F, P, generator=g).to(device)
    mask = count = None
    if kind == "masked":
        lens = torch.tensor([N - 37, 60])
        m = (torch.arange(N).view(1, N) < lens.view(B, 1)).float()
        m[1, :5] = 0   # a leading gap: rows before the first valid one are zero-filled
        mask = m.to(device)
        count = mask.sum(1)
    spec = _rope(kind if kind in ("1d", "2d") else None, N, P, device)
    d0 = torch.zeros(B, N, 2 * P, dtype=DT, device=device)
    gc0 = ops.agg_backward(x, coeff, K, fl, go, d0[..., :P], mask, count, 0, spec)
    d1 = torch.zeros(B, N, 2 * P, dtype=DT, device=device)
    dyt = torch.full((2 * P, B * N), float("nan"), dtype=DT, device=device)
    gc1 = ops.agg_backward(x, coeff, K, fl, go, d1[..., :P], mask, count, 0, spec, grad_x_t=dyt[:P],
                           grad_x_rows=d1.view(B * N, 2 * P)[:, :P])
    assert torch.equal(d1, d0)
    assert torch.equal(dyt[:P], d1.view(B * N, 2 * P)[:, :P].t())
    assert torch.isnan(dyt[P:].float()).all()
    assert torch.allclose(gc1, gc0, rtol=1e-4, atol=1e-4)


def test_token_causal_copy_falls_back_to_transpose(device):
    """Token-causal aggregation has no fused copy: the wrapper transposes."""
    B, N, P = 2, 64, 64
    y, g = _inputs(B, N, P, device)
    x = y[..., :P]
    coeff = (torch.randn(P, 2, generator=g) * 0.3).to(device)
    go = torch.randn(B, N, P, generator=g).to(device)
    d = torch.zeros(B, N, 2 * P, dtype=DT, device=device)
    dyt = torch.full((2 * P, B * N), float("nan"), dtype=DT, device=device)
    ops.agg_backward(x, coeff, 2, 1, go, d[..., :P], grad_x_t=dyt[:P], grad_x_rows=d.view(B * N, 2 * P)[:, :P])
    assert torch.equal(dyt[:P], d.view(B * N, 2 * P)[:, :P].t())
