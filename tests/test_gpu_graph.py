"""A PoM layer forward + backward captured in a HIP graph replays to the
eager results, bit for bit, across several replays with eager work and
synchronisations in between (no memset nodes: the kernels' scratch needs no
initialisation), and after an in-place update of every parameter (the
graph must recompute the parameter-derived copies, fp32 coefficients and
transposed weights, on each replay)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

import pom_amd  # noqa: E402


@pytest.mark.parametrize("variant", ["mean", "block", "masked", "rope2d", "heads"])
def test_layer_graph_replays_match_eager(device, variant):
    torch.manual_seed(0)
    B, N, D = 4, 256, 128
    if variant == "rope2d":
        m = pom_amd.PoMRoPE(D, 2, 2, max_h=16, max_w=16, rope_2d=True).to(device, torch.bfloat16)
        pos = torch.stack(torch.meshgrid(torch.arange(16), torch.arange(16), indexing="ij"), -1).reshape(-1, 2)
        pos = pos.to(device)
        fwd = lambda x: m(x, positions_hw=pos)
    elif variant == "heads":
        # per-head gating: Y is P + 4 = 260 columns, padded to 320 (zero rows appended to W_qc)
        m = pom_amd.PoM(D, 2, 2, n_sel_heads=4).to(device, torch.bfloat16)
        fwd = lambda x: m(x)
    else:
        m = pom_amd.PoM(D, 2, 2).to(device, torch.bfloat16)
        if variant == "block":
            fwd = lambda x: m(x, mask=pom_amd.block_causal(64))
        elif variant == "masked":
            mask = (torch.arange(N).view(1, N) < torch.tensor([256, 100, 30, 200]).view(B, 1)).to(device)
            fwd = lambda x: m(x, mask=mask)
        else:
            fwd = lambda x: m(x)
    with torch.no_grad():
        m.po_coeff.normal_(0, 0.1)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, N, D, generator=g).to(device, torch.bfloat16).requires_grad_(True)
    go = torch.randn(B, N, D, generator=g).to(device, torch.bfloat16)
    params = list(m.parameters())

    def eager():
        for p in params:
            p.grad = None
        x.grad = None
        out = fwd(x)
        out.backward(go)
        return [out.detach().clone(), x.grad.clone()] + [p.grad.clone() for p in params]

    ref = eager()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for p in params:
        p.grad = None
    x.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fwd(x)
        out.backward(go)
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        got = [out, x.grad] + [p.grad for p in params]
        for a, b in zip(got, ref):
            assert torch.equal(a, b), f"replay {r}"
        # eager work between replays, then compare again
        eager()
        torch.cuda.synchronize()
    # an optimizer-like in-place update of every parameter between replays
    with torch.no_grad():
        for i, p in enumerate(params):
            p.mul_(0.75 + 0.05 * i)
    ref2 = eager()
    graph.replay()
    torch.cuda.synchronize()
    got = [out, x.grad] + [p.grad for p in params]
    for a, b in zip(got, ref2):
        assert torch.equal(a, b), "replay after parameter update"
