"""The layer's C++ launch sequence (pom_layer_fwd / pom_layer_bwd) against
the Python one (ops._PoMLayer with POM_AMD_NATIVE_LAYER off) on the baseline
configurations at full size.  Both run the same kernels with the same GEMM
solutions on the same operands, so the output, grad_x and every parameter
gradient are bit-identical; the output-projection bias gradient is a sum over
tokens that the two sequences reduce in different orders (fp32), checked to
one bf16 rounding."""
import pytest
import torch

pytestmark = pytest.mark.gpu

import bench  # noqa: E402
from pom_amd import gemm_select, ops  # noqa: E402


def _run(m, fwd, x, go):
    m.zero_grad(set_to_none=True)
    xd = x.clone().requires_grad_(True)
    out = fwd(m, xd)
    out.backward(go)
    return out.detach(), xd.grad, {n: p.grad.clone() for n, p in m.named_parameters() if p.grad is not None}


@pytest.mark.parametrize("name,bias", [("c2", False), ("c2", True), ("c2h", False), ("c2h", True), ("c3", False),
                                       ("c4", False), ("c5", False)])
def test_native_layer_matches_python_sequence(device, monkeypatch, name, bias):
    if not gemm_select.native_ready():
        pytest.skip("the C library does not resolve to torch's rocBLAS / hipBLASLt, or torch rejected the table")
    cfg = bench.CONFIGS[name]
    x, go, extra = bench.make_inputs(cfg)
    m = bench.make_module(cfg)
    if bias:   # the output projection's bias (the baseline modules have none)
        torch.manual_seed(5)
        m.ag_proj.bias = torch.nn.Parameter(torch.randn(cfg["D"]) * 0.1)
    m = m.to(device, torch.bfloat16)
    fwd = bench.forward_fn(cfg, {k: v.to(device) for k, v in extra.items()})
    x, go = x.to(device, torch.bfloat16), go.to(device, torch.bfloat16)
    monkeypatch.setattr(ops, "_NATIVE_LAYER", True)
    calls = list(ops.native_layer_calls)
    out_n, gx_n, gp_n = _run(m, fwd, x, go)
    assert ops.native_layer_calls[0] == calls[0] + 1 and ops.native_layer_calls[1] == calls[1] + 1, \
        "the C sequence did not run"
    monkeypatch.setattr(ops, "_NATIVE_LAYER", False)
    out_p, gx_p, gp_p = _run(m, fwd, x, go)
    assert ops.native_layer_calls == [calls[0] + 1, calls[1] + 1]
    assert torch.equal(out_n, out_p), "output"
    assert torch.equal(gx_n, gx_p), "grad_x"
    assert gp_n.keys() == gp_p.keys()
    for n in gp_n:
        a, b = gp_n[n].float(), gp_p[n].float()
        if n.endswith("ag_proj.bias"):
            assert bool(((a - b).abs() <= b.abs() * 2.0 ** -7 + 1e-6).all()), n
        else:
            assert torch.equal(gp_n[n], gp_p[n]), n


@pytest.mark.parametrize("name", ["c2", "c5"])
def test_native_backward_second_stream_is_bit_identical(device, monkeypatch, name):
    """POM_AMD_LAYER_OVERLAP (read by pom_layer_bwd at each call) runs dW_qc
    beside dx and / or dW_ag beside the data-gradient chain on a second stream,
    each with its own split-K workspace; the caller's stream waits for that
    stream before the call returns.  Every gradient equals the one-stream run's."""
    if not gemm_select.native_ready():
        pytest.skip("the C library does not resolve to torch's rocBLAS / hipBLASLt, or torch rejected the table")
    cfg = bench.CONFIGS[name]
    x, go, extra = bench.make_inputs(cfg)
    m = bench.make_module(cfg).to(device, torch.bfloat16)
    fwd = bench.forward_fn(cfg, {k: v.to(device) for k, v in extra.items()})
    x, go = x.to(device, torch.bfloat16), go.to(device, torch.bfloat16)
    monkeypatch.setattr(ops, "_NATIVE_LAYER", True)
    monkeypatch.setenv("POM_AMD_LAYER_OVERLAP", "0")
    ref = _run(m, fwd, x, go)
    for mode in ("1", "2", "3"):
        monkeypatch.setenv("POM_AMD_LAYER_OVERLAP", mode)
        calls = ops.native_layer_calls[1]
        got = _run(m, fwd, x, go)
        assert ops.native_layer_calls[1] == calls + 1, "the C sequence did not run"
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1]), f"mode {mode}: output / grad_x"
        for n in ref[2]:
            assert torch.equal(got[2][n], ref[2][n]), f"mode {mode}: {n}"
