"""pom_agg_fwd_noalloc (static device scratch, no workspace argument) against
pom_agg_fwd with a workspace: identical bits on two calls in a row, the second
with a smaller input, for each aggregation mode; shapes beyond the static
scratch are refused before anything is launched."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

from pom_amd import _lib  # noqa: E402


def _agg(device, noalloc, x, coeff, K, frame_len, mask=None, carry=None, n_past=0, rope=None):
    lib = _lib.load()
    B, N, P = x.shape
    out = torch.full((B, N // frame_len, P), float("nan"), dtype=x.dtype, device=device)
    count = torch.empty(B, dtype=torch.float32, device=device) if mask is not None else None
    xv = _lib.view3(x)
    args = [_lib.dtype_code(x), _lib.dtype_code(coeff), B, N, P, K, ctypes.byref(xv), coeff.data_ptr(),
            _lib.ptr(mask), mask.stride(0) if mask is not None else 0, mask.stride(1) if mask is not None else 0,
            frame_len, _lib.ptr(carry), n_past, _lib.rope_ptr(rope), out.data_ptr(), _lib.ptr(count)]
    stream = _lib.stream_handle(device)
    if noalloc:
        before = torch.cuda.memory_allocated(device)
        rc = lib.pom_agg_fwd_noalloc(*args, stream)
        assert torch.cuda.memory_allocated(device) == before
        _lib.check(rc, "pom_agg_fwd_noalloc")
    else:
        nbytes = lib.pom_agg_workspace_size(args[0], B, N, P, K, frame_len,
                                            rope.kind if rope is not None else 0, 0)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _lib.check(lib.pom_agg_fwd(*args, ws.data_ptr(), ws.numel(), stream), "pom_agg_fwd")
    torch.cuda.synchronize(device)
    return out, count


def _inputs(device, B, N, P, K, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, N, P, generator=g) * 0.8).to(dtype).to(device)
    c = (torch.randn(P, K, generator=g) * 0.2).to(device)
    return x, c


CASES = {
    # name: (big shape, small shape) as (B, N, P, K, frame_len)
    "mean": ((16, 1024, 2304, 2, 1024), (2, 256, 512, 2, 256)),
    "frames": ((4, 4096, 1024, 2, 512), (2, 512, 256, 3, 128)),
    "masked": ((8, 2048, 1024, 3, 2048), (3, 300, 96, 2, 300)),
    "causal": ((2, 2048, 512, 2, 1), (2, 192, 64, 2, 1)),
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("mode", list(CASES))
def test_noalloc_matches_workspace_entry(device, mode, dtype):
    for i, (B, N, P, K, fl) in enumerate(CASES[mode]):
        print(f"noalloc {mode} {dtype} call {i}: B{B} N{N} P{P} K{K} frame_len {fl}", flush=True)
        x, c = _inputs(device, B, N, P, K, dtype, 10 + i)
        mask = None
        if mode == "masked":
            lens = torch.randint(1, N + 1, (B,), generator=torch.Generator().manual_seed(3))
            mask = (torch.arange(N).view(1, N) < lens.view(B, 1)).float().to(device)
        a, ca = _agg(device, True, x, c, K, fl, mask)
        b, cb = _agg(device, False, x, c, K, fl, mask)
        assert torch.equal(a, b), f"{mode} call {i}"
        if mask is not None:
            assert torch.equal(ca, cb)


def test_noalloc_carry_and_rope(device):
    """A state_forward step (carry, n_past) and a 2-D RoPE mean, back to back."""
    x, c = _inputs(device, 4, 1024, 512, 2, torch.bfloat16, 1)
    carry = (torch.randn(4, 512) * 0.1).to(torch.bfloat16).to(device)
    a, _ = _agg(device, True, x, c, 2, 1024, carry=carry, n_past=3)
    b, _ = _agg(device, False, x, c, 2, 1024, carry=carry, n_past=3)
    assert torch.equal(a, b)
    H = W = 16
    rc, rs = torch.randn(H, 64).to(device), torch.randn(H, 64).to(device)
    cc, cs = torch.randn(W, 64).to(device), torch.randn(W, 64).to(device)
    pos = torch.stack(torch.meshgrid(torch.arange(H), torch.arange(W), indexing="ij"), -1).reshape(-1, 2)
    spec = _lib.RopeSpec(_lib.ROPE_2D, [rc, rs, cc, cs], pos, device)
    x2, c2 = _inputs(device, 2, H * W, 256, 2, torch.bfloat16, 2)
    a, _ = _agg(device, True, x2, c2, 2, H * W, rope=spec)
    b, _ = _agg(device, False, x2, c2, 2, H * W, rope=spec)
    assert torch.equal(a, b)


def test_noalloc_refuses_oversize_shape(device):
    """Token-causal at C4's length needs 64 MiB of scratch: refused, output untouched."""
    x, c = _inputs(device, 4, 16384, 4096, 2, torch.bfloat16, 1)
    lib = _lib.load()
    out = torch.zeros(4, 16384, 4096, dtype=torch.bfloat16, device=device)
    xv = _lib.view3(x)
    rc = lib.pom_agg_fwd_noalloc(1, 0, 4, 16384, 4096, 2, ctypes.byref(xv), c.data_ptr(), None, 0, 0, 1, None, 0,
                                 None, out.data_ptr(), None, _lib.stream_handle(device))
    assert rc == _lib.POM_ERR_WORKSPACE and b"static scratch" in lib.pom_last_error()
    torch.cuda.synchronize(device)
    assert int(out.abs().sum()) == 0
