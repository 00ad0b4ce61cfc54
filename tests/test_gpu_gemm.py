"""pom_gemm (the matrix-core projection GEMM) against torch's fp32 product of
the same bf16 operands: every operand layout, tile, split count and output
dtype, pipeline lengths 1-5 and 16 steps, the stream-K schedule, partial
edge tiles, padded leading dimensions, strided views, the C2 weight-gradient
shapes at full size, and determinism."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

from pom_amd import _lib, ops  # noqa: E402

TILES = {0: (256, 256), 1: (256, 192), 2: (192, 256), 3: (256, 128), 4: (128, 256), 5: (128, 128)}


def _operands(M, N, K, a_mn, b_mn, device, seed, pad=0):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn((K, M + pad) if a_mn else (M, K + pad), generator=g).to(device, torch.bfloat16)
    b = torch.randn((K, N + pad) if b_mn else (N, K + pad), generator=g).to(device, torch.bfloat16)
    if pad:
        a = a[:, :M] if a_mn else a[:, :K]
        b = b[:, :N] if b_mn else b[:, :K]
    return a, b


def _reference(a, a_mn, b, b_mn):
    """(A B in fp32, |A| |B|): the product and the scale of its accumulation error."""
    A = a.float().t() if a_mn else a.float()
    B = b.float() if b_mn else b.float().t()
    return A @ B, A.abs() @ B.abs()


def _run(a, a_mn, b, b_mn, M, N, K, out_dtype, tile, splits):
    lib = _lib.load()
    c = torch.full((M, N), float("nan"), dtype=out_dtype, device=a.device)
    wsb = lib.pom_gemm_workspace_size(M, N, K, tile, splits)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=a.device)
    rc = lib.pom_gemm(int(a_mn), int(b_mn), M, N, K, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
                      _lib.dtype_code(c), c.data_ptr(), c.stride(0), tile, splits, ws.data_ptr(), wsb,
                      _lib.stream_handle(a.device))
    _lib.check(rc, "pom_gemm")
    return c


def _check(c, refs, out_dtype, what):
    ref, absref = refs
    r = ref.double()
    d = (c.double() - r).abs()
    # fp32 accumulation in another order: a few units of 2^-24 times sum |a_k b_k|
    acc = absref.double() * 2.0 ** -20
    if out_dtype == torch.float32:
        e = ((c.double() - r).norm() / r.norm()).item()
        assert e <= 1e-5, f"{what}: fp32 relative error {e:.3g}"
        assert bool((d <= acc).all()), f"{what}: max abs diff {d.max().item():.3g}"
    else:
        # plus one bf16 rounding of the result
        assert bool((d <= r.abs() * 2.0 ** -7 + acc).all()), f"{what}: max abs diff {d.max().item():.3g}"
    assert not torch.isnan(c.float()).any(), f"{what}: unwritten outputs"


@pytest.mark.parametrize("a_mn,b_mn", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("tile", sorted(TILES))
def test_gemm_layouts_and_tiles(device, a_mn, b_mn, tile):
    bm, bn = TILES[tile]
    M, N = 2 * bm, bn
    for K, splits in ((64, 1), (128, 1), (192, 1), (320, 1), (1024, 1), (640, 2), (1024, 3)):
        a, b = _operands(M, N, K, a_mn, b_mn, device, seed=K + tile)
        ref = _reference(a, a_mn, b, b_mn)
        for out_dtype in (torch.bfloat16, torch.float32):
            c = _run(a, a_mn, b, b_mn, M, N, K, out_dtype, tile, splits)
            _check(c, ref, out_dtype, f"tile {bm}x{bn} A{int(a_mn)} B{int(b_mn)} K{K} s{splits} {out_dtype}")


@pytest.mark.parametrize("a_mn,b_mn", [(False, True), (True, True)])
def test_gemm_padded_leading_dimensions(device, a_mn, b_mn):
    M, N, K = 512, 384, 448
    a, b = _operands(M, N, K, a_mn, b_mn, device, seed=3, pad=24)
    assert a.stride(0) != (M if a_mn else K)
    ref = _reference(a, a_mn, b, b_mn)
    for tile, splits in ((1, 1), (5, 2), (3, 4)):
        if M % TILES[tile][0] or N % TILES[tile][1]:
            continue
        _check(_run(a, a_mn, b, b_mn, M, N, K, torch.float32, tile, splits), ref, torch.float32, f"tile {tile}")


def test_gemm_strided_projection_half(device):
    # the h-half of a fused projection output as the M-contiguous operand of a weight gradient
    T, P, D = 1024, 256, 192
    y = torch.randn(T, 2 * P).to(device, torch.bfloat16)
    x = torch.randn(T, D).to(device, torch.bfloat16)
    h = y[:, :P]
    got = ops.hip_gemm(h, True, x, True, torch.float32)
    _check(got, _reference(h, True, x, True), torch.float32, "h^T x")


def test_gemm_output_is_c_row_major_with_ldc(device):
    M, N, K = 256, 256, 128
    a, b = _operands(M, N, K, False, False, device, seed=5)
    lib = _lib.load()
    big = torch.full((M, N + 64), 7.0, dtype=torch.bfloat16, device=device)
    rc = lib.pom_gemm(0, 0, M, N, K, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), 1, big.data_ptr(),
                      big.stride(0), 0, 1, None, 0, _lib.stream_handle(device))
    _lib.check(rc, "pom_gemm")
    _check(big[:, :N], _reference(a, False, b, False), torch.bfloat16, "ldc")
    assert bool((big[:, N:] == 7.0).all()), "columns past N were written"


@pytest.mark.parametrize("name,M,N,K", [("ag_wgrad", 1152, 2304, 16384), ("qc_wgrad", 4608, 1152, 16384)])
def test_gemm_c2_weight_gradients_full_size(device, name, M, N, K):
    # dW_ag = g^T sh and dW_qc = dY^T x at config 2: token-major operands read in place
    a, b = _operands(M, N, K, True, True, device, seed=11)
    ref = _reference(a, True, b, True)
    got = ops.hip_gemm(a, True, b, True, torch.float32)
    _check(got, ref, torch.float32, name)
    got16 = ops.hip_gemm(a, True, b, True, torch.bfloat16)
    _check(got16, ref, torch.bfloat16, name + " bf16")


def test_gemm_deterministic_with_splits(device):
    M, N, K = 768, 512, 4096
    a, b = _operands(M, N, K, True, True, device, seed=9)
    for tile, splits in ((1, 1), (5, 3), (4, 8)):
        if M % TILES[tile][0] or N % TILES[tile][1]:
            continue
        c1 = _run(a, True, b, True, M, N, K, torch.float32, tile, splits)
        c2 = _run(a, True, b, True, M, N, K, torch.float32, tile, splits)
        assert torch.equal(c1, c2)


@pytest.mark.parametrize("a_mn,b_mn", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("tile", sorted(TILES))
def test_gemm_stream_k_layouts_and_tiles(device, a_mn, b_mn, tile):
    """Stream-K: 256 workgroups over 6 tiles x nk steps.  nk = 43 gives
    segments of one or two steps (many workgroups per tile), 100 and 171
    ranges that end inside a tile and carry on into the next; 256 puts every
    workgroup boundary at a multiple of a sixth of a tile."""
    bm, bn = TILES[tile]
    M, N = 3 * bm, 2 * bn
    for nk in (43, 100, 171, 256):
        K = 64 * nk
        a, b = _operands(M, N, K, a_mn, b_mn, device, seed=nk + 7 * tile)
        ref = _reference(a, a_mn, b, b_mn)
        for out_dtype in (torch.bfloat16, torch.float32):
            c = _run(a, a_mn, b, b_mn, M, N, K, out_dtype, tile, _lib.GEMM_STREAM_K)
            _check(c, ref, out_dtype, f"stream-K tile {bm}x{bn} A{int(a_mn)} B{int(b_mn)} nk{nk} {out_dtype}")


def test_gemm_stream_k_deterministic_and_padded(device):
    M, N, K = 768, 512, 4096
    a, b = _operands(M, N, K, True, True, device, seed=13, pad=40)
    ref = _reference(a, True, b, True)
    for tile in (0, 5):
        if M % TILES[tile][0] or N % TILES[tile][1]:
            continue
        c1 = _run(a, True, b, True, M, N, K, torch.float32, tile, _lib.GEMM_STREAM_K)
        c2 = _run(a, True, b, True, M, N, K, torch.float32, tile, _lib.GEMM_STREAM_K)
        assert torch.equal(c1, c2)
        _check(c1, ref, torch.float32, f"stream-K padded tile {tile}")


def test_gemm_plan_is_valid(device):
    lib = _lib.load()
    for (M, N, K) in ((16384, 4608, 1152), (1152, 2304, 16384), (4608, 1152, 16384), (65536, 1024, 4096),
                      (2368, 1152, 16384)):
        t, s = ctypes.c_int(), ctypes.c_int()
        assert lib.pom_gemm_plan(M, N, K, 0, 0, ctypes.byref(t), ctypes.byref(s)) == 0
        assert t.value in TILES and (1 <= s.value <= K // 64 or s.value == _lib.GEMM_STREAM_K)


@pytest.mark.parametrize("a_mn,b_mn", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("tile", sorted(TILES))
def test_gemm_partial_edge_tiles(device, a_mn, b_mn, tile):
    """M and N that the tile does not divide (the last row and column tiles
    partial, down to 8 of the tile's rows or columns): every output written
    once, nothing stored past N in a wider C, for direct, split-K and stream-K
    runs and both output dtypes."""
    bm, bn = TILES[tile]
    lib = _lib.load()
    for M, N in ((bm + 8, bn + 64), (2 * bm - 56, bn - 8), (8, 16)):
        for K, splits in ((320, 1), (1024, 3), (64 * 256, _lib.GEMM_STREAM_K)):
            if splits == _lib.GEMM_STREAM_K and -(-M // bm) * -(-N // bn) * (K // 64) < 256:
                continue
            a, b = _operands(M, N, K, a_mn, b_mn, device, seed=M + N + K + tile)
            ref = _reference(a, a_mn, b, b_mn)
            for out_dtype in (torch.bfloat16, torch.float32):
                c = torch.full((M, N + 24), float("nan"), dtype=out_dtype, device=device)
                c[:, N:] = 7.0
                wsb = lib.pom_gemm_workspace_size(M, N, K, tile, splits)
                ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=device)
                rc = lib.pom_gemm(int(a_mn), int(b_mn), M, N, K, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
                                  _lib.dtype_code(c), c.data_ptr(), c.stride(0), tile, splits, ws.data_ptr(), wsb,
                                  _lib.stream_handle(device))
                _lib.check(rc, "pom_gemm")
                what = f"edge tile {bm}x{bn} M{M} N{N} K{K} s{splits} A{int(a_mn)} B{int(b_mn)} {out_dtype}"
                _check(c[:, :N], ref, out_dtype, what)
                assert bool((c[:, N:] == 7.0).all()), what + ": columns past N were written"
