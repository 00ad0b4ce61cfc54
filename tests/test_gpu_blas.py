"""pom_blas_gemm (the library GEMMs of the layer's C++ launch sequence)
against torch.mm under the same offline-tuned selection table: for every
"tn" entry of the table, the same solution must give the same bits."""
import pytest
import torch

pytestmark = pytest.mark.gpu

from pom_amd import _lib, gemm_select  # noqa: E402


def _native_or_skip():
    if not gemm_select.native_ready():
        pytest.skip("the C library does not resolve to torch's rocBLAS / hipBLASLt, or torch rejected the table")


def _blas(a, b, ldc, ws):
    """C (n, m) = a (m, k) b (n, k)^T through pom_blas_gemm."""
    m, k = a.shape
    n = b.shape[0]
    c = torch.full((n, ldc), float("nan"), dtype=torch.bfloat16, device=a.device)
    rc = _lib.load().pom_blas_gemm(m, n, k, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), c.data_ptr(), ldc,
                                   ws.data_ptr(), ws.numel(), _lib.stream_handle(a.device))
    _lib.check(rc, "pom_blas_gemm")
    return c[:, :m]


@pytest.mark.parametrize("entry", gemm_select.table_entries(), ids=lambda e: "x".join(str(v) for v in e[0][:3]))
def test_blas_gemm_matches_torch_tuned(device, entry):
    _native_or_skip()
    (m, n, k, lda, ldb, ldc), _, _ = entry
    assert lda == k and ldb == k and ldc == m   # the form torch.mm(B, A^T) takes for row-major operands
    g = torch.Generator().manual_seed(m * 7 + n + k)
    a = torch.randn(m, k, generator=g).to(device, torch.bfloat16)
    b = torch.randn(n, k, generator=g).to(device, torch.bfloat16)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=device)
    got = _blas(a, b, ldc, ws)
    with gemm_select.tuned_gemms():
        ref = torch.mm(b, a.t())
    torch.cuda.synchronize()
    assert torch.equal(got, ref), f"max diff {(got.float() - ref.float()).abs().max().item()}"


def test_blas_gemm_refuses_unregistered_shapes(device):
    _native_or_skip()
    lib = _lib.load()
    assert lib.pom_blas_has_solution(192, 320, 448, 448, 448, 192) == 0
    a = torch.zeros(192, 448, dtype=torch.bfloat16, device=device)
    b = torch.zeros(320, 448, dtype=torch.bfloat16, device=device)
    c = torch.zeros(320, 192, dtype=torch.bfloat16, device=device)
    rc = lib.pom_blas_gemm(192, 320, 448, a.data_ptr(), 448, b.data_ptr(), 448, c.data_ptr(), 192, None, 0,
                           _lib.stream_handle(device))
    with pytest.raises(NotImplementedError, match="no solution registered"):
        _lib.check(rc, "pom_blas_gemm")
