// Launch interface of the matrix-core GEMM (gemm.hip), shared with the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pom {

// bf16 GEMM C = A B on the matrix cores (gemm.hip).  Operands in either
// row-major layout: a_mn = false: A(m, k) = A[m * lda + k], true: A[k * lda + m];
// b_mn = false: B(k, n) = B[n * ldb + k], true: B[k * ldb + n].  C row-major
// (ldc), bf16 or fp32.  M, N multiples of 8 (the last tile of a row or column
// may be partial), K of 64, leading dimensions and pointers 16-byte aligned.  splits > 1 cuts K into that many
// parts whose fp32 partials (splits * M * N floats of workspace) are summed
// in split order.  splits == GEMM_STREAM_K runs the stream-K schedule:
// kStreamKGroups workgroups share the tiles' 64-steps evenly (needs
// tiles x K / 64 >= kStreamKGroups and gemm_streamk_ws_bytes of workspace).
constexpr int GEMM_STREAM_K = 256;
constexpr int kStreamKGroups = 256;
enum GemmTile {
  GEMM_TILE_256x256 = 0, GEMM_TILE_256x192, GEMM_TILE_192x256, GEMM_TILE_256x128, GEMM_TILE_128x256,
  GEMM_TILE_128x128, GEMM_TILE_COUNT
};
struct GemmProblem {
  const void* A = nullptr;
  const void* B = nullptr;
  void* C = nullptr;
  void* workspace = nullptr;
  int64_t lda = 0, ldb = 0, ldc = 0;
  int64_t M = 0, N = 0, K = 0;
  bool a_mn = false, b_mn = false, out_f32 = false;
  int tile = GEMM_TILE_256x256;
  int splits = 1;
};
void gemm_tile_dims(int tile, int* bm, int* bn);
// fp32 tile partials of the stream-K schedule: one per (tile, workgroup) segment, at most tiles + groups - 1
inline size_t gemm_streamk_ws_bytes(int64_t M, int64_t N, int bm, int bn) {
  return (size_t)(((M + bm - 1) / bm) * ((N + bn - 1) / bn) + kStreamKGroups - 1) * (size_t)bm * (size_t)bn * 4;
}
hipError_t gemm_bf16(const GemmProblem& p, hipStream_t st);

}  // namespace pom
