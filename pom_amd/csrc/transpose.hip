// Out-of-place 2-D transpose, used to lay out the PoM layer's projection-GEMM
// operands contiguously along the reduction dimension.
//
// The matrix cores are fed fastest when both GEMM operands are contiguous in
// K.  The weight gradients dW_qc = dY^T x and dW_ag = g^T sh reduce over
// tokens, the row index of every activation, so they take token-contiguous
// copies (x^T, g^T, sh^T, dY^T); the data gradients dx = dY W_qc and
// dsh = g W_ag take the transposed weights.
//
// Each lane moves one E x E block (E = 16 bytes / element size: 8 for 16-bit
// types, 4 for fp32): E 16-byte row loads, a transpose in registers
// (v_perm_b32 for 16-bit pairs), E 16-byte column stores.  Eight lanes span
// one 128-byte row segment and the wave's eight row groups are adjacent, so a
// wave moves an 8E x 8E tile with every load and store instruction touching
// whole 128-byte lines.  No LDS, no synchronisation.  Blocks that cross the
// matrix edge fall back to element accesses with bounds checks; operands that
// are not 16-byte aligned use the element kernel throughout.
#include <hip/hip_runtime.h>
#include <cstdint>

#include "pom_internal.h"

namespace pom {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTThreads = 256;
constexpr int kTWaves = kTThreads / 64;

template <int EB>
struct Elem;
template <>
struct Elem<2> { using type = uint16_t; };
template <>
struct Elem<4> { using type = uint32_t; };

// In-register E x E transpose: a[k] holds row k (E elements), b[i] receives column i.
__device__ __forceinline__ void transpose_regs(const u32x4 (&a)[8], u32x4 (&b)[8]) {
  // 16-bit elements: element i of row k sits in dword i/2, half i%2 of a[k].
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // low half <- row 2j, high half <- row 2j+1, both element i
      const unsigned sel = (i & 1) ? 0x07060302u : 0x05040100u;
      b[i][j] = __builtin_amdgcn_perm(a[2 * j + 1][i >> 1], a[2 * j][i >> 1], sel);
    }
}

__device__ __forceinline__ void transpose_regs(const u32x4 (&a)[4], u32x4 (&b)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) b[i][j] = a[j][i];
}

template <int EB>
__global__ void __launch_bounds__(kTThreads) transpose_blocks(const char* __restrict__ src, int64_t lds,
                                                              char* __restrict__ dst, int64_t ldd, int64_t R,
                                                              int64_t C, int64_t tiles_c) {
  constexpr int E = 16 / EB, TILE = 8 * E;
  using V = typename Elem<EB>::type;
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * kTWaves + (threadIdx.x >> 6);
  const int64_t tr = wid / tiles_c, tc = wid - tr * tiles_c;
  const int64_t r0 = tr * TILE + (lane >> 3) * E, c0 = tc * TILE + (lane & 7) * E;
  if (r0 >= R || c0 >= C) return;
  const V* s = reinterpret_cast<const V*>(src);
  V* d = reinterpret_cast<V*>(dst);
  if (r0 + E <= R && c0 + E <= C) {
    u32x4 a[E], b[E];
#pragma unroll
    for (int k = 0; k < E; ++k) a[k] = *reinterpret_cast<const u32x4*>(s + (r0 + k) * lds + c0);
    transpose_regs(a, b);
#pragma unroll
    for (int i = 0; i < E; ++i) *reinterpret_cast<u32x4*>(d + (c0 + i) * ldd + r0) = b[i];
  } else {
    for (int k = 0; k < E && r0 + k < R; ++k)
      for (int i = 0; i < E && c0 + i < C; ++i) d[(c0 + i) * ldd + r0 + k] = s[(r0 + k) * lds + c0 + i];
  }
}

// Element kernel for unaligned operands: one thread per element, reads along rows.
template <int EB>
__global__ void __launch_bounds__(kTThreads) transpose_elems(const char* __restrict__ src, int64_t lds,
                                                             char* __restrict__ dst, int64_t ldd, int64_t R,
                                                             int64_t C) {
  using V = typename Elem<EB>::type;
  const int64_t idx = (int64_t)blockIdx.x * kTThreads + threadIdx.x;
  if (idx >= R * C) return;
  const int64_t r = idx / C, c = idx - r * C;
  reinterpret_cast<V*>(dst)[c * ldd + r] = reinterpret_cast<const V*>(src)[r * lds + c];
}

template <int EB>
hipError_t transpose_eb(const void* src, int64_t lds, void* dst, int64_t ldd, int64_t R, int64_t C,
                        hipStream_t st) {
  constexpr int E = 16 / EB, TILE = 8 * E;
  const bool vec = (reinterpret_cast<uintptr_t>(src) % 16 == 0) && (reinterpret_cast<uintptr_t>(dst) % 16 == 0) &&
                   lds % E == 0 && ldd % E == 0;
  if (vec) {
    const int64_t tiles_r = (R + TILE - 1) / TILE, tiles_c = (C + TILE - 1) / TILE;
    const int64_t waves = tiles_r * tiles_c;
    const dim3 grid((unsigned)((waves + kTWaves - 1) / kTWaves));
    hipLaunchKernelGGL((transpose_blocks<EB>), grid, dim3(kTThreads), 0, st, static_cast<const char*>(src), lds,
                       static_cast<char*>(dst), ldd, R, C, tiles_c);
  } else {
    const dim3 grid((unsigned)((R * C + kTThreads - 1) / kTThreads));
    hipLaunchKernelGGL((transpose_elems<EB>), grid, dim3(kTThreads), 0, st, static_cast<const char*>(src), lds,
                       static_cast<char*>(dst), ldd, R, C);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t transpose_t(int elem_bytes, const void* src, int64_t lds, void* dst, int64_t ldd, int64_t R, int64_t C,
                       hipStream_t st) {
  return elem_bytes == 4 ? transpose_eb<4>(src, lds, dst, ldd, R, C, st)
                         : transpose_eb<2>(src, lds, dst, ldd, R, C, st);
}

}  // namespace pom
