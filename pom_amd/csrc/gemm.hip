// bf16 GEMM for the PoM projections on gfx950 (CDNA4) matrix cores.
//
//   C[m, n] = sum_k A(m, k) * B(k, n),  fp32 accumulation, C in bf16 or fp32
//
// Each operand is read in place in either of its two row-major layouts, so
// no projection needs a transposed copy of an activation or weight:
//   A "K-contiguous":  A(m, k) = A[m * lda + k]     (x, sh, g, dY in the forward / data gradients)
//   A "M-contiguous":  A(m, k) = A[k * lda + m]     (g, dY as the weight gradients' left operand)
//   B "K-contiguous":  B(k, n) = B[n * ldb + k]     (W_qc, W_ag in the forward)
//   B "N-contiguous":  B(k, n) = B[k * ldb + n]     (W_qc, W_ag in the data gradients; x, sh in the
//                                                    weight gradients)
//
// Kernel structure (one 256-thread workgroup per BM x BN output tile):
//   * 4 waves in a 2 x 2 grid; a wave owns a (BM/2) x (BN/2) sub-tile of
//     32 x 32 blocks, computed with v_mfma_f32_32x32x16_bf16 into fp32
//     accumulators held in the AGPR half of the register file (one wave
//     per SIMD);
//   * the k-loop steps 64 at a time.  Tile t is loaded from global memory
//     into register set t % 2 during step t - 3, stored to LDS stage t % 2
//     during step t - 1 and multiplied during step t, so every global load
//     has two steps to land; one workgroup barrier per step, which waits
//     for LDS traffic only (the global loads stay in flight across it);
//   * operand loads are buffer loads: a wave-uniform descriptor, one 32-bit
//     offset per thread, the k advance and row steps in the scalar offset.
//     The descriptor's size ends at the operand's last element, so a partial
//     edge tile (M or N not a multiple of the tile) never reads past it: rows
//     and columns beyond M / N read zeros or other in-bounds elements, which
//     only reach outputs the epilogue does not store;
//   * LDS layout of an operand (R rows x 64 k): four sub-arrays, one per
//     16-k sub-step, each R rows of 32 bytes plus 32 bytes of padding, rows
//     and halves permuted within row octets (lds_addr) so that fragment
//     reads and the stores of either layout are free of bank conflicts, and
//     a lane's fragment reads and stores address off two base registers
//     with immediate offsets;
//   * an M/N-contiguous operand is loaded as 8 x 8 blocks (8 k-rows of 8
//     consecutive m) and transposed in registers (v_perm_b32) before its
//     LDS store, so both layouts share one LDS layout and one fragment read;
//   * the MFMA is issued with B as its first operand, so each lane ends with
//     4 consecutive n of one output row per 4 accumulators (8-byte bf16 or
//     16-byte fp32 stores);
//   * split-K: the k range is cut into S contiguous parts (whole 64-steps),
//     each written as an fp32 partial (S, M, N); gemm_splitk_reduce sums the
//     partials in split order, so results do not depend on scheduling;
//   * stream-K: G workgroups (one per CU) share the tiles' 64-steps evenly.
//     Workgroup w takes the global steps [w I / G, (w + 1) I / G) of the
//     I = tiles x steps in tile order, so its range may end inside one tile
//     and continue into the next; each (tile t, workgroup w) segment writes
//     an fp32 tile partial into slot t + w (distinct for every segment, as
//     each next segment advances t, w or both), and gemm_streamk_reduce sums
//     a tile's segments in workgroup order (deterministic).  This fills every
//     CU when tiles x splits would leave some idle;
//   * workgroups are dispatched to the 8 XCDs round-robin; the grid index is
//     remapped so each XCD owns a contiguous run of tiles, ordered in groups
//     of GM row tiles, and its 32 CUs share operand panels in their L2.
#include <type_traits>

#include "gemm.h"

namespace pom {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kBK = 64;        // k per pipeline step
constexpr int kThreads = 256;  // 4 waves
constexpr int kGroupM = 8;     // row tiles per ordering group

struct GemmArgs {
  const uint16_t* A;
  const uint16_t* B;
  void* C;                    // bf16 output, or the fp32 partials (S, M, N)
  int64_t lda, ldb, ldc;      // elements
  int64_t a_elems, b_elems;   // operand extents in elements (end of the last row)
  int64_t split_stride;       // elements between the fp32 partials of two splits
  int M, N;
  int nk;                     // 64-steps over the whole K
  int splits;
  int tiles_m, tiles_n;
};

// Stream-K segments of tile t: the first and last workgroup whose step range
// meets the tile's steps [t nk, (t + 1) nk), for G workgroups over I steps
// (workgroup w owns [floor(w I / G), floor((w + 1) I / G)), never empty as I >= G).
__host__ __device__ inline int64_t sk_first(int64_t t, int64_t nk, int64_t I, int64_t G) {
  return (((t * nk + 1) * G + I - 1) / I) - 1;
}
__host__ __device__ inline int64_t sk_last(int64_t t, int64_t nk, int64_t I, int64_t G) {
  return ((((t + 1) * nk) * G + I - 1) / I) - 1;
}

// row tile and column tile of tile index t: tiles run in groups of kGroupM row tiles, column-major
// within a group, so consecutive workgroups share operand panels
__host__ __device__ inline void tile_coords(int t, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int span = kGroupM * tiles_n;
  const int grp = t / span;
  const int first_m = grp * kGroupM;
  const int gsz = tiles_m - first_m < kGroupM ? tiles_m - first_m : kGroupM;
  t -= grp * span;
  tm = first_m + t % gsz;
  tn = t / gsz;
}
__host__ __device__ inline int tile_index(int tm, int tn, int tiles_m, int tiles_n) {
  const int grp = tm / kGroupM, first_m = grp * kGroupM;
  const int gsz = tiles_m - first_m < kGroupM ? tiles_m - first_m : kGroupM;
  return grp * kGroupM * tiles_n + tn * gsz + (tm - first_m);
}

// LDS bytes of one operand's sub-array (one 16-k sub-step) and of the operand.
template <int R>
constexpr int sub_bytes() { return R * 32 + 32; }
template <int R>
constexpr int opnd_bytes() { return 4 * sub_bytes<R>(); }

// Offset of the 16-byte half `h` (k = 16 s + 8 h .. + 7) of row `row` in sub-array s.
// gfx950's LDS serves a 16-byte read 16 lanes at a time from a 256-byte bank window and a 16-byte
// write 8 lanes at a time from a 128-byte window (measured with the bank-conflict counter), so the
// 16 lanes of a read and the 8 lanes of a write must each touch distinct 16-byte slots of their window.
// Rows are 32 bytes; within a row octet o the rows are permuted by o & 3, the two halves swap when
// bit 0 of o or bit 2 of o is set, and sub-arrays are 32 bytes out of step.  Then 16 consecutive rows
// of one half (a fragment read), the 8 halves of one row (a K-contiguous store) and one column of 8
// consecutive octets (an M/N-contiguous store) all spread over their windows.
template <int R>
__device__ __forceinline__ int lds_addr(int s, int row, int h) {
  const int oct = row >> 3;
  return s * sub_bytes<R>() + ((row ^ (oct & 3)) << 5) + ((h ^ (oct & 1) ^ ((oct >> 2) & 1)) << 4);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4_t buf_load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Addressing of one operand, shared by both register sets.
//   K-contiguous, instruction j of wave w, lane l: row (4 j + w) * 8 + (l >> 3), 16-byte chunk l & 7
//   (k = 8 (l & 7)); consecutive lanes read consecutive 16-byte pieces of one 128-byte row segment.
//   M/N-contiguous, block b of the thread (b < R; threads past R repeat b % R and store the same bytes
//   to the same addresses as its owner): columns 8 mo .. 8 mo + 7 with mo = b % (R/8), k-rows
//   8 kg .. 8 kg + 7 with kg = b / (R/8); 8 consecutive lanes read 128 contiguous bytes of a k-row.
template <int R, bool MN>
struct Operand {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t voff;
  uint32_t sstride;   // K-contiguous: bytes of 32 rows; M/N-contiguous: bytes of one k-row
  int st0;            // LDS store base: K: row j at (j odd ? st1 : st0) + 1024 j; M/N: column i at
  int st1;            //   st0 + ((i ^ st1) << 5)
  __device__ __forceinline__ void init(const uint16_t* base, int64_t ld, uint32_t bytes, int tid, int b) {
    rsrc = make_rsrc(base, bytes);
    if constexpr (MN) {
      b %= R;
      const int mo = b % (R / 8), kg = b / (R / 8);
      voff = (uint32_t)(((int64_t)kg * 8 * ld + mo * 8) * 2);
      sstride = (uint32_t)(ld * 2);
      st0 = lds_addr<R>(kg >> 1, mo * 8, kg & 1) - ((mo & 3) << 5);
      st1 = mo & 3;
    } else {
      const int w = tid >> 6, l = tid & 63, c = l & 7, row = w * 8 + (l >> 3);
      voff = (uint32_t)(((int64_t)row * ld + c * 8) * 2);
      sstride = (uint32_t)(ld * 64);
      st0 = lds_addr<R>(c >> 1, row, c & 1);
      st1 = lds_addr<R>(c >> 1, row + 32, c & 1) - 32 * 32;
    }
  }
};

template <int R, bool MN>
struct Staged {
  static constexpr int J = MN ? 8 : R / 32;   // global loads and LDS stores per 64-step
  u32x4_t v[J];
  // global load j (K-contiguous: rows 32 j ..; M/N-contiguous: k-row j of the block)
  __device__ __forceinline__ void load_one(const Operand<R, MN>& o, int k0, int j) {
    const uint32_t soff = MN ? ((uint32_t)k0 + j) * o.sstride : (uint32_t)k0 * 2 + (uint32_t)j * o.sstride;
    v[j] = buf_load(o.rsrc, o.voff, soff);
  }
  __device__ __forceinline__ void load(const Operand<R, MN>& o, int k0) {
#pragma unroll
    for (int j = 0; j < J; ++j) load_one(o, k0, j);
  }
  // LDS store j into the operand's region `lds` (M/N-contiguous: column j of the block, which reads
  // every loaded k-row, so an operand's loads may only follow all of its stores)
  __device__ __forceinline__ void store_one(char* lds, const Operand<R, MN>& o, int j) const {
    if constexpr (MN) {
      // column j: k-pairs (2e, 2e+1) from rows 2e and 2e+1, half j % 2 of dword j / 2
      const unsigned sel = (j & 1) ? 0x07060302u : 0x05040100u;
      u32x4_t w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = __builtin_amdgcn_perm(v[2 * e + 1][j >> 1], v[2 * e][j >> 1], sel);
      *reinterpret_cast<u32x4_t*>(lds + o.st0 + ((j ^ o.st1) << 5)) = w;
    } else {
      *reinterpret_cast<u32x4_t*>(lds + ((j & 1) ? o.st1 : o.st0) + j * 32 * 32) = v[j];
    }
  }
  __device__ __forceinline__ void store(char* lds, const Operand<R, MN>& o) const {
#pragma unroll
    for (int j = 0; j < J; ++j) store_one(lds, o, j);
  }
};

// LDS writes of this wave are complete and every wave has reached this point.
// Outstanding global loads are not waited for.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One output tile over the 64-steps [it0, it1): C(m, n) at c + (m - LOCAL ? m0 : 0) * ldc + (n - LOCAL ? n0 : 0).
template <int BM, int BN, bool A_MN, bool B_MN, bool OUT_F32, bool LOCAL>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, char* smem, int t, int it0, int it1, void* cout,
                                          int64_t ldc) {
  constexpr int WM = BM / 2, WN = BN / 2, MB = WM / 32, NB = WN / 32;
  constexpr int A_BYTES = opnd_bytes<BM>(), STAGE = opnd_bytes<BM>() + opnd_bytes<BN>();
  static_assert(MB >= 1 && NB >= 1 && WM % 32 == 0 && WN % 32 == 0, "tile");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int tm, tn;
  tile_coords(t, g.tiles_m, g.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = it1 - it0;
  const int kbeg = it0 * kBK;

  Operand<BM, A_MN> oa;
  Operand<BN, B_MN> ob;
  {
    const int64_t a_off = A_MN ? m0 : (int64_t)m0 * g.lda, b_off = B_MN ? n0 : (int64_t)n0 * g.ldb;
    oa.init(g.A + a_off, g.lda, (uint32_t)((g.a_elems - a_off) * 2), tid, tid);
    ob.init(g.B + b_off, g.ldb, (uint32_t)((g.b_elems - b_off) * 2), tid, kThreads - 1 - tid);
  }
  Staged<BM, A_MN> ta0, ta1;
  Staged<BN, B_MN> tb0, tb1;

  f32x16_t acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // this lane's fragment rows: A rows wm * WM + 32 i + (lane & 31), B rows wn * WN + 32 j + (lane & 31),
  // half lane >> 5 of each 16-k sub-step
  // (blocks 2 q and 2 q + 1 differ in the half swap, so even and odd blocks have their own base)
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int fa0 = lds_addr<BM>(0, wm * WM + lrow, lhalf);
  const int fa1 = lds_addr<BM>(0, wm * WM + 32 + lrow, lhalf) - 32 * 32;
  const int fb0 = A_BYTES + lds_addr<BN>(0, wn * WN + lrow, lhalf);
  const int fb1 = A_BYTES + lds_addr<BN>(0, wn * WN + 32 + lrow, lhalf) - 32 * 32;

  auto read_frags = [&](const char* st, int s, bf16x8_t (&af)[MB], bf16x8_t (&bfr)[NB]) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
      af[i] = *reinterpret_cast<const bf16x8_t*>(st + ((i & 1) ? fa1 : fa0) + s * sub_bytes<BM>() + i * 32 * 32);
#pragma unroll
    for (int j = 0; j < NB; ++j)
      bfr[j] = *reinterpret_cast<const bf16x8_t*>(st + ((j & 1) ? fb1 : fb0) + s * sub_bytes<BN>() + j * 32 * 32);
  };
  auto mfmas = [&](const bf16x8_t (&af)[MB], const bf16x8_t (&bfr)[NB]) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
  };
  // One 64-step on stage `cur`: the staged tile of register set (sa, sb) is written into stage `nxt`,
  // the set is refilled with the tile at k0, and the four 16-k sub-steps' MFMAs run on fragments read
  // one sub-step ahead.  The memory instructions are spread one or two at a time between the MFMAs,
  // in a fixed order (a scheduling fence after each MFMA slot): issued in bursts, the global loads and
  // LDS stores back up the address and LDS queues and block the wave from issuing MFMAs (measured:
  // about a third of a step).  The stores take the first two sub-steps and the loads the last two,
  // so every load refills registers whose store has issued.
  constexpr int NMF = MB * NB, NRD = MB + NB;
  constexpr int JA = Staged<BM, A_MN>::J, JB = Staged<BN, B_MN>::J, NWR = JA + JB;
  auto step64 = [&](const char* cur, char* nxt, Staged<BM, A_MN>& sa, Staged<BN, B_MN>& sb, int k0) {
    bf16x8_t af[2][MB], bfr[2][NB];
    read_frags(cur, 0, af[0], bfr[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int m = 0; m < NMF; ++m) {
        const int i = m / NB, j = m % NB;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[q & 1][j], af[q & 1][i], acc[i][j], 0, 0, 0);
        if (q < 3) {   // next sub-step's fragments r in [lo, hi)
          const int lo = (m * NRD + NMF - 1) / NMF, hi = ((m + 1) * NRD + NMF - 1) / NMF;
#pragma unroll
          for (int r = lo; r < hi; ++r) {
            if (r < MB)
              af[(q + 1) & 1][r] = *reinterpret_cast<const bf16x8_t*>(
                  cur + ((r & 1) ? fa1 : fa0) + (q + 1) * sub_bytes<BM>() + r * 32 * 32);
            else
              bfr[(q + 1) & 1][r - MB] = *reinterpret_cast<const bf16x8_t*>(
                  cur + (((r - MB) & 1) ? fb1 : fb0) + (q + 1) * sub_bytes<BN>() + (r - MB) * 32 * 32);
          }
        }
        // stores (sub-steps 0-1) or loads (sub-steps 2-3) w in [lo, hi) of NWR
        const int g = (q & 1) * NMF + m;
        const int lo = (g * NWR + 2 * NMF - 1) / (2 * NMF), hi = ((g + 1) * NWR + 2 * NMF - 1) / (2 * NMF);
#pragma unroll
        for (int w = lo; w < hi; ++w) {
          if (q < 2) {
            if (w < JA) sa.store_one(nxt, oa, w);
            else sb.store_one(nxt + A_BYTES, ob, w - JA);
          } else {
            if (w < JA) sa.load_one(oa, k0, w);
            else sb.load_one(ob, k0, w - JA);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    lds_barrier();
  };

  // Prologue: tiles 0 and 1 into the register sets, tile 0 into stage 0, tile 2 into set 0.  Every
  // step stores and loads, so the loop body is one straight-line form: past the end the loads repeat
  // the last tile (cache hits) and the store fills a stage that is not read again.
  const int klast = kbeg + (nk - 1) * kBK;
  ta0.load(oa, kbeg);
  tb0.load(ob, kbeg);
  ta1.load(oa, kbeg + min(1, nk - 1) * kBK);
  tb1.load(ob, kbeg + min(1, nk - 1) * kBK);
  ta0.store(smem, oa);
  tb0.store(smem + A_BYTES, ob);
  ta0.load(oa, kbeg + min(2, nk - 1) * kBK);
  tb0.load(ob, kbeg + min(2, nk - 1) * kBK);
  lds_barrier();

  int it = 0;
  for (; it + 2 <= nk; it += 2) {
    step64(smem, smem + STAGE, ta1, tb1, min(kbeg + (it + 3) * kBK, klast));
    step64(smem + STAGE, smem, ta0, tb0, min(kbeg + (it + 4) * kBK, klast));
  }
  if (it < nk) step64(smem, smem + STAGE, ta1, tb1, klast);

  // epilogue: lane holds C[m = mrow][n = n0 + ... + 8q + 4 * lhalf + (0..3)] in acc[i][j][4q .. 4q+3]
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    const int64_t m = (LOCAL ? 0 : m0) + wm * WM + 32 * i + lrow;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = (LOCAL ? 0 : n0) + wn * WN + 32 * j + 8 * q + 4 * lhalf;
        // edge tiles: rows past M and columns past N (groups of 4, N a multiple of 8) are not stored
        if (!LOCAL && (m >= g.M || n >= g.N)) continue;
        if constexpr (OUT_F32) {
          float* c = static_cast<float*>(cout) + m * ldc + n;
          f32x4_t v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          *reinterpret_cast<f32x4_t*>(c) = v;
        } else {
          uint16_t* c = static_cast<uint16_t*>(cout) + m * ldc + n;
          f32x2_t lo = {acc[i][j][4 * q], acc[i][j][4 * q + 1]};
          f32x2_t hi = {acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          bf16x2_t blo = __builtin_convertvector(lo, bf16x2_t);
          bf16x2_t bhi = __builtin_convertvector(hi, bf16x2_t);
          u32x2_t w = {__builtin_bit_cast(unsigned, blo), __builtin_bit_cast(unsigned, bhi)};
          *reinterpret_cast<u32x2_t*>(c) = w;
        }
      }
    }
  }
}

// SK false: one workgroup per (split, tile); true: the stream-K schedule over gridDim.x workgroups.
template <int BM, int BN, bool A_MN, bool B_MN, bool OUT_F32, bool SK>
__global__ __launch_bounds__(kThreads, 1) void gemm_bf16_kernel(GemmArgs g) {
  constexpr int STAGE = opnd_bytes<BM>() + opnd_bytes<BN>();
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];
  // workgroups reach the 8 XCDs round-robin: give each XCD a contiguous run of work.  XCD x receives the
  // workgroups x, x + 8, ...: total / 8 of them, one more when x < total % 8, mapped to one run of indices.
  const int total = (int)gridDim.x;
  int bid = (int)blockIdx.x;
  {
    const int q = total >> 3, r = total & 7, x = bid & 7;
    bid = x * q + (x < r ? x : r) + (bid >> 3);
  }
  const int ntile = g.tiles_m * g.tiles_n;
  if constexpr (SK) {
    const int64_t I = (int64_t)ntile * g.nk, G = total;
    int64_t lo = (int64_t)bid * I / G;
    const int64_t hi = ((int64_t)bid + 1) * I / G;
    while (lo < hi) {
      const int t = (int)(lo / g.nk);
      const int64_t end = min(hi, ((int64_t)t + 1) * g.nk);
      float* part = static_cast<float*>(g.C) + ((int64_t)t + bid) * (BM * BN);
      gemm_tile<BM, BN, A_MN, B_MN, true, true>(g, smem, t, (int)(lo - (int64_t)t * g.nk),
                                                (int)(end - (int64_t)t * g.nk), part, BN);
      lo = end;
    }
  } else {
    const int split = bid / ntile;
    const int t = bid - split * ntile;
    const int it0 = (int)(((int64_t)split * g.nk) / g.splits);
    const int it1 = (int)(((int64_t)(split + 1) * g.nk) / g.splits);
    void* c = OUT_F32 ? static_cast<void*>(static_cast<float*>(g.C) + (int64_t)split * g.split_stride) : g.C;
    gemm_tile<BM, BN, A_MN, B_MN, OUT_F32, false>(g, smem, t, it0, it1, c, g.ldc);
  }
}

// out[m, n] = sum over s of part[s, m, n], in split order; 8 outputs per thread.
template <bool OUT_F32>
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const float* __restrict__ part, int64_t split_stride,
                                                          int splits, int M, int N, void* __restrict__ out,
                                                          int64_t ldo) {
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (idx >= (int64_t)M * N) return;
  const int64_t m = idx / N, n = idx - m * N;
  const float* p = part + idx;
  f32x4_t a = *reinterpret_cast<const f32x4_t*>(p), b = *reinterpret_cast<const f32x4_t*>(p + 4);
  for (int s = 1; s < splits; ++s) {
    const float* q = p + s * split_stride;
    a += *reinterpret_cast<const f32x4_t*>(q);
    b += *reinterpret_cast<const f32x4_t*>(q + 4);
  }
  if constexpr (OUT_F32) {
    float* o = static_cast<float*>(out) + m * ldo + n;
    *reinterpret_cast<f32x4_t*>(o) = a;
    *reinterpret_cast<f32x4_t*>(o + 4) = b;
  } else {
    u32x4_t w;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      f32x2_t x = {a[2 * e], a[2 * e + 1]}, y = {b[2 * e], b[2 * e + 1]};
      w[e] = __builtin_bit_cast(unsigned, __builtin_convertvector(x, bf16x2_t));
      w[e + 2] = __builtin_bit_cast(unsigned, __builtin_convertvector(y, bf16x2_t));
    }
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(out) + m * ldo + n) = w;
  }
}

// out[m, n] = sum over the stream-K segments of (m, n)'s tile, in workgroup order; 8 outputs per thread
// (BN is a multiple of 8, so they share a tile).
template <bool OUT_F32>
__global__ __launch_bounds__(256) void gemm_streamk_reduce(const float* __restrict__ part, int bm, int bn,
                                                           int tiles_m, int tiles_n, int nk, int groups, int M,
                                                           int N, void* __restrict__ out, int64_t ldo) {
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (idx >= (int64_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx - (int64_t)m * N);
  const int tm = m / bm, tn = n / bn;
  const int64_t t = tile_index(tm, tn, tiles_m, tiles_n);
  const int64_t I = (int64_t)tiles_m * tiles_n * nk;
  const int64_t w0 = sk_first(t, nk, I, groups), w1 = sk_last(t, nk, I, groups);
  const int64_t tsz = (int64_t)bm * bn;
  const float* p = part + (t + w0) * tsz + (int64_t)(m - tm * bm) * bn + (n - tn * bn);
  f32x4_t a = *reinterpret_cast<const f32x4_t*>(p), b = *reinterpret_cast<const f32x4_t*>(p + 4);
  for (int64_t w = w0 + 1; w <= w1; ++w) {
    p += tsz;
    a += *reinterpret_cast<const f32x4_t*>(p);
    b += *reinterpret_cast<const f32x4_t*>(p + 4);
  }
  if constexpr (OUT_F32) {
    float* o = static_cast<float*>(out) + (int64_t)m * ldo + n;
    *reinterpret_cast<f32x4_t*>(o) = a;
    *reinterpret_cast<f32x4_t*>(o + 4) = b;
  } else {
    u32x4_t wv;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      f32x2_t x = {a[2 * e], a[2 * e + 1]}, y = {b[2 * e], b[2 * e + 1]};
      wv[e] = __builtin_bit_cast(unsigned, __builtin_convertvector(x, bf16x2_t));
      wv[e + 2] = __builtin_bit_cast(unsigned, __builtin_convertvector(y, bf16x2_t));
    }
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(out) + (int64_t)m * ldo + n) = wv;
  }
}

template <int BM, int BN, bool A_MN, bool B_MN>
hipError_t launch_tile(const GemmArgs& g, bool out_f32, hipStream_t st) {
  if (g.splits == GEMM_STREAM_K) {
    hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, A_MN, B_MN, true, true>), dim3(kStreamKGroups), dim3(kThreads), 0,
                       st, g);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)(g.tiles_m * g.tiles_n * g.splits));
  if (out_f32)
    hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, A_MN, B_MN, true, false>), grid, dim3(kThreads), 0, st, g);
  else
    hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, A_MN, B_MN, false, false>), grid, dim3(kThreads), 0, st, g);
  return hipGetLastError();
}

template <bool A_MN, bool B_MN>
hipError_t launch_layout(int tile, const GemmArgs& g, bool out_f32, hipStream_t st) {
  switch (tile) {
    case GEMM_TILE_256x256: return launch_tile<256, 256, A_MN, B_MN>(g, out_f32, st);
    case GEMM_TILE_256x192: return launch_tile<256, 192, A_MN, B_MN>(g, out_f32, st);
    case GEMM_TILE_192x256: return launch_tile<192, 256, A_MN, B_MN>(g, out_f32, st);
    case GEMM_TILE_256x128: return launch_tile<256, 128, A_MN, B_MN>(g, out_f32, st);
    case GEMM_TILE_128x256: return launch_tile<128, 256, A_MN, B_MN>(g, out_f32, st);
    case GEMM_TILE_128x128: return launch_tile<128, 128, A_MN, B_MN>(g, out_f32, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

void gemm_tile_dims(int tile, int* bm, int* bn) {
  static const int dims[GEMM_TILE_COUNT][2] = {{256, 256}, {256, 192}, {192, 256}, {256, 128}, {128, 256}, {128, 128}};
  *bm = dims[tile][0];
  *bn = dims[tile][1];
}

hipError_t gemm_bf16(const GemmProblem& p, hipStream_t st) {
  int bm, bn;
  gemm_tile_dims(p.tile, &bm, &bn);
  GemmArgs g;
  g.A = static_cast<const uint16_t*>(p.A);
  g.B = static_cast<const uint16_t*>(p.B);
  g.lda = p.lda;
  g.ldb = p.ldb;
  g.a_elems = p.a_mn ? (p.K - 1) * p.lda + p.M : (p.M - 1) * p.lda + p.K;
  g.b_elems = p.b_mn ? (p.K - 1) * p.ldb + p.N : (p.N - 1) * p.ldb + p.K;
  g.M = (int)p.M;
  g.N = (int)p.N;
  g.nk = (int)(p.K / kBK);
  g.splits = p.splits;
  g.tiles_m = (int)((p.M + bm - 1) / bm);   // the last row / column tile may be partial
  g.tiles_n = (int)((p.N + bn - 1) / bn);
  const bool sk = p.splits == GEMM_STREAM_K;
  const bool direct = p.splits == 1;
  const bool f32 = p.out_f32 || !direct;
  if (sk) {
    g.C = p.workspace;
    g.ldc = bn;
    g.split_stride = 0;
  } else if (direct) {
    g.C = p.C;
    g.ldc = p.ldc;
    g.split_stride = 0;
  } else {
    g.C = p.workspace;
    g.ldc = p.N;
    g.split_stride = p.M * p.N;
  }
  hipError_t e;
  const int lay = (p.a_mn ? 2 : 0) | (p.b_mn ? 1 : 0);
  switch (lay) {
    case 0: e = launch_layout<false, false>(p.tile, g, f32, st); break;
    case 1: e = launch_layout<false, true>(p.tile, g, f32, st); break;
    case 2: e = launch_layout<true, false>(p.tile, g, f32, st); break;
    default: e = launch_layout<true, true>(p.tile, g, f32, st); break;
  }
  if (e != hipSuccess || direct) return e;
  const int64_t n8 = p.M * p.N / 8;
  const dim3 grid((unsigned)((n8 + 255) / 256));
  if (sk) {
    if (p.out_f32)
      hipLaunchKernelGGL((gemm_streamk_reduce<true>), grid, dim3(256), 0, st, static_cast<const float*>(p.workspace),
                         bm, bn, g.tiles_m, g.tiles_n, g.nk, kStreamKGroups, g.M, g.N, p.C, p.ldc);
    else
      hipLaunchKernelGGL((gemm_streamk_reduce<false>), grid, dim3(256), 0, st, static_cast<const float*>(p.workspace),
                         bm, bn, g.tiles_m, g.tiles_n, g.nk, kStreamKGroups, g.M, g.N, p.C, p.ldc);
    return hipGetLastError();
  }
  if (p.out_f32)
    hipLaunchKernelGGL((gemm_splitk_reduce<true>), grid, dim3(256), 0, st, static_cast<const float*>(p.workspace),
                       g.split_stride, p.splits, g.M, g.N, p.C, p.ldc);
  else
    hipLaunchKernelGGL((gemm_splitk_reduce<false>), grid, dim3(256), 0, st, static_cast<const float*>(p.workspace),
                       g.split_stride, p.splits, g.M, g.N, p.C, p.ldc);
  return hipGetLastError();
}

}  // namespace pom
