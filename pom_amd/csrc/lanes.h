// Lane -> channel mapping shared by the aggregation and gating kernels.
//
// Plain mode: a lane owns CPT consecutive channels [vcol*CPT, vcol*CPT+CPT).
// RoPE modes: a lane owns CPT consecutive rotation pairs; slot i < CPT is the
// first channel of pair i, slot CPT+i its partner.
//   1-D (pom/pom_rope.py:152-180): pair j = (j, j + P/2), table column j.
//   2-D (pom/pom_rope.py:183-235): q = P/4; pair j < q = (j, j+q) on the row
//        tables, pair j >= q = (2q + j', 3q + j'), j' = j - q, on the column
//        tables.
#pragma once
#include "common.h"
#include "pom_internal.h"

namespace pom {

// Parameter element i in fp32 / stored from fp32, in the parameter's dtype.
__device__ __forceinline__ float param_get(const ParamIn& a, int64_t i) {
  if (a.dt == DT_BF16) return to_f32<__hip_bfloat16>(static_cast<const __hip_bfloat16*>(a.ptr)[i]);
  if (a.dt == DT_F16) return to_f32<__half>(static_cast<const __half*>(a.ptr)[i]);
  return static_cast<const float*>(a.ptr)[i];
}
// out[q] = a[idx(q)] in fp32 for q < N, with one dtype dispatch around all the
// loads: a dispatch per element (param_get) puts each load's wait inside its
// branch, so the loads of a lane run one after another.  idx(q) must be a valid
// element index for every q.
template <int N, typename Idx>
__device__ __forceinline__ void param_gather(const ParamIn& a, Idx&& idx, float (&out)[N]) {
  auto run = [&](auto tag) {
    using PT = decltype(tag);
    const PT* s = static_cast<const PT*>(a.ptr);
    PT raw[N];
#pragma unroll
    for (int q = 0; q < N; ++q) raw[q] = s[idx(q)];
#pragma unroll
    for (int q = 0; q < N; ++q) out[q] = to_f32<PT>(raw[q]);
  };
  if (a.dt == DT_BF16) run(__hip_bfloat16{});
  else if (a.dt == DT_F16) run(__half{});
  else run(float{});
}

__device__ __forceinline__ void param_set(const ParamOut& a, int64_t i, float v) {
  if (a.dt == DT_BF16) static_cast<__hip_bfloat16*>(a.ptr)[i] = from_f32<__hip_bfloat16>(v);
  else if (a.dt == DT_F16) static_cast<__half*>(a.ptr)[i] = from_f32<__half>(v);
  else static_cast<float*>(a.ptr)[i] = v;
}


// Channel mapping for one lane: slot i in [0, CPT2) -> channel index.
template <int CPT, int MODE>
struct LaneMap {
  static constexpr int LAY = mode_layout(MODE);
  static constexpr int CPT2 = (LAY == MODE_ROPE1D || LAY == MODE_ROPE2D) ? 2 * CPT : CPT;
  int64_t c1 = 0, c2 = 0, tcol = 0;
  int table = 0;   // 0 = row / 1-D tables, 1 = column tables (2-D)

  __device__ __forceinline__ void init(int64_t vcol, int64_t P) {
    if constexpr (LAY == MODE_ROPE1D) {
      const int64_t j = vcol * CPT;
      c1 = j; c2 = j + P / 2; tcol = j;
    } else if constexpr (LAY == MODE_ROPE2D) {
      const int64_t q = P / 4, j = vcol * CPT;
      if (j < q) { c1 = j; c2 = j + q; tcol = j; table = 0; }
      else { const int64_t jj = j - q; c1 = 2 * q + jj; c2 = 3 * q + jj; tcol = jj; table = 1; }
    } else {
      c1 = vcol * CPT;
    }
  }
  __device__ __forceinline__ int64_t chan(int i) const {
    if constexpr (CPT2 == CPT) return c1 + i;
    else return i < CPT ? c1 + i : c2 + (i - CPT);
  }
};

// RoPE mapping with one lane per half of a rotation pair (the aggregation
// backward's): a lane owns CPT consecutive channels [c1, c1 + CPT), all first
// or all second halves of CPT consecutive pairs.  cp is the partner half's
// first channel and sign the sign of the partner's term in the transposed
// rotation: a first half's upstream weight is w cos + w_partner sin, a
// second half's w cos - w_partner sin.
//   1-D: channels [0, P/2) are first halves (partner c + P/2), table column c.
//   2-D: q = P/4; [0, q) and [q, 2q) are the first and second halves on the
//        row tables, [2q, 3q) and [3q, 4q) on the column tables.
// A lane never straddles two blocks: CPT divides P/2 (1-D) or P/4 (2-D).
template <int CPT, int MODE>
struct HalfMap {
  static constexpr int LAY = mode_layout(MODE);
  int64_t c1 = 0, cp = 0, tcol = 0;
  int table = 0;
  float sign = 1.0f;

  __device__ __forceinline__ void init(int64_t vcol, int64_t P) {
    c1 = vcol * CPT;
    const int64_t q = LAY == MODE_ROPE1D ? P / 2 : P / 4;
    const int64_t blk = c1 / q;
    const bool second = (blk & 1) != 0;
    table = LAY == MODE_ROPE1D ? 0 : (int)(blk >> 1);
    tcol = c1 - blk * q;
    cp = second ? c1 - q : c1 + q;
    sign = second ? -1.0f : 1.0f;
  }
  __device__ __forceinline__ int64_t chan(int i) const { return c1 + i; }
};

// Slot s of the partial buffers -> channel (same mapping as LaneMap).
template <int CPT, int MODE>
__device__ __forceinline__ int64_t slot_chan(int64_t s, int64_t P) {
  constexpr int CPT2 = LaneMap<CPT, MODE>::CPT2;
  LaneMap<CPT, MODE> m;
  m.init(s / CPT2, P);
  return m.chan((int)(s % CPT2));
}

// cos/sin of token n for CPT consecutive rotation pairs starting at table column
// tcol.  A position p in [-rows, 0) selects row p + rows, as torch's indexing of
// the tables does (pom/pom_rope.py:173-174, :211-212); positions still outside
// the table are clamped, so a bad position can never read outside it (the host
// rejects them where it can check them without a device sync).
// The two halves of the lookup: the position (a load that the streaming
// kernels issue together with the step's row loads) and the table entries
// at that position.
__device__ __forceinline__ int rope_pos(const RopeTables& t, int table, int64_t n) {
  const int64_t v = t.pos[n * t.pos_sn + table];
  // saturated to int: the table lookup sees the same side of the table
  return v < -0x7fffffff ? -0x7fffffff : (v > 0x7fffffff ? 0x7fffffff : (int)v);
}

__device__ __forceinline__ int64_t table_row(int64_t pos, int64_t rows) {
  const int64_t r = pos < 0 ? pos + rows : pos;
  return r < 0 ? 0 : (r >= rows ? rows - 1 : r);
}

template <int CPT>
__device__ __forceinline__ void load_table_at(const RopeTables& t, int table, int pos, int64_t tcol,
                                              float (&cs)[CPT], float (&sn)[CPT]) {
  const int64_t r = table_row(pos, table ? t.rows1 : t.rows0);
  load_f32<CPT>((table ? t.cos1 : t.cos0) + r * t.stride + tcol, cs);
  load_f32<CPT>((table ? t.sin1 : t.sin0) + r * t.stride + tcol, sn);
}

template <int CPT>
__device__ __forceinline__ void load_table(const RopeTables& t, int table, int64_t n, int64_t tcol,
                                           float (&cs)[CPT], float (&sn)[CPT]) {
  const int64_t r = table_row(t.pos[n * t.pos_sn + table], table ? t.rows1 : t.rows0);
  load_f32<CPT>((table ? t.cos1 : t.cos0) + r * t.stride + tcol, cs);
  load_f32<CPT>((table ? t.sin1 : t.sin0) + r * t.stride + tcol, sn);
}

}  // namespace pom
