// Fused activation + polynomial expansion + sequence aggregation (forward and
// backward) for the Polynomial Mixer, written for gfx950 (CDNA4).
//
// One kernel family covers the reference's mean, masked, frame-causal and RoPE
// aggregations (pom/pom_triton.py:68-321, pom/pom_triton_masked.py:72-345,
// pom/pom.py:233-262 + :41-45, pom/pom_triton_rope.py:93-475,
// pom/pom_rope.py:242-296).
//
// Work decomposition:
//   grid = (slabs, chunks, B), 256 threads (4 waves) per workgroup.
//   A workgroup streams the rows of one chunk of one batch row through one
//   channel slab.  Within a wave, 2^lpr_log2 lanes cover one token row (each
//   lane cpt consecutive units, one 16-byte load for bf16) and 64/2^lpr_log2
//   rows are processed side by side; the four waves interleave rows.  Loads of
//   U rows are issued before any arithmetic so every lane keeps U 16-byte
//   loads in flight.  Accumulation is fp32 in registers.
//   At the end, lanes sharing a column are summed with cross-lane shuffles,
//   the four waves through LDS, and the chunk's result is written either as
//   the final output (one chunk per batch row) or as an fp32 partial that a
//   finalize kernel sums in a fixed order.  No floating-point atomics and no
//   inter-workgroup synchronisation: results are deterministic run to run.
//
// Frames: tokens are grouped in F frames of L tokens (F = 1 for the plain
// mean).  The finalize kernel turns frame sums into frame means and runs the
// running-mean recurrence of PoM.state_forward across frames
// (pom/pom.py:255-259) with the reference's rounding in the element type, so
// a full-sequence frame-causal call and the frame-by-frame state_forward loop
// produce identical bits.
#pragma once

#include "common.h"
#include "pom_internal.h"
#include "lanes.h"

namespace pom {

struct LaneGeom {
  int tid, wave, lane, lb, lpr, rpw, rs, lrow, lcol;
  __device__ __forceinline__ explicit LaneGeom(int lpr_log2) {
    tid = threadIdx.x;
    wave = tid / kWave;
    lane = tid % kWave;
    lb = lpr_log2;
    lpr = 1 << lb;
    rpw = kWave >> lb;          // rows per wave step
    rs = kWaves * rpw;          // rows per workgroup step
    lrow = lane >> lb;
    lcol = lane & (lpr - 1);
  }
};

// Row range of chunk `chunk` (frames never straddled).
__device__ __forceinline__ void chunk_rows(const Geom& g, int64_t chunk, int64_t N, int64_t& f, int64_t& rbeg,
                                           int64_t& rend) {
  f = chunk / g.cpf;
  rbeg = f * g.L + (chunk - f * g.cpf) * g.RC;
  const int64_t fe = (f + 1) * g.L;
  rend = rbeg + g.RC < fe ? rbeg + g.RC : fe;
  if (rend > N) rend = N;
}

template <int MODE>
struct Mode_ {
  static constexpr bool rope = (mode_layout(MODE) == MODE_ROPE1D || mode_layout(MODE) == MODE_ROPE2D);
  static constexpr int U = rope ? 4 : 8;   // rows in flight per lane
};

// Rows of a chunk as seen by one lane: step `it` covers rows
// base + row0 + u * rs (u < U), base = it * rs * U.  Every step but the last
// is full; the last clamps its row indices into the chunk (so every load
// stays in bounds and is issued without a branch) and its compute drops the
// rows past the end.
//
// RowWalk::consecutive gives each lane U adjacent rows instead
// (row base + row0 * U + u): the kernels that also write a channel-major copy
// of their output use it, so a lane holds U consecutive tokens of each of its
// channels, one vector write per channel into the staging tile.
struct RowWalk {
  int64_t rbeg, nrows, step;
  int row0, rs;
  __device__ __forceinline__ RowWalk(int64_t rbeg_, int64_t rend_, int row0_, int rs_, int U)
      : rbeg(rbeg_), nrows(rend_ - rbeg_), step((int64_t)rs_ * U), row0(row0_), rs(rs_) {}
  __device__ __forceinline__ static RowWalk consecutive(int64_t rbeg_, int64_t rend_, int row0_, int rs_, int U) {
    RowWalk w(rbeg_, rend_, row0_ * U, 1, U);
    w.step = (int64_t)rs_ * U;
    return w;
  }
  __device__ __forceinline__ int64_t full_steps() const { return nrows / step; }
  __device__ __forceinline__ bool has_tail() const { return full_steps() * step < nrows; }
  __device__ __forceinline__ bool valid(int64_t base, int u) const { return base + row0 + (int64_t)u * rs < nrows; }
  // absolute row; clamped into the chunk when `clamp`
  __device__ __forceinline__ int64_t row(int64_t base, int u, bool clamp) const {
    int64_t rel = base + row0 + (int64_t)u * rs;
    if (clamp && rel >= nrows) rel = nrows - 1;
    return rbeg + rel;
  }
};

// Walk over a chunk's steps: load(buf, base, clamp) fills buf with the rows
// of the step at `base` (clamped into the chunk for the tail step), then
// work(buf, base, tail_tag) consumes them.  The step count is the same for
// every lane of the workgroup, so work() may synchronise the workgroup.
template <typename Buf, typename Load, typename Work>
__device__ __forceinline__ void walk_rows(const RowWalk& W, Load&& load, Work&& work) {
  const int64_t nfull = W.full_steps();
  for (int64_t it = 0; it < nfull; ++it) {
    Buf bf;
    load(bf, it * W.step, false);
    work(bf, it * W.step, std::false_type{});
  }
  if (W.has_tail()) {
    Buf bf;
    load(bf, nfull * W.step, true);
    work(bf, nfull * W.step, std::true_type{});
  }
}

// A compiler fence for memory operations (no instruction is emitted): no
// load or store is moved across it by any pass, where a sched_barrier holds
// only in the machine scheduler.  Used after a step's loads so that each is
// issued there rather than sunk to its first use and waited for on the spot.
__device__ __forceinline__ void mem_fence_compiler() { asm volatile("" ::: "memory"); }

// walk_rows with a prefetch stage for loads whose addresses depend on other
// loads (RoPE: a row's table entries on its position).  pre(pb, base) loads
// the addresses of the step at `base` (rows clamped into the chunk) one step
// ahead, so load(bf, pb, base, clamp) issues the dependent loads at once,
// next to the row loads.  Vector memory operations complete in issue order,
// so a load is waited for together with everything issued before it: the
// prefetch is issued with the step's loads, before the step's stores, and
// the next step waits for it without waiting for those.  load() must end
// with a fence for memory operations (mem_fence_compiler) so that no pass
// moves the prefetch after the stores.  The chunk must hold at least one row.
template <typename Buf, typename Pre, typename PreLoad, typename Load, typename Work>
__device__ __forceinline__ void walk_rows_pre(const RowWalk& W, PreLoad&& pre, Load&& load, Work&& work) {
  const int64_t nfull = W.full_steps();
  Pre pc;
  pre(pc, 0);
  for (int64_t it = 0; it < nfull; ++it) {
    Pre pn;
    Buf bf;
    pre(pn, (it + 1) * W.step);
    load(bf, pc, it * W.step, false);
    work(bf, it * W.step, std::false_type{});
    pc = pn;
  }
  if (W.has_tail()) {
    Buf bf;
    load(bf, pc, nfull * W.step, true);
    work(bf, nfull * W.step, std::true_type{});
  }
}

// walk_rows with the next step's row loads issued before the current step's
// arithmetic and stores (two buffers in registers): a step's stores are then
// never ahead of the loads the following step waits for, which vector memory's
// in-order completion would otherwise make it wait for too.  The last step is
// peeled, so nothing is loaded past the chunk.
template <typename Buf, typename Load, typename Work>
__device__ __forceinline__ void walk_rows_pipe(const RowWalk& W, Load&& load, Work&& work) {
  if (W.nrows <= 0) return;
  const int64_t nfull = W.full_steps();
  const int64_t nsteps = nfull + (W.has_tail() ? 1 : 0);
  Buf cur;
  load(cur, 0, nfull == 0);
  for (int64_t it = 0; it + 1 < nsteps; ++it) {   // step `it` is full: only the last can be partial
    Buf nxt;
    load(nxt, (it + 1) * W.step, true);
    mem_fence_compiler();
    work(cur, it * W.step, std::false_type{});
    cur = nxt;
  }
  if (W.has_tail()) work(cur, nfull * W.step, std::true_type{});
  else work(cur, (nfull - 1) * W.step, std::false_type{});
}

// Channel-major copy of one workgroup step, staged through LDS.  The step
// covers tokens [tok0, tok0 + S) of batch row b, S = kWaves * rpw * U, for
// the lpr * NS channel slots of the slab; each lane holds U consecutive tokens
// of its NS slots (RowWalk::consecutive).  Lanes write their U x NS block into
// an LDS tile (one row per slot), then the workgroup stores the tile row by
// row: a store instruction writes runs of S tokens of one channel (512 bytes
// for bf16 at U = 8) where direct stores from the lanes would write 128-byte
// pieces of eight channel rows each, which measured 2-3x slower.
// chan(l, i): channel of slot i of lane column l, or -1 past the channels.
// nvalid: tokens of the step inside the chunk.  Every wave of the workgroup
// calls it once per step (it synchronises the workgroup).
// Channel of slot i of lane column l of a slab (LaneMap), or -1 past the channels.
template <int CPT, int MODE>
__device__ __forceinline__ int64_t slab_chan(int64_t slab, int lpr, int64_t nvec, int64_t P, int l, int i) {
  const int64_t vc = slab * lpr + l;
  if (vc >= nvec) return -1;
  LaneMap<CPT, MODE> m;
  m.init(vc, P);
  return m.chan(i);
}

template <int U, int NS>
struct TrTile {
  static constexpr int kElems = kWaves * kWave * U * NS + 8 * kMaxLpr * NS;
};

template <typename T, int U, int NS, typename Chan>
__device__ __forceinline__ void store_tr_staged(const TrOut& t, const LaneGeom& G, int64_t b, int64_t tok0,
                                                int64_t nvalid, const Chan& chan, const float (&v)[U][NS],
                                                T* tile) {
  const int S = kWaves * G.rpw * U;          // tokens per step
  const int pitch = S + 8;                   // elements; rows start on distinct banks
  const int R = G.lpr * NS;                  // channel slots of the slab
  __syncthreads();                           // the previous step's readers are done
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    float col[U];
#pragma unroll
    for (int u = 0; u < U; ++u) col[u] = v[u][i];
    VecIO<T, U>::store(tile + (G.lcol * NS + i) * pitch + (G.wave * G.rpw + G.lrow) * U, col);
  }
  __syncthreads();
  using Raw = typename RawVec<16>::type;
  T* base = reinterpret_cast<T*>(t.data) + b * t.sb + tok0;
  const bool vec = t.ld % 8 == 0 && reinterpret_cast<uintptr_t>(base) % 16 == 0;
  const int CR = S / 8;                      // 16-byte chunks per tile row
  for (int idx = G.tid; idx < R * CR; idx += kThreads) {
    const int row = idx / CR, c = idx - row * CR;
    const int64_t ch = chan(row / NS, row % NS);
    const int tok = c * 8;
    if (ch < 0 || tok >= nvalid) continue;
    const T* src = tile + row * pitch + tok;
    T* dst = base + ch * t.ld + tok;
    if (vec && tok + 8 <= nvalid) {
      *reinterpret_cast<Raw*>(dst) = *reinterpret_cast<const Raw*>(src);
    } else {
      for (int e = 0; e < 8 && tok + e < nvalid; ++e) dst[e] = src[e];
    }
  }
}

// Zeros in the channel-major copy for tokens [n_lo, n_hi) of batch row b and
// the nch channels starting at c0 (rows a masked kernel never loads).
template <typename T>
__device__ __forceinline__ void zero_tr(const TrOut& t, int64_t b, int64_t n_lo, int64_t n_hi,
                                        int64_t c0, int64_t nch) {
  T* base = reinterpret_cast<T*>(t.data) + b * t.sb;
  for (int64_t c = 0; c < nch; ++c)
    for (int64_t n = n_lo + threadIdx.x; n < n_hi; n += kThreads) base[(c0 + c) * t.ld + n] = from_f32<T>(0.0f);
}

// Masked mode: the chunk's first and last rows with a nonzero weight and the
// sum of its weights, from one pass over the chunk's mask entries.  Rows
// outside [first, last] are never loaded.
__device__ __forceinline__ void mask_extent(const AggParams& p, int64_t b, int64_t rbeg, int64_t rend,
                                            int64_t& first, int64_t& last, float& total) {
  __shared__ int64_t s_first[kWaves], s_last[kWaves];
  __shared__ float s_tot[kWaves];
  int64_t lo = rend, hi = rbeg - 1;
  float t = 0.0f;
  for (int64_t n = rbeg + threadIdx.x; n < rend; n += kThreads) {
    const float m = p.mask[b * p.msb + n * p.msn];
    if (m != 0.0f) {
      lo = n < lo ? n : lo;
      hi = n > hi ? n : hi;
      t += m;
    }
  }
  for (int off = 1; off < kWave; off <<= 1) {
    const int64_t olo = __shfl_xor(lo, off, kWave), ohi = __shfl_xor(hi, off, kWave);
    lo = olo < lo ? olo : lo;
    hi = ohi > hi ? ohi : hi;
    t += __shfl_xor(t, off, kWave);
  }
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    s_first[wave] = lo;
    s_last[wave] = hi;
    s_tot[wave] = t;
  }
  __syncthreads();
  first = s_first[0];
  last = s_last[0];
  total = s_tot[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    first = s_first[w] < first ? s_first[w] : first;
    last = s_last[w] > last ? s_last[w] : last;
    total += s_tot[w];
  }
}

// ---------------------------------------------------------------------------
// Forward chunk kernel
// ---------------------------------------------------------------------------
template <typename T, int CPT, int KM, int MODE>
__global__ void __launch_bounds__(kThreads) agg_fwd_chunk(const AggParams p) {
  using Map = LaneMap<CPT, MODE>;
  constexpr int CPT2 = Map::CPT2;
  constexpr bool ROPE = Mode_<MODE>::rope;
  constexpr bool MASKED = mode_masked(MODE);
  // the plain mode walks pipelined (walk_rows_pipe): 4 rows a step, 8 in flight
  // (the masked forward measured slower pipelined: C3 54.0 against 48.9 us)
  constexpr bool PIPE = !ROPE && !MASKED;
  constexpr int U = PIPE ? 4 : Mode_<MODE>::U;
  __shared__ float red[kWaves][kMaxLpr * CPT2];

  const LaneGeom G(p.g.lpr_log2);
  const int64_t slab = blockIdx.x, chunk = blockIdx.y, b = blockIdx.z;
  int64_t f, rbeg, rend;
  chunk_rows(p.g, chunk, p.N, f, rbeg, rend);
  float total = 0.0f;
  if constexpr (MASKED) {
    int64_t first, last;
    mask_extent(p, b, rbeg, rend, first, last, total);
    rbeg = first;
    rend = last >= first ? last + 1 : first;   // empty when the chunk has no valid row
  }
  const int64_t vcol = slab * G.lpr + G.lcol;
  const bool active = vcol < p.g.nvec;
  Map map;
  map.init(active ? vcol : 0, p.P);

  float c[CPT2][KM];
  {
    float flat[CPT2 * KM];
    param_gather<CPT2 * KM>(p.coeff, [&](int q) {
      const int j = q % KM;
      return map.chan(q / KM) * p.K + (j < p.K ? j : p.K - 1);
    }, flat);
#pragma unroll
    for (int i = 0; i < CPT2; ++i)
#pragma unroll
      for (int j = 0; j < KM; ++j) c[i][j] = (active && j < p.K) ? flat[i * KM + j] : 0.0f;
  }

  float acc[CPT2];
#pragma unroll
  for (int i = 0; i < CPT2; ++i) acc[i] = 0.0f;

  const T* xb = reinterpret_cast<const T*>(p.x) + b * p.sxb;
  const RowWalk W(rbeg, rend, G.wave * G.rpw + G.lrow, G.rs, U);

  struct Buf {
    Pack<T, CPT> v1[U], v2[ROPE ? U : 1];
    float wv[MASKED ? U : 1];
  };
  auto load = [&](Buf& bf, int64_t base, bool clamp) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t rr = W.row(base, u, clamp);
      const T* row = xb + rr * p.sxn;
      bf.v1[u].load_stream(row + map.c1);
      if constexpr (ROPE) bf.v2[u].load_stream(row + map.c2);
      if constexpr (MASKED) bf.wv[u] = p.mask[b * p.msb + rr * p.msn];
    }
  };
  auto step = [&](const Buf& bf, int64_t base, auto tail_tag) {
    constexpr bool TAIL = decltype(tail_tag)::value;
    const auto& v1 = bf.v1;
    const auto& v2 = bf.v2;
    const auto& wv = bf.wv;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      bool keep = !TAIL || W.valid(base, u);
      if constexpr (MASKED) keep = keep && wv[u] != 0.0f;   // also drops NaN padding
      if constexpr (ROPE) {
        float cs[CPT], sn[CPT];
        load_table<CPT>(p.rope, map.table, W.row(base, u, TAIL), map.tcol, cs, sn);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          float h1 = act(v1[u].get(i)), h2 = act(v2[u].get(i));
          if (TAIL || MASKED) {
            h1 = keep ? h1 : 0.0f;
            h2 = keep ? h2 : 0.0f;
          }
          float p1 = poly<KM>(h1, c[i]);
          float p2 = poly<KM>(h2, c[CPT + i]);
          if constexpr (MASKED) {   // the mask weights the rotated features
            p1 *= wv[u];
            p2 *= wv[u];
          }
          acc[i] += p1 * cs[i] - p2 * sn[i];
          acc[CPT + i] += p2 * cs[i] + p1 * sn[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          float h = act(v1[u].get(i));
          if (TAIL || MASKED) h = keep ? h : 0.0f;   // p(0) = 0
          const float q = poly_q<KM>(h, c[i]);
          if constexpr (MASKED) acc[i] = fmaf(q, h * wv[u], acc[i]);
          else acc[i] = fmaf(q, h, acc[i]);
        }
      }
    }
  };

  if (active) {
    if constexpr (PIPE) walk_rows_pipe<Buf>(W, load, step);
    else walk_rows<Buf>(W, load, step);
  }

  // Rows -> one value per column: shuffles inside the wave, LDS across waves.
#pragma unroll
  for (int i = 0; i < CPT2; ++i) acc[i] = xor_sum_rows(acc[i], G.lb);
  if (G.lrow == 0) {
#pragma unroll
    for (int i = 0; i < CPT2; ++i) red[G.wave][G.lcol * CPT2 + i] = acc[i];
  }
  __syncthreads();
  const int nslot = G.lpr * CPT2;
  for (int s = G.tid; s < nslot; s += kThreads) {
    const int l = s / CPT2, i = s - l * CPT2;
    const int64_t vc = slab * G.lpr + l;
    if (vc >= p.g.nvec) continue;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) v += red[w][s];
    Map m2;
    m2.init(vc, p.P);
    const int64_t ch = m2.chan(i);
    if (p.direct) {
      float mean;
      if constexpr (MASKED) mean = total != 0.0f ? v / total : 0.0f;   // empty row -> 0
      else mean = v / (float)p.g.L;
      reinterpret_cast<T*>(p.out)[b * p.P + ch] = from_f32<T>(mean);
    } else {
      p.part[(b * p.g.nch + chunk) * p.P + ch] = v;
    }
  }
  if constexpr (MASKED) {
    if (slab == 0 && G.tid == 0) {
      if (p.direct) {
        if (p.count_out) p.count_out[b] = total;
      } else {
        p.pcnt[b * p.g.nch + chunk] = total;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Forward finalize: chunk sums -> frame means -> running-mean recurrence.
// One thread per (batch row, channel).
// ---------------------------------------------------------------------------
template <typename T, bool MASKED>
__global__ void __launch_bounds__(kThreads) agg_fwd_finalize(const AggParams p) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= p.B * p.P) return;
  const int64_t b = idx / p.P, c = idx - b * p.P;
  const int64_t nch = p.g.nch, cpf = p.g.cpf, F = p.g.F;
  const float* part = p.part + b * nch * p.P + c;
  float cnt = 0.0f;
  if (MASKED) {
    for (int64_t k = 0; k < nch; ++k) cnt += p.pcnt[b * nch + k];
    if (c == 0 && p.count_out) p.count_out[b] = cnt;
  }
  T* out = reinterpret_cast<T*>(p.out) + b * F * p.P + c;
  const bool recur = F > 1 || p.carry != nullptr;
  bool have = p.carry != nullptr;
  float h = have ? to_f32<T>(reinterpret_cast<const T*>(p.carry)[b * p.P + c]) : 0.0f;
  float n = (float)p.n_past;
  constexpr int FB = 8;   // frames whose partial loads are issued together
  for (int64_t f0 = 0; f0 < F; f0 += FB) {
    float sf[FB];
#pragma unroll
    for (int q = 0; q < FB; ++q) sf[q] = 0.0f;
    for (int64_t k = 0; k < cpf; ++k) {   // each frame's chunks summed in chunk order
      float v[FB];
#pragma unroll
      for (int q = 0; q < FB; ++q) v[q] = f0 + q < F ? part[((f0 + q) * cpf + k) * p.P] : 0.0f;
#pragma unroll
      for (int q = 0; q < FB; ++q) sf[q] += v[q];
    }
#pragma unroll
    for (int q = 0; q < FB; ++q) {
      const int64_t f = f0 + q;
      if (f >= F) break;
      const float m = MASKED ? (cnt != 0.0f ? sf[q] / cnt : 0.0f) : sf[q] / (float)p.g.L;
      if (!recur) {
        out[0] = from_f32<T>(m);
        return;
      }
      // The per-frame mean is a tensor of the element type in the reference
      // (pom/pom_triton.py:348) before it enters the recurrence.
      const float mt = round_to<T>(m);
      h = have ? running_mean_step<T>(h, mt, n) : mt;
      have = true;
      out[f * p.P] = from_f32<T>(h);
      n += 1.0f;
    }
  }
}

// ---------------------------------------------------------------------------
// Backward: per-frame token weights for F > 1 frames.
//   dM_f = sum_{g >= f} dH_g / (n_past + g + 1),   token weight = dM_f / L
// ---------------------------------------------------------------------------
static __global__ void __launch_bounds__(kThreads) agg_frame_weights(const AggParams p, float* wf) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= p.B * p.P) return;
  const int64_t b = idx / p.P, c = idx - b * p.P;
  const int64_t F = p.g.F;
  constexpr int FB = 8;   // frames whose loads are issued together (suffix order kept)
  float s = 0.0f;
  for (int64_t f1 = F - 1; f1 >= 0; f1 -= FB) {
    float v[FB];
#pragma unroll
    for (int q = 0; q < FB; ++q) v[q] = f1 - q >= 0 ? p.go[(b * F + f1 - q) * p.P + c] : 0.0f;
#pragma unroll
    for (int q = 0; q < FB; ++q) {
      const int64_t f = f1 - q;
      if (f < 0) break;
      s += v[q] / ((float)(p.n_past + f) + 1.0f);
      wf[(b * F + f) * p.P + c] = s / (float)p.g.L;
    }
  }
}

// ---------------------------------------------------------------------------
// Backward chunk kernel: grad_x for every row of the chunk (written into a
// strided view, e.g. the h-half of dY) and the chunk's grad_coeff partial.
// ---------------------------------------------------------------------------
// With the channel-major copy a lane holds U x CPT2 output values until the
// staged store, so that variant walks 4 rows per lane instead of 8.
template <typename T, int CPT, int KM, int MODE, bool TR>
__device__ __forceinline__ void agg_bwd_body(const AggParams& p) {
  using Map = LaneMap<CPT, MODE>;
  constexpr int CPT2 = Map::CPT2;
  constexpr bool ROPE = Mode_<MODE>::rope;
  constexpr bool MASKED = mode_masked(MODE);
  // with the channel-major copy: 4 rows in flight, 2 for RoPE (its pairs and
  // tile slots double the per-lane state; 4 fills all 256 VGPRs).  Without it
  // the walk is pipelined (walk_rows_pipe): 4 rows per step, 8 in flight.
  constexpr bool PIPE = !TR && !ROPE;
  constexpr int U = PIPE ? 4 : (TR ? (ROPE ? 2 : 4) : Mode_<MODE>::U);
  __shared__ float red[kWaves][kMaxLpr * CPT2];

  const LaneGeom G(p.g.lpr_log2);
  const int64_t slab = blockIdx.x, chunk = blockIdx.y, b = blockIdx.z;
  int64_t f, rbeg, rend;
  chunk_rows(p.g, chunk, p.N, f, rbeg, rend);
  const int64_t vcol = slab * G.lpr + G.lcol;
  const bool active = vcol < p.g.nvec;
  Map map;
  map.init(active ? vcol : 0, p.P);

  // d[i][j] = (j+1) c[i][j]; w = the gradient weight of one token of this frame.
  float d[CPT2][KM], g[CPT2][KM], w[CPT2];
  float cntv = 1.0f;
  if constexpr (MASKED) cntv = p.count_in[b];
  {
    float flat[CPT2 * KM];
    param_gather<CPT2 * KM>(p.coeff, [&](int q) {
      const int j = q % KM;
      return map.chan(q / KM) * p.K + (j < p.K ? j : p.K - 1);
    }, flat);
#pragma unroll
    for (int i = 0; i < CPT2; ++i)
#pragma unroll
      for (int j = 0; j < KM; ++j) {
        d[i][j] = (active && j < p.K) ? flat[i * KM + j] * (float)(j + 1) : 0.0f;
        g[i][j] = 0.0f;
      }
  }
  {
    // all weight loads first (one source for the whole lane), then the
    // per-mode arithmetic
    const float* wsrc = (!MASKED && p.wf) ? p.wf + (b * p.g.F + f) * p.P : p.go + b * p.P;
    float raw[CPT2];
#pragma unroll
    for (int i = 0; i < CPT2; ++i) raw[i] = wsrc[map.chan(i)];
#pragma unroll
    for (int i = 0; i < CPT2; ++i) {
      float wi;
      if constexpr (MASKED) wi = cntv != 0.0f ? raw[i] / cntv : 0.0f;
      else if (p.wf) wi = raw[i];
      else wi = (raw[i] / ((float)p.n_past + 1.0f)) / (float)p.g.L;
      w[i] = active ? wi : 0.0f;
    }
  }
  float w01[CPT2];
#pragma unroll
  for (int i = 0; i < CPT2; ++i) w01[i] = 0.01f * w[i];

  const T* xb = reinterpret_cast<const T*>(p.x) + b * p.sxb;
  T* gxb = reinterpret_cast<T*>(p.gx) + b * p.sgb;
  if constexpr (MASKED) {
    // Rows before the first and after the last valid row get a zero gradient
    // without their x being read.
    int64_t first, last;
    float unused;
    mask_extent(p, b, rbeg, rend, first, last, unused);
    if (last < first) first = last = rend;   // no valid row: zero the whole chunk
    else ++last;
    if (active) {
      float z[CPT];
#pragma unroll
      for (int i = 0; i < CPT; ++i) z[i] = 0.0f;
      for (int64_t n = rbeg + G.wave * G.rpw + G.lrow; n < first; n += G.rs) {
        VecIO<T, CPT>::store(gxb + n * p.sgn + map.c1, z);
        if constexpr (ROPE) VecIO<T, CPT>::store(gxb + n * p.sgn + map.c2, z);
      }
      for (int64_t n = last + G.wave * G.rpw + G.lrow; n < rend; n += G.rs) {
        VecIO<T, CPT>::store(gxb + n * p.sgn + map.c1, z);
        if constexpr (ROPE) VecIO<T, CPT>::store(gxb + n * p.sgn + map.c2, z);
      }
    }
    if constexpr (TR && !ROPE) {
      const int64_t c0 = slab * G.lpr * CPT;
      const int64_t nc = p.P - c0 < G.lpr * CPT ? p.P - c0 : G.lpr * CPT;
      zero_tr<T>(p.gxt, b, rbeg, first, c0, nc);
      zero_tr<T>(p.gxt, b, last, rend, c0, nc);
    }
    rbeg = first;
    rend = last;
  }
  const RowWalk W = TR ? RowWalk::consecutive(rbeg, rend, G.wave * G.rpw + G.lrow, G.rs, U)
                       : RowWalk(rbeg, rend, G.wave * G.rpw + G.lrow, G.rs, U);
  __shared__ __attribute__((aligned(16))) unsigned char tile_raw[TR ? TrTile<U, CPT2>::kElems * sizeof(T) : 16];
  T* tile = reinterpret_cast<T*>(tile_raw);

  struct Buf {
    Pack<T, CPT> v1[U], v2[ROPE ? U : 1];
    float mv[MASKED ? U : 1];
    int tp[ROPE ? U : 1];   // table positions, loaded with the rows
  };
  auto load = [&](Buf& bf, int64_t base, bool clamp) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t rr = W.row(base, u, clamp);
      const T* row = xb + rr * p.sxn;
      bf.v1[u].load_stream(row + map.c1);
      if constexpr (ROPE) {
        bf.v2[u].load_stream(row + map.c2);
        bf.tp[u] = rope_pos(p.rope, map.table, rr);
      }
      if constexpr (MASKED) bf.mv[u] = p.mask[b * p.msb + rr * p.msn];
    }
  };
  auto step = [&](const Buf& bf, int64_t base, auto tail_tag) {
    constexpr bool TAIL = decltype(tail_tag)::value;
    float gt[TR ? U : 1][CPT2];
    const auto& v1 = bf.v1;
    const auto& v2 = bf.v2;
    const auto& mv = bf.mv;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool in = !TAIL || W.valid(base, u);
      const int64_t n = W.row(base, u, TAIL);
      T* grow = gxb + n * p.sgn;
      float gv1[CPT], gv2[CPT];
      if constexpr (ROPE) {
        float cs[CPT], sn[CPT];
        load_table_at<CPT>(p.rope, map.table, bf.tp[u], map.tcol, cs, sn);
        bool keep = in;
        float mw = 1.0f;
        if constexpr (MASKED) {
          keep = keep && mv[u] != 0.0f;
          mw = mv[u];
        }
#pragma unroll
        for (int i = 0; i < CPT; ++i) {   // R^T applied to (w1, w2), times the token's mask weight
          const float wa = (w[i] * cs[i] + w[CPT + i] * sn[i]) * mw;
          const float wb = (w[CPT + i] * cs[i] - w[i] * sn[i]) * mw;
          const float x1 = v1[u].get(i), x2 = v2[u].get(i);
          const float l1 = leaky(x1), l2 = leaky(x2);
          const float h1 = clamp_act(l1), h2 = clamp_act(l2);
          gv1[i] = weighted_act_grad(x1, l1, h1, wa, 0.01f * wa) * poly_d<KM>(h1, d[i]);
          gv2[i] = weighted_act_grad(x2, l2, h2, wb, 0.01f * wb) * poly_d<KM>(h2, d[CPT + i]);
          if constexpr (MASKED) {   // padded token: zero gradient
            gv1[i] = keep ? gv1[i] : 0.0f;
            gv2[i] = keep ? gv2[i] : 0.0f;
          }
          pow_acc<KM>(keep ? h1 : 0.0f, wa, g[i]);
          pow_acc<KM>(keep ? h2 : 0.0f, wb, g[CPT + i]);
        }
        if (active && in) {
          VecIO<T, CPT>::store(grow + map.c1, gv1);
          VecIO<T, CPT>::store(grow + map.c2, gv2);
        }
        if constexpr (TR) {
#pragma unroll
          for (int i = 0; i < CPT; ++i) {
            gt[u][i] = gv1[i];
            gt[u][CPT + i] = gv2[i];
          }
        }
      } else {
        bool keep = in;
        if constexpr (MASKED) keep = keep && mv[u] != 0.0f;
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const float xx = v1[u].get(i);
          const float l = leaky(xx), h = clamp_act(l);
          if constexpr (MASKED) {
            const float wt = w[i] * mv[u];
            const float gxv = weighted_act_grad(xx, l, h, wt, 0.01f * wt) * poly_d<KM>(h, d[i]);
            gv1[i] = keep ? gxv : 0.0f;   // padded token: zero gradient
            pow_acc<KM>(keep ? h : 0.0f, wt, g[i]);
          } else {
            gv1[i] = weighted_act_grad(xx, l, h, w[i], w01[i]) * poly_d<KM>(h, d[i]);
            pow_sum<KM>(TAIL ? (in ? h : 0.0f) : h, g[i]);   // scaled by w at the end
          }
        }
        if (active && in) VecIO<T, CPT>::store(grow + map.c1, gv1);
        if constexpr (TR) {
#pragma unroll
          for (int i = 0; i < CPT; ++i) gt[u][i] = gv1[i];
        }
      }
    }
    if constexpr (TR) {
      const int64_t left = W.nrows - base;
      store_tr_staged<T, U, CPT2>(
          p.gxt, G, b, W.rbeg + base, left < W.step ? left : W.step,
          [&](int l, int i) { return slab_chan<CPT, MODE>(slab, G.lpr, p.g.nvec, p.P, l, i); }, gt, tile);
    }
  };

  // every lane walks (lanes past the channels on channel 0 with zero weights,
  // storing nothing): the staged channel-major stores synchronise the workgroup
  if constexpr (PIPE) walk_rows_pipe<Buf>(W, load, step);
  else walk_rows<Buf>(W, load, step);
  if constexpr (!ROPE && !MASKED) {
#pragma unroll
    for (int i = 0; i < CPT2; ++i)
#pragma unroll
      for (int j = 0; j < KM; ++j) g[i][j] *= w[i];
  }

  // grad_coeff partial of the chunk, one degree at a time.
  const int nslot = G.lpr * CPT2;
  for (int j = 0; j < p.K; ++j) {
#pragma unroll
    for (int i = 0; i < CPT2; ++i) {
      float v = 0.0f;
#pragma unroll
      for (int jj = 0; jj < KM; ++jj) v = (jj == j) ? g[i][jj] : v;
      v = xor_sum_rows(v, G.lb);
      if (G.lrow == 0) red[G.wave][G.lcol * CPT2 + i] = v;
    }
    __syncthreads();
    for (int s = G.tid; s < nslot; s += kThreads) {
      const int l = s / CPT2, i = s - l * CPT2;
      const int64_t vc = slab * G.lpr + l;
      if (vc >= p.g.nvec) continue;
      float v = 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < kWaves; ++w2) v += red[w2][s];
      Map m2;
      m2.init(vc, p.P);
      p.part[((b * p.g.nch + chunk) * p.K + j) * p.P + m2.chan(i)] = v;
    }
    __syncthreads();
  }
}

template <typename T, int CPT, int KM, int MODE, bool TR>
__global__ void __launch_bounds__(kThreads) agg_bwd_chunk(const AggParams p) {
  agg_bwd_body<T, CPT, KM, MODE, TR>(p);
}

// Plain mode at degree <= 2 runs at three waves per SIMD: the kernel is
// memory-bound and latency-limited, and the register cap costs it at most a
// few bytes of spill.  Higher degrees and the masked / RoPE modes hold more
// per-lane state; capped, they spill inside the row loop and run slower.
template <typename T, int CPT, int KM, int MODE, bool TR>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3)))
agg_bwd_chunk_w3(const AggParams p) {
  agg_bwd_body<T, CPT, KM, MODE, TR>(p);
}

// ---------------------------------------------------------------------------
// RoPE backward with one lane per half of a rotation pair (HalfMap).
// grad_x of a channel at token n is act'(x) p'(h) times its upstream weight
// rotated back to the token: w cos + sign w_partner sin, from the cos / sin
// table row of n's position (pom/pom_rope.py:258-296 differentiated).  The
// upstream weights are constant over the chunk, so nothing but that table row
// couples the two halves: a lane holds the coefficients and sums of its own
// CPT channels only, half the state of a pair lane.
// The table row of a position serves every batch row (positions are per
// token), so a workgroup walks NB batch rows at once: a lane loads the table
// entries of U tokens and the x of those tokens in NB batch rows, NB x U = 4
// rows in flight for U table lookups.  At NB = 4 the lookups cost 2 bytes per
// element instead of 8 (at C5's shape: 105-116 us against 142-148 for
// NB = 1).  The NB batch rows' upstream weights are read from LDS at each row
// (in registers they would hold the kernel under three waves per SIMD).
// NB divides B (the host picks it so), so every row of the walk exists and
// the stores need no branch.  grad_coeff partials are per (batch group,
// chunk): the NB rows of a token are added in batch order, the tokens in walk
// order.  The step's loads are issued before its arithmetic (walk_rows_pre).
// ---------------------------------------------------------------------------
template <int NB>
struct RopeHalfShape {
  static constexpr int U = NB >= 4 ? 1 : (NB == 2 ? 2 : 4);   // token rows per step
};

// o = p[0 .. V) from LDS in 16-byte (or narrower) reads; p aligned to them.
template <int V>
__device__ __forceinline__ void lds_load_f32(const float* p, float (&o)[V]) {
  if constexpr (V % 4 == 0) {
#pragma unroll
    for (int i = 0; i < V; i += 4) {
      const float4 a = *reinterpret_cast<const float4*>(p + i);
      o[i] = a.x; o[i + 1] = a.y; o[i + 2] = a.z; o[i + 3] = a.w;
    }
  } else if constexpr (V == 2) {
    const float2 a = *reinterpret_cast<const float2*>(p);
    o[0] = a.x; o[1] = a.y;
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = p[i];
  }
}

template <typename T, int CPT, int KM, int MODE, int NB>
__device__ __forceinline__ void agg_bwd_rope_half_body(const AggParams& p) {
  using Map = HalfMap<CPT, MODE>;
  constexpr bool MASKED = mode_masked(MODE);
  static_assert(!MASKED || NB == 1, "masked rows are walked one batch row at a time");
  constexpr int U = RopeHalfShape<NB>::U;
  __shared__ float red[kWaves][kMaxLpr * CPT];

  const LaneGeom G(p.g.lpr_log2);
  const int64_t slab = blockIdx.x, chunk = blockIdx.y, bg = blockIdx.z;
  const int64_t b0 = bg * NB;
  int64_t f, rbeg, rend;
  chunk_rows(p.g, chunk, p.N, f, rbeg, rend);
  const int64_t vcol = slab * G.lpr + G.lcol;
  const bool active = vcol < p.g.nvec;
  Map map;
  map.init(active ? vcol : 0, p.P);

  // d[i][j] = (j+1) c[i][j]; wsh[k][0 / 1] = own and (signed) partner upstream
  // weights of batch row b0 + k, one slot per channel of the slab
  float d[CPT][KM], g[CPT][KM];
  __shared__ __attribute__((aligned(16))) float wsh[NB][2][kMaxLpr * CPT];
  {
    float flat[CPT * KM];
    param_gather<CPT * KM>(p.coeff, [&](int q) {
      const int j = q % KM;
      return map.chan(q / KM) * p.K + (j < p.K ? j : p.K - 1);
    }, flat);
#pragma unroll
    for (int i = 0; i < CPT; ++i)
#pragma unroll
      for (int j = 0; j < KM; ++j) {
        d[i][j] = (active && j < p.K) ? flat[i * KM + j] * (float)(j + 1) : 0.0f;
        g[i][j] = 0.0f;
      }
  }
#pragma unroll
  for (int k = 0; k < NB; ++k) {
    const int64_t bk = b0 + k;
    float cntv = 1.0f;
    if constexpr (MASKED) cntv = p.count_in[bk];
    const float* wsrc = (!MASKED && p.wf) ? p.wf + (bk * p.g.F + f) * p.P : p.go + bk * p.P;
    float raw[2 * CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      raw[i] = wsrc[map.c1 + i];
      raw[CPT + i] = wsrc[map.cp + i];
    }
#pragma unroll
    for (int i = 0; i < 2 * CPT; ++i) {
      float wi;
      if constexpr (MASKED) wi = cntv != 0.0f ? raw[i] / cntv : 0.0f;
      else if (p.wf) wi = raw[i];
      else wi = (raw[i] / ((float)p.n_past + 1.0f)) / (float)p.g.L;
      raw[i] = active ? wi : 0.0f;
    }
    if (G.wave == 0 && G.lrow == 0) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        wsh[k][0][G.lcol * CPT + i] = raw[i];
        wsh[k][1][G.lcol * CPT + i] = map.sign * raw[CPT + i];
      }
    }
  }
  __syncthreads();

  auto xrow = [&](int k) { return reinterpret_cast<const T*>(p.x) + (b0 + k) * p.sxb; };
  if constexpr (MASKED) {
    // rows before the first and after the last valid row: zero gradient, x not read
    T* gxb = reinterpret_cast<T*>(p.gx) + b0 * p.sgb;
    int64_t first, last;
    float unused;
    mask_extent(p, b0, rbeg, rend, first, last, unused);
    if (last < first) first = last = rend;
    else ++last;
    if (active) {
      float z[CPT];
#pragma unroll
      for (int i = 0; i < CPT; ++i) z[i] = 0.0f;
      for (int64_t n = rbeg + G.wave * G.rpw + G.lrow; n < first; n += G.rs)
        VecIO<T, CPT>::store(gxb + n * p.sgn + map.c1, z);
      for (int64_t n = last + G.wave * G.rpw + G.lrow; n < rend; n += G.rs)
        VecIO<T, CPT>::store(gxb + n * p.sgn + map.c1, z);
    }
    rbeg = first;
    rend = last;
  }
  const RowWalk W(rbeg, rend, G.wave * G.rpw + G.lrow, G.rs, U);

  struct Pos {
    int tp[U];   // table positions, loaded one step ahead
  };
  struct Buf {
    Pack<T, CPT> v[U][NB];
    float mv[MASKED ? U : 1];
    float cs[U][CPT], sn[U][CPT];
  };
  auto pre = [&](Pos& pb, int64_t base) {
#pragma unroll
    for (int u = 0; u < U; ++u) pb.tp[u] = rope_pos(p.rope, map.table, W.row(base, u, true));
  };
  auto load = [&](Buf& bf, const Pos& pb, int64_t base, bool clamp) {
#pragma unroll
    for (int u = 0; u < U; ++u) load_table_at<CPT>(p.rope, map.table, pb.tp[u], map.tcol, bf.cs[u], bf.sn[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t rr = W.row(base, u, clamp);
#pragma unroll
      for (int k = 0; k < NB; ++k) bf.v[u][k].load_stream(xrow(k) + rr * p.sxn + map.c1);
      if constexpr (MASKED) bf.mv[u] = p.mask[b0 * p.msb + rr * p.msn];
    }
    mem_fence_compiler();   // every load of the step issued before its arithmetic
  };
  auto step = [&](const Buf& bf, int64_t base, auto tail_tag) {
    constexpr bool TAIL = decltype(tail_tag)::value;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool in = !TAIL || W.valid(base, u);
      const int64_t n = W.row(base, u, TAIL);
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        bool keep = in;
        float mw = 1.0f;
        if constexpr (MASKED) {
          keep = keep && bf.mv[u] != 0.0f;
          mw = bf.mv[u];
        }
        float gv[CPT], wok[CPT], wpk[CPT];
        lds_load_f32<CPT>(&wsh[k][0][G.lcol * CPT], wok);
        lds_load_f32<CPT>(&wsh[k][1][G.lcol * CPT], wpk);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const float we = (wok[i] * bf.cs[u][i] + wpk[i] * bf.sn[u][i]) * mw;
          const float x = bf.v[u][k].get(i);
          const float l = leaky(x), h = clamp_act(l);
          gv[i] = weighted_act_grad(x, l, h, we, 0.01f * we) * poly_d<KM>(h, d[i]);
          if constexpr (MASKED) gv[i] = keep ? gv[i] : 0.0f;   // padded token: zero gradient
          pow_acc<KM>((MASKED || TAIL) ? (keep ? h : 0.0f) : h, we, g[i]);
        }
        if (in)
          VecIO<T, CPT>::store(reinterpret_cast<T*>(p.gx) + (b0 + k) * p.sgb + n * p.sgn + map.c1, gv);
      }
    }
  };
  if (active && W.nrows > 0) walk_rows_pre<Buf, Pos>(W, pre, load, step);

  // grad_coeff partial of the chunk, one degree at a time.
  const int nslot = G.lpr * CPT;
  for (int j = 0; j < p.K; ++j) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      float v = 0.0f;
#pragma unroll
      for (int jj = 0; jj < KM; ++jj) v = (jj == j) ? g[i][jj] : v;
      v = xor_sum_rows(v, G.lb);
      if (G.lrow == 0) red[G.wave][G.lcol * CPT + i] = v;
    }
    __syncthreads();
    for (int s = G.tid; s < nslot; s += kThreads) {
      const int l = s / CPT, i = s - l * CPT;
      const int64_t vc = slab * G.lpr + l;
      if (vc >= p.g.nvec) continue;
      float v = 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < kWaves; ++w2) v += red[w2][s];
      p.part[((bg * p.g.nch + chunk) * p.K + j) * p.P + vc * CPT + i] = v;
    }
    __syncthreads();
  }
}

// Three waves per SIMD where the state fits 168 VGPRs without spilling
// (degree <= 3 at NB = 4, <= 2 at NB = 2, 1 at NB = 1, unmasked); the rest run
// uncapped, as capped they spill inside the row loop.
template <int CPT, int KM, int MODE, int NB>
constexpr bool kRopeHalfW3 = !mode_masked(MODE) && (NB >= 4 ? KM <= 3 : (NB == 2 ? KM <= 2 : KM <= 1));

template <typename T, int CPT, int KM, int MODE, int NB>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3)))
agg_bwd_rope_half_w3(const AggParams p) {
  agg_bwd_rope_half_body<T, CPT, KM, MODE, NB>(p);
}

template <typename T, int CPT, int KM, int MODE, int NB>
__global__ void __launch_bounds__(kThreads) agg_bwd_rope_half(const AggParams p) {
  agg_bwd_rope_half_body<T, CPT, KM, MODE, NB>(p);
}

template <typename T, int CPT, int KM, int MODE, int NB>
void launch_rope_half(const AggParams& p, dim3 grid, hipStream_t st) {
  if constexpr (kRopeHalfW3<CPT, KM, MODE, NB>)
    hipLaunchKernelGGL((agg_bwd_rope_half_w3<T, CPT, KM, MODE, NB>), grid, dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL((agg_bwd_rope_half<T, CPT, KM, MODE, NB>), grid, dim3(kThreads), 0, st, p);
}

// grad_coeff[c, j] = sum over the rows (batch row, chunk) of the partials.
// A workgroup owns 64 outputs.  From 64 rows on, each of its four waves sums
// a quarter of the rows (sixteen loads in flight, in row order) and the
// quarters are added in a fixed order, so a long row list costs a quarter of
// the round trips; shorter lists are summed by one wave in row order.
constexpr int kGcOut = kThreads / 4;   // outputs per workgroup (one wave per quarter)

static __global__ void __launch_bounds__(kThreads) coeff_grad_finalize(const float* __restrict__ part, int64_t rows,
                                                                int64_t P, int K, ParamOut gc) {
  __shared__ float red[kThreads];
  const int o = threadIdx.x % kGcOut, qtr = threadIdx.x / kGcOut;
  const int64_t idx = (int64_t)blockIdx.x * kGcOut + o;
  const bool live = idx < P * K;
  const int64_t j = live ? idx / P : 0, c = live ? idx - j * P : 0;
  const float* src = part + j * P + c;
  const int64_t stride = (int64_t)K * P;
  const int nq = rows >= 64 ? 4 : 1;
  const int64_t per = (rows + nq - 1) / nq, r0 = qtr * per, r1 = r0 + per < rows ? r0 + per : rows;
  float s = 0.0f;
  if (live && qtr < nq) {
    int64_t r = r0;
    for (; r + 16 <= r1; r += 16) {
      float v[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = src[(r + q) * stride];
#pragma unroll
      for (int q = 0; q < 16; ++q) s += v[q];
    }
    for (; r < r1; ++r) s += src[r * stride];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  if (qtr == 0 && live)
    param_set(gc, c * K + j,
              nq == 1 ? red[o] : ((red[o] + red[kGcOut + o]) + red[2 * kGcOut + o]) + red[3 * kGcOut + o]);
}

inline hipError_t launch_coeff_grad_finalize(const float* part, int64_t rows, int64_t P, int K, ParamOut gc,
                                             hipStream_t st) {
  hipLaunchKernelGGL(coeff_grad_finalize, dim3((unsigned)((P * K + kGcOut - 1) / kGcOut)), dim3(kThreads), 0, st,
                     part, rows, P, K, gc);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Host-side launch helpers
// ---------------------------------------------------------------------------
inline dim3 flat_grid(int64_t n) { return dim3((unsigned)((n + kThreads - 1) / kThreads)); }

template <typename T, int CPT, int KM>
hipError_t agg_fwd_mode(const AggParams& p, hipStream_t st) {
  const dim3 grid((unsigned)p.g.nslabs, (unsigned)p.g.nch, (unsigned)p.B), block(kThreads);
  switch (p.mode) {
    case MODE_PLAIN: hipLaunchKernelGGL((agg_fwd_chunk<T, CPT, KM, MODE_PLAIN>), grid, block, 0, st, p); break;
    case MODE_MASKED: hipLaunchKernelGGL((agg_fwd_chunk<T, CPT, KM, MODE_MASKED>), grid, block, 0, st, p); break;
    case MODE_ROPE1D: hipLaunchKernelGGL((agg_fwd_chunk<T, CPT, KM, MODE_ROPE1D>), grid, block, 0, st, p); break;
    case MODE_ROPE2D: hipLaunchKernelGGL((agg_fwd_chunk<T, CPT, KM, MODE_ROPE2D>), grid, block, 0, st, p); break;
    case MODE_ROPE1D_MASKED:
      hipLaunchKernelGGL((agg_fwd_chunk<T, CPT, KM, MODE_ROPE1D_MASKED>), grid, block, 0, st, p);
      break;
    case MODE_ROPE2D_MASKED:
      hipLaunchKernelGGL((agg_fwd_chunk<T, CPT, KM, MODE_ROPE2D_MASKED>), grid, block, 0, st, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int CPT, int KM, bool TR>
hipError_t agg_bwd_tr(const AggParams& p, hipStream_t st) {
  const dim3 grid((unsigned)p.g.nslabs, (unsigned)p.g.nch, (unsigned)p.B), block(kThreads);
  if (p.g.half) {   // RoPE modes without the channel-major copy
    if constexpr (TR) {
      return hipErrorInvalidValue;
    } else {
      auto launch = [&](auto nb_tag) -> hipError_t {
        constexpr int NB = decltype(nb_tag)::value;
        const dim3 hgrid((unsigned)p.g.nslabs, (unsigned)p.g.nch, (unsigned)(p.B / NB));
        switch (p.mode) {
          case MODE_ROPE1D:
            launch_rope_half<T, CPT, KM, MODE_ROPE1D, NB>(p, hgrid, st);
            break;
          case MODE_ROPE2D:
            launch_rope_half<T, CPT, KM, MODE_ROPE2D, NB>(p, hgrid, st);
            break;
          case MODE_ROPE1D_MASKED:
            if constexpr (NB != 1) return hipErrorInvalidValue;
            else launch_rope_half<T, CPT, KM, MODE_ROPE1D_MASKED, 1>(p, hgrid, st);
            break;
          case MODE_ROPE2D_MASKED:
            if constexpr (NB != 1) return hipErrorInvalidValue;
            else launch_rope_half<T, CPT, KM, MODE_ROPE2D_MASKED, 1>(p, hgrid, st);
            break;
          default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
      };
      if constexpr (CPT >= 4) {
        if (p.g.nb == 4) return launch(std::integral_constant<int, 4>{});
        if (p.g.nb == 2) return launch(std::integral_constant<int, 2>{});
      }
      if (p.g.nb == 1) return launch(std::integral_constant<int, 1>{});
      return hipErrorInvalidValue;
    }
  }
  switch (p.mode) {
    case MODE_PLAIN:
      if constexpr (KM <= 2) hipLaunchKernelGGL((agg_bwd_chunk_w3<T, CPT, KM, MODE_PLAIN, TR>), grid, block, 0, st, p);
      else hipLaunchKernelGGL((agg_bwd_chunk<T, CPT, KM, MODE_PLAIN, TR>), grid, block, 0, st, p);
      break;
    case MODE_MASKED: hipLaunchKernelGGL((agg_bwd_chunk<T, CPT, KM, MODE_MASKED, TR>), grid, block, 0, st, p); break;
    // RoPE with pair lanes: only with the channel-major copy (without it the
    // half-pair kernel above runs; masked RoPE has no copy, the C ABI rejects it)
    case MODE_ROPE1D:
      if constexpr (!TR) return hipErrorInvalidValue;
      else hipLaunchKernelGGL((agg_bwd_chunk<T, CPT, KM, MODE_ROPE1D, true>), grid, block, 0, st, p);
      break;
    case MODE_ROPE2D:
      if constexpr (!TR) return hipErrorInvalidValue;
      else hipLaunchKernelGGL((agg_bwd_chunk<T, CPT, KM, MODE_ROPE2D, true>), grid, block, 0, st, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The channel-major copy is built for 16-bit types with 16-byte lanes only
// (the C ABI rejects other requests).
template <typename T, int CPT>
constexpr bool kTrBuilt = sizeof(T) == 2 && CPT == 8;

template <typename T, int CPT, int KM>
hipError_t agg_bwd_mode(const AggParams& p, hipStream_t st) {
  if constexpr (kTrBuilt<T, CPT>) {
    if (p.gxt.data) return agg_bwd_tr<T, CPT, KM, true>(p, st);
  } else {
    if (p.gxt.data) return hipErrorInvalidValue;
  }
  return agg_bwd_tr<T, CPT, KM, false>(p, st);
}

// Degree bound KM: exact for K <= 4, then 8 and 16 with zero coefficients.
#define POM_K_SWITCH(K_, CALL)                   \
  switch (K_) {                                  \
    case 1: { constexpr int KM = 1; CALL; }      \
    case 2: { constexpr int KM = 2; CALL; }      \
    case 3: { constexpr int KM = 3; CALL; }      \
    case 4: { constexpr int KM = 4; CALL; }      \
    default: break;                              \
  }                                              \
  if ((K_) <= 8) { constexpr int KM = 8; CALL; } \
  { constexpr int KM = 16; CALL; }

template <typename T, int CPT>
hipError_t agg_fwd_cpt(const AggParams& p, hipStream_t st) {
  POM_K_SWITCH(p.K, return (agg_fwd_mode<T, CPT, KM>(p, st)))
}

template <typename T, int CPT>
hipError_t agg_bwd_cpt(const AggParams& p, hipStream_t st) {
  POM_K_SWITCH(p.K, return (agg_bwd_mode<T, CPT, KM>(p, st)))
}

// Vector widths: 16-byte loads when pointers and strides allow, else narrower.
#define POM_CPT_SWITCH(T_, CPT_, FN, ...)                                   \
  switch (CPT_) {                                                           \
    case 8: if constexpr (sizeof(T_) == 2) return FN<T_, 8>(__VA_ARGS__); else break; \
    case 4: return FN<T_, 4>(__VA_ARGS__);                                  \
    case 2: return FN<T_, 2>(__VA_ARGS__);                                  \
    case 1: return FN<T_, 1>(__VA_ARGS__);                                  \
    default: break;                                                         \
  }                                                                         \
  return hipErrorInvalidValue;

template <typename T>
hipError_t agg_fwd_chunks(const AggParams& p, hipStream_t st) {
  POM_CPT_SWITCH(T, p.g.cpt, agg_fwd_cpt, p, st)
}

template <typename T>
hipError_t agg_bwd_chunks(const AggParams& p, hipStream_t st) {
  POM_CPT_SWITCH(T, p.g.cpt, agg_bwd_cpt, p, st)
}

template <typename T>
hipError_t agg_fwd_t(const AggParams& p, hipStream_t st) {
  hipError_t e = agg_fwd_chunks<T>(p, st);
  if (e != hipSuccess || p.direct) return e;
  if (mode_masked(p.mode))
    hipLaunchKernelGGL((agg_fwd_finalize<T, true>), flat_grid(p.B * p.P), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL((agg_fwd_finalize<T, false>), flat_grid(p.B * p.P), dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <typename T>
hipError_t agg_bwd_t(const AggParams& p, hipStream_t st) {
  if (p.wf) {
    hipLaunchKernelGGL(agg_frame_weights, flat_grid(p.B * p.P), dim3(kThreads), 0, st, p,
                       const_cast<float*>(p.wf));
    if (hipError_t e = hipGetLastError()) return e;
  }
  if (hipError_t e = agg_bwd_chunks<T>(p, st)) return e;
  return launch_coeff_grad_finalize(p.part, p.B / p.g.nb * p.g.nch, p.P, p.K, p.gc, st);
}

}  // namespace pom
