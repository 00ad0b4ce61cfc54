// Fused activation + polynomial expansion + sequence aggregation (forward and
// backward) for the Polynomial Mixer, written for gfx950 (CDNA4).
//
// One kernel family covers the reference's mean, masked, frame-causal and RoPE
// aggregations (pom/pom_triton.py:68-321, pom/pom_triton_masked.py:72-345,
// pom/pom.py:233-262 + :41-45, pom/pom_triton_rope.py:93-475,
// pom/pom_rope.py:242-296).
//
// Work decomposition (all variants):
//   grid = B x nchunks x nslabs workgroups of 256 threads (4 waves).
//   A workgroup owns RC consecutive tokens ("chunk") of one batch row and one
//   channel slab.  Within a wave, LPR lanes cover one token row (each lane CPT
//   consecutive channels, one 16-byte load for bf16 CPT=8) and 64/LPR rows are
//   processed side by side; the four waves interleave rows.  Loads of U rows
//   are issued before any arithmetic so every lane keeps U 16-byte loads in
//   flight.  Accumulation is fp32 in registers.
//   Partials of the chunk are reduced across the workgroup in LDS, written to a
//   workspace, and the last workgroup of each group (device-scope atomic
//   election, no float atomics) sums them in a fixed order, so results are
//   deterministic run to run.
//
// Frames: tokens are grouped in frames of L tokens (L = N for the plain mean).
// Frame f's output is the running mean of frame means, the recurrence that
// PoM.state_forward applies per call (pom/pom.py:255-259):
//   H_f = (n * H_{f-1} + M_f) / (n + 1),  n = n_past + f,
// with H rounded to the element type after every frame exactly as the
// reference's carry tensor is.  Token-causal aggregation (L = 1) keeps the
// running value in fp32 and rounds only the output, as the reference's fused
// causal kernel does (pom/pom_triton_causal.py:150-159).  A chunk never
// straddles two frames (RC | L).
#include "common.h"
#include "pom_internal.h"
#include "lanes.h"

namespace pom {

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <typename T, int CPT, int KM, int MODE>
__global__ void __launch_bounds__(kThreads)
agg_fwd_kernel(const AggParams p) {
  using Map = LaneMap<CPT, MODE>;
  constexpr int CPT2 = Map::CPT2;
  constexpr bool ROPE = (MODE == MODE_ROPE1D || MODE == MODE_ROPE2D);
  constexpr int U = ROPE ? 2 : 4;

  __shared__ float red[kThreads * CPT2];
  __shared__ int flag;
  __shared__ float cnt_red[kThreads];

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int lpr = 1 << p.lpr_log2;
  const int rpw = kWave >> p.lpr_log2;         // rows per wave step
  const int rs = kWaves * rpw;                  // rows per workgroup step
  const int lrow = lane >> p.lpr_log2, lcol = lane & (lpr - 1);

  int64_t wg = blockIdx.x;
  const int64_t slab = wg % p.nslabs; wg /= p.nslabs;
  const int64_t chunk = wg % p.nchunks; wg /= p.nchunks;
  const int64_t b = wg;
  const int64_t f = chunk / p.cpf;

  const int64_t vcol = slab * lpr + lcol;
  const bool active = vcol < p.nvec;
  Map map;
  map.init(active ? vcol : 0, p.P);

  float c[CPT2][KM];
#pragma unroll
  for (int i = 0; i < CPT2; ++i)
#pragma unroll
    for (int j = 0; j < KM; ++j)
      c[i][j] = (active && j < p.K) ? p.coeff[map.chan(i) * p.K + j] : 0.0f;

  float acc[CPT2];
#pragma unroll
  for (int i = 0; i < CPT2; ++i) acc[i] = 0.0f;

  const T* xb = reinterpret_cast<const T*>(p.x) + b * p.sxb;
  const int64_t n0 = chunk * p.RC;
  const int row0 = wave * rpw + lrow;

  if (active) {
    for (int64_t r = row0; r < p.RC; r += (int64_t)rs * U) {
      float xv[U][CPT2];
      float wv[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t rr = r + (int64_t)u * rs;
        ok[u] = rr < p.RC;
        wv[u] = 1.0f;
        if constexpr (MODE == MODE_MASKED) {
          if (ok[u]) {
            wv[u] = p.mask[b * p.msb + (n0 + rr) * p.msn];
            ok[u] = wv[u] != 0.0f;   // padded tokens are never loaded
          }
        }
        if (ok[u]) {
          const T* row = xb + (n0 + rr) * p.sxn;
          float tmp[CPT];
          VecIO<T, CPT>::load(row + map.c1, tmp);
#pragma unroll
          for (int i = 0; i < CPT; ++i) xv[u][i] = tmp[i];
          if constexpr (ROPE) {
            VecIO<T, CPT>::load(row + map.c2, tmp);
#pragma unroll
            for (int i = 0; i < CPT; ++i) xv[u][CPT + i] = tmp[i];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!ok[u]) continue;
        float pv[CPT2];
#pragma unroll
        for (int i = 0; i < CPT2; ++i) pv[i] = poly<KM>(act(xv[u][i]), c[i]);
        if constexpr (ROPE) {
          float cs[CPT], sn[CPT];
          load_table<CPT>(p.rope, map.table, n0 + r + (int64_t)u * rs, map.tcol, cs, sn);
#pragma unroll
          for (int i = 0; i < CPT; ++i) {
            acc[i] += pv[i] * cs[i] - pv[CPT + i] * sn[i];
            acc[CPT + i] += pv[CPT + i] * cs[i] + pv[i] * sn[i];
          }
        } else {
#pragma unroll
          for (int i = 0; i < CPT2; ++i) acc[i] += wv[u] * pv[i];
        }
      }
    }
  }

  // Workgroup reduction of the chunk partial in a fixed order.
  const int width = lpr * CPT2;            // slots of this slab
  const int rslot = wave * rpw + lrow;     // 0 .. rs-1
#pragma unroll
  for (int i = 0; i < CPT2; ++i) red[rslot * width + lcol * CPT2 + i] = acc[i];
  __syncthreads();
  const int64_t slot0 = slab * (int64_t)width;
  const int64_t nslot = p.nvec * CPT2;
  for (int col = tid; col < width; col += kThreads) {
    float s = 0.0f;
    for (int q = 0; q < rs; ++q) s += red[q * width + col];
    if (slot0 + col < nslot) p.partial[(b * p.nchunks + chunk) * p.P + slot0 + col] = s;
  }

  // Level 1: last chunk of the frame forms the frame mean.
  if (!elect_last(p.cnt1 + (b * p.NF + f) * p.nslabs + slab, (int)p.cpf, &flag)) return;

  float inv = 1.0f / (float)p.L;
  if constexpr (MODE == MODE_MASKED) {
    float s = 0.0f;
    for (int64_t n = tid; n < p.N; n += kThreads) s += p.mask[b * p.msb + n * p.msn];
    cnt_red[tid] = s;
    __syncthreads();
    if (tid == 0) {
      float t = 0.0f;
      for (int q = 0; q < kThreads; ++q) t += cnt_red[q];
      cnt_red[0] = t;
      if (slab == 0 && p.count_out) p.count_out[b] = t;
    }
    __syncthreads();
    const float cnt = cnt_red[0];
    inv = cnt != 0.0f ? 1.0f / cnt : 0.0f;   // an all-masked row aggregates to 0
  }
  const bool direct = (p.NF == 1) && (p.carry == nullptr);
  T* out = reinterpret_cast<T*>(p.out);
  for (int col = tid; col < width; col += kThreads) {
    const int64_t s = slot0 + col;
    if (s >= nslot) continue;
    float m = 0.0f;
    for (int64_t k = 0; k < p.cpf; ++k) m += p.partial[(b * p.nchunks + f * p.cpf + k) * p.P + s];
    m = m * inv;
    if (direct) out[b * p.P + slot_chan<CPT, MODE>(s, p.P)] = from_f32<T>(m);
    else p.fmean[(b * p.NF + f) * p.P + s] = m;
  }
  if (direct) return;

  // Level 2: the last frame of the batch row runs the frame recurrence.
  if (!elect_last(p.cnt2 + b * p.nslabs + slab, (int)p.NF, &flag)) return;
  const T* carry = reinterpret_cast<const T*>(p.carry);
  for (int col = tid; col < width; col += kThreads) {
    const int64_t s = slot0 + col;
    if (s >= nslot) continue;
    const int64_t ch = slot_chan<CPT, MODE>(s, p.P);
    float h = carry ? to_f32<T>(carry[b * p.P + ch]) : 0.0f;
    float n = (float)p.n_past;
    for (int64_t g = 0; g < p.NF; ++g) {
      const float m = p.fmean[(b * p.NF + g) * p.P + s];
      h = (g == 0 && carry == nullptr) ? m : (n * h + m) / (n + 1.0f);
      if (p.round_carry) h = round_to<T>(h);
      out[(b * p.NF + g) * p.P + ch] = from_f32<T>(h);
      n += 1.0f;
    }
  }
}

// ---------------------------------------------------------------------------
// Backward: grad_x (written into a strided view, e.g. the h-half of dY) and
// grad_coeff (two-level deterministic reduction).
// ---------------------------------------------------------------------------
template <typename T, int CPT, int KM, int MODE>
__global__ void __launch_bounds__(kThreads)
agg_bwd_kernel(const AggParams p) {
  using Map = LaneMap<CPT, MODE>;
  constexpr int CPT2 = Map::CPT2;
  constexpr bool ROPE = (MODE == MODE_ROPE1D || MODE == MODE_ROPE2D);
  constexpr int U = ROPE ? 2 : 4;

  __shared__ float red[kThreads * CPT2];
  __shared__ int flag;

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int lpr = 1 << p.lpr_log2;
  const int rpw = kWave >> p.lpr_log2;
  const int rs = kWaves * rpw;
  const int lrow = lane >> p.lpr_log2, lcol = lane & (lpr - 1);

  int64_t wg = blockIdx.x;
  const int64_t slab = wg % p.nslabs; wg /= p.nslabs;
  const int64_t chunk = wg % p.nchunks; wg /= p.nchunks;
  const int64_t b = wg;
  const int64_t f = chunk / p.cpf;

  const int64_t vcol = slab * lpr + lcol;
  const bool active = vcol < p.nvec;
  Map map;
  map.init(active ? vcol : 0, p.P);

  float c[CPT2][KM], g[CPT2][KM], w[CPT2];
#pragma unroll
  for (int i = 0; i < CPT2; ++i) {
    const int64_t ch = map.chan(i);
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      c[i][j] = (active && j < p.K) ? p.coeff[ch * p.K + j] : 0.0f;
      g[i][j] = 0.0f;
    }
    // Weight of one token of frame f in the frame outputs it feeds:
    //   dM_f = sum_{g >= f} dH_g / (n_past + g + 1),  d token = dM_f / L
    // (masked: dH / count, scaled per token by its mask value).
    float s = 0.0f;
    if (active) {
      if constexpr (MODE == MODE_MASKED) {
        const float cnt = p.count_in[b];
        s = cnt != 0.0f ? p.go[b * p.P + ch] / cnt : 0.0f;
      } else {
        for (int64_t gg = p.NF - 1; gg >= f; --gg)
          s += p.go[(b * p.NF + gg) * p.P + ch] / ((float)(p.n_past + gg) + 1.0f);
        s = s / (float)p.L;
      }
    }
    w[i] = s;
  }

  const T* xb = reinterpret_cast<const T*>(p.x) + b * p.sxb;
  T* gxb = reinterpret_cast<T*>(p.gx) + b * p.sgb;
  const int64_t n0 = chunk * p.RC;
  const int row0 = wave * rpw + lrow;

  if (active) {
    for (int64_t r = row0; r < p.RC; r += (int64_t)rs * U) {
      float xv[U][CPT2];
      float mv[U];
      bool in[U], ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t rr = r + (int64_t)u * rs;
        in[u] = rr < p.RC;
        ok[u] = in[u];
        mv[u] = 1.0f;
        if constexpr (MODE == MODE_MASKED) {
          if (in[u]) {
            mv[u] = p.mask[b * p.msb + (n0 + rr) * p.msn];
            ok[u] = mv[u] != 0.0f;
          }
        }
        if (ok[u]) {
          const T* row = xb + (n0 + rr) * p.sxn;
          float tmp[CPT];
          VecIO<T, CPT>::load(row + map.c1, tmp);
#pragma unroll
          for (int i = 0; i < CPT; ++i) xv[u][i] = tmp[i];
          if constexpr (ROPE) {
            VecIO<T, CPT>::load(row + map.c2, tmp);
#pragma unroll
            for (int i = 0; i < CPT; ++i) xv[u][CPT + i] = tmp[i];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!in[u]) continue;
        const int64_t n = n0 + r + (int64_t)u * rs;
        float gv[CPT2];
        if (!ok[u]) {
#pragma unroll
          for (int i = 0; i < CPT2; ++i) gv[i] = 0.0f;   // padded token: zero gradient
        } else {
          float wt[CPT2];
          if constexpr (ROPE) {
            float cs[CPT], sn[CPT];
            load_table<CPT>(p.rope, map.table, n, map.tcol, cs, sn);
#pragma unroll
            for (int i = 0; i < CPT; ++i) {   // R^T applied to (w1, w2)
              wt[i] = w[i] * cs[i] + w[CPT + i] * sn[i];
              wt[CPT + i] = w[CPT + i] * cs[i] - w[i] * sn[i];
            }
          } else {
#pragma unroll
            for (int i = 0; i < CPT2; ++i) wt[i] = w[i] * mv[u];
          }
#pragma unroll
          for (int i = 0; i < CPT2; ++i) {
            const float xx = xv[u][i];
            const float dp = poly_grad_acc<KM>(act(xx), wt[i], c[i], g[i]);
            gv[i] = wt[i] * dp * act_grad(xx);
          }
        }
        T* grow = gxb + n * p.sgn;
        float tmp[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) tmp[i] = gv[i];
        VecIO<T, CPT>::store(grow + map.c1, tmp);
        if constexpr (ROPE) {
#pragma unroll
          for (int i = 0; i < CPT; ++i) tmp[i] = gv[CPT + i];
          VecIO<T, CPT>::store(grow + map.c2, tmp);
        }
      }
    }
  }

  // grad_coeff partial of this chunk, one degree at a time through LDS.
  const int width = lpr * CPT2;
  const int rslot = wave * rpw + lrow;
  const int64_t slot0 = slab * (int64_t)width;
  const int64_t nslot = p.nvec * CPT2;
  for (int j = 0; j < p.K; ++j) {
#pragma unroll
    for (int i = 0; i < CPT2; ++i) {
      float v = 0.0f;
#pragma unroll
      for (int jj = 0; jj < KM; ++jj) v = (jj == j) ? g[i][jj] : v;
      red[rslot * width + lcol * CPT2 + i] = v;
    }
    __syncthreads();
    for (int col = tid; col < width; col += kThreads) {
      float s = 0.0f;
      for (int q = 0; q < rs; ++q) s += red[q * width + col];
      if (slot0 + col < nslot) p.partial[((b * p.nchunks + chunk) * p.K + j) * p.P + slot0 + col] = s;
    }
    __syncthreads();
  }

  // Level 1: per (batch row, slab) over its chunks.
  if (!elect_last(p.cnt1 + b * p.nslabs + slab, (int)p.nchunks, &flag)) return;
  for (int col = tid; col < width; col += kThreads) {
    const int64_t s = slot0 + col;
    if (s >= nslot) continue;
    for (int j = 0; j < p.K; ++j) {
      float t = 0.0f;
      for (int64_t k = 0; k < p.nchunks; ++k) t += p.partial[((b * p.nchunks + k) * p.K + j) * p.P + s];
      p.fmean[(b * p.K + j) * p.P + s] = t;
    }
  }
  // Level 2: per slab over the batch.
  if (!elect_last(p.cnt2 + slab, (int)p.B, &flag)) return;
  for (int col = tid; col < width; col += kThreads) {
    const int64_t s = slot0 + col;
    if (s >= nslot) continue;
    const int64_t ch = slot_chan<CPT, MODE>(s, p.P);
    for (int j = 0; j < p.K; ++j) {
      float t = 0.0f;
      for (int64_t bb = 0; bb < p.B; ++bb) t += p.fmean[(bb * p.K + j) * p.P + s];
      p.gc[ch * p.K + j] = t;
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch over (dtype, CPT, K bound, mode).
// ---------------------------------------------------------------------------
template <typename T, int CPT, int KM>
static hipError_t launch_mode(const AggParams& p, bool bwd, hipStream_t st) {
  const dim3 grid((unsigned)(p.B * p.nchunks * p.nslabs)), block(kThreads);
  switch (p.mode) {
#define POM_CASE(M)                                                                     \
  case M:                                                                               \
    if (bwd) hipLaunchKernelGGL((agg_bwd_kernel<T, CPT, KM, M>), grid, block, 0, st, p); \
    else hipLaunchKernelGGL((agg_fwd_kernel<T, CPT, KM, M>), grid, block, 0, st, p);     \
    break;
    POM_CASE(MODE_PLAIN)
    POM_CASE(MODE_MASKED)
    POM_CASE(MODE_ROPE1D)
    POM_CASE(MODE_ROPE2D)
#undef POM_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int CPT>
static hipError_t launch_k(const AggParams& p, bool bwd, hipStream_t st) {
  if (p.K <= 2) return launch_mode<T, CPT, 2>(p, bwd, st);
  if (p.K <= 4) return launch_mode<T, CPT, 4>(p, bwd, st);
  if (p.K <= 8) return launch_mode<T, CPT, 8>(p, bwd, st);
  return launch_mode<T, CPT, 16>(p, bwd, st);
}

template <typename T>
static hipError_t launch_t(const AggParams& p, bool bwd, hipStream_t st) {
  switch (p.cpt) {
    case 8: if constexpr (sizeof(T) == 2) return launch_k<T, 8>(p, bwd, st); else break;
    case 4: return launch_k<T, 4>(p, bwd, st);
    case 2: return launch_k<T, 2>(p, bwd, st);
    case 1: return launch_k<T, 1>(p, bwd, st);
    default: break;
  }
  return hipErrorInvalidValue;
}

hipError_t launch_agg(const AggParams& p, bool bwd, hipStream_t st) {
  switch (p.dtype) {
    case DT_F32: return launch_t<float>(p, bwd, st);
    case DT_BF16: return launch_t<__hip_bfloat16>(p, bwd, st);
    case DT_F16: return launch_t<__half>(p, bwd, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pom
