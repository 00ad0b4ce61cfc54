// Per-head gating of the Polynomial Mixer (n_sel_heads = H > 1) for gfx950.
//
// Forward (pom/pom.py:118-122 with the gate of pom/pom.py:207 and the query
// RoPE of pom/pom_rope.py:417-437, :522), P = H * hd channels:
//   s[b,n,h]  = hardsigmoid(y_s[b,n,h] + bias[h])             (H gate channels)
//   s'        = R(pos_n) s                                    (RoPE over the H channels)
//   sh[b,n,c] = s'[b,n,c / hd] * hagg[b, group(n), c]
// One thread per V-element chunk of a token row (V divides hd, so a chunk lies
// in one head); the gate scalars are recomputed per chunk from cached loads.
//
// Backward:
//   ds'[b,n,h]  = sum_{c in head h} dsh[b,n,c] * hagg[b,g,c]
//   ds = R^T ds',  dz = ds * hardsigmoid'(z)  -> dY_s, dbias[h] = sum_{b,n} dz
//   dhagg[b,g,c] = sum_{n in g} s'[b,n,c / hd] * dsh[b,n,c]
// heads_bwd_token: one wave per token row forms the head sums from per-chunk
// dot products staged in LDS (fixed order), then dz, dY_s, s' (fp32 scratch)
// and workgroup bias partials.  heads_bwd_hagg: channel-parallel sums of
// s' * dsh over each group's tokens, in chunks; heads_bwd_finalize adds the
// chunk and bias partials in a fixed order.
#pragma once

#include "agg_impl.h"

namespace pom {

// cos / sin of one table column for token n (position clamped into the table).
__device__ __forceinline__ void table_cs(const RopeTables& t, int table, int64_t n, int64_t col, float& cs,
                                         float& sn) {
  int64_t pos = t.pos[n * t.pos_sn + table];
  const int64_t rows = table ? t.rows1 : t.rows0;
  pos = pos < 0 ? 0 : (pos >= rows ? rows - 1 : pos);
  cs = (table ? t.cos1 : t.cos0)[pos * t.stride + col];
  sn = (table ? t.sin1 : t.sin0)[pos * t.stride + col];
}

// Rotation pair of head h over H gate channels: (blk, col, partner, table).
template <int MODE>
__device__ __forceinline__ void head_pair(int64_t H, int64_t h, int& blk, int64_t& col, int64_t& partner,
                                          int& table) {
  if constexpr (MODE == MODE_ROPE1D) {
    const int64_t half = H / 2;
    blk = h < half ? 0 : 1;
    col = blk ? h - half : h;
    partner = blk ? h - half : h + half;
    table = 0;
  } else {
    const int64_t q = H / 4;
    const int64_t qb = h / q;
    col = h - qb * q;
    blk = (int)(qb & 1);
    partner = blk ? h - q : h + q;
    table = qb >= 2;
  }
}

// Gate value of head h for token n: rotated hardsigmoid of y_s + bias.
// 1-D: pair (h, h + H/2) on table column h mod H/2.  2-D: q = H/4, pairs
// (h, h + q) for h < q on the row table and (2q + j, 3q + j) on the column
// table (the full-width channel layout of pom/pom_rope.py:183-235 applied to
// the H gate channels).
template <typename T, int MODE>
__device__ __forceinline__ float head_gate(const HeadsParams& p, const T* __restrict__ yrow, int64_t n, int64_t h) {
  auto sg = [&](int64_t k) {
    const float z = to_f32<T>(yrow[k]) + (p.bias.ptr ? param_get(p.bias, k) : 0.0f);
    return hsig(z);
  };
  const float s = sg(h);
  if constexpr (MODE == MODE_PLAIN) {
    return s;
  } else {
    int blk, table;
    int64_t col, partner;
    head_pair<MODE>(p.H, h, blk, col, partner, table);
    const float sp = sg(partner);
    float cs, sn;
    table_cs(p.rope, table, n, col, cs, sn);
    return blk ? s * cs + sp * sn : s * cs - sp * sn;
  }
}

template <typename T, int V, int MODE>
__global__ void __launch_bounds__(kThreads) heads_fwd_kernel(const HeadsParams p) {
  const int64_t cpr = p.P / V;
  const int64_t total = p.B * p.N * cpr;
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total; idx += stride) {
    const int64_t row = idx / cpr, j = idx - row * cpr;
    const int64_t b = row / p.N, n = row - b * p.N;
    const int64_t c0 = j * V, h = c0 / p.hd;
    const T* yrow = reinterpret_cast<const T*>(p.ys) + b * p.ysb + n * p.ysn;
    const float g = head_gate<T, MODE>(p, yrow, n, h);
    float hv[V], o[V];
    VecIO<T, V>::load(reinterpret_cast<const T*>(p.hagg) + (b * p.G + n / p.L) * p.P + c0, hv);
#pragma unroll
    for (int v = 0; v < V; ++v) o[v] = g * hv[v];
    VecIO<T, V>::store(reinterpret_cast<T*>(p.sh) + b * p.shb + n * p.shn + c0, o);
  }
}

// Backward, token rows: every wave of a workgroup takes one row per round
// (rounds are uniform over the workgroup, so the barriers are too).
template <typename T, int V, int MODE>
__global__ void __launch_bounds__(kThreads) heads_bwd_token_kernel(const HeadsParams p) {
  extern __shared__ float hs_smem[];
  const int w = threadIdx.x >> 6, l = threadIdx.x & (kWave - 1);
  const int64_t cpr = p.P / V, cph = p.hd / V, H = p.H;
  float* dots = hs_smem + w * (cpr + 2 * H);   // per-chunk dot products of this wave's row
  float* dsp = dots + cpr;                     // d s' per head
  float* dbl = dsp + H;                        // this wave's bias-gradient sums
  for (int64_t h = l; h < H; h += kWave) dbl[h] = 0.0f;
  const int64_t ntok = p.B * p.N;
  for (int64_t base = (int64_t)blockIdx.x * kWaves; base < ntok; base += (int64_t)gridDim.x * kWaves) {
    const int64_t tok = base + w;
    const bool live = tok < ntok;
    const int64_t b = live ? tok / p.N : 0, n = live ? tok - b * p.N : 0;
    if (live) {
      const T* grow = reinterpret_cast<const T*>(p.dsh) + b * p.dsb + n * p.dsn;
      const T* hrow = reinterpret_cast<const T*>(p.hagg) + (b * p.G + n / p.L) * p.P;
      for (int64_t j = l; j < cpr; j += kWave) {
        float gv[V], hv[V];
        VecIO<T, V>::load(grow + j * V, gv);
        VecIO<T, V>::load(hrow + j * V, hv);
        float d = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) d = fmaf(gv[v], hv[v], d);
        dots[j] = d;
      }
    }
    __syncthreads();
    if (live) {
      for (int64_t h = l; h < H; h += kWave) {
        float s = 0.0f;
        for (int64_t k = 0; k < cph; ++k) s += dots[h * cph + k];
        dsp[h] = s;
      }
    }
    __syncthreads();
    if (live) {
      const T* yrow = reinterpret_cast<const T*>(p.ys) + b * p.ysb + n * p.ysn;
      T* dyrow = reinterpret_cast<T*>(p.dys) + b * p.dyb + n * p.dyn;
      for (int64_t h = l; h < H; h += kWave) {
        float ds = dsp[h];
        if constexpr (MODE != MODE_PLAIN) {
          int blk, table;
          int64_t col, partner;
          head_pair<MODE>(H, h, blk, col, partner, table);
          float cs, sn;
          table_cs(p.rope, table, n, col, cs, sn);
          // R = [[c, -s], [s, c]] on (first, second); R^T maps (d first', d second')
          // to (c d1 + s d2, -s d1 + c d2)
          ds = blk ? dsp[h] * cs - dsp[partner] * sn : dsp[h] * cs + dsp[partner] * sn;
        }
        const float z = to_f32<T>(yrow[h]) + (p.bias.ptr ? param_get(p.bias, h) : 0.0f);
        const float dz = ds * hsig_grad(z);
        dyrow[h] = from_f32<T>(dz);
        dbl[h] += dz;
        p.sgate[tok * H + h] = head_gate<T, MODE>(p, yrow, n, h);
      }
    }
    __syncthreads();
  }
  __syncthreads();
  // workgroup bias partial: the waves' sums in wave order
  for (int64_t h = threadIdx.x; h < H; h += kThreads) {
    float s = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) s += hs_smem[ww * (cpr + 2 * H) + cpr + H + h];
    p.part_b[(int64_t)blockIdx.x * H + h] = s;
  }
}

// Backward, aggregate gradient: thread = one V-chunk of channels, walking the
// rows of one chunk of one group.
template <typename T, int V>
__global__ void __launch_bounds__(kThreads) heads_bwd_hagg_kernel(const HeadsParams p) {
  const int64_t cpr = p.P / V;
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= cpr) return;   // no barriers below
  const int64_t chunk = blockIdx.y, b = blockIdx.z;
  const int64_t f = chunk / p.cpf;
  const int64_t rbeg = f * p.L + (chunk - f * p.cpf) * p.RC;
  int64_t rend = rbeg + p.RC;
  if (rend > (f + 1) * p.L) rend = (f + 1) * p.L;
  const int64_t c0 = j * V, h = c0 / p.hd;
  const T* gb = reinterpret_cast<const T*>(p.dsh) + b * p.dsb;
  const float* sg = p.sgate + b * p.N * p.H + h;
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  for (int64_t n = rbeg; n < rend; ++n) {
    float gv[V];
    VecIO<T, V>::load(gb + n * p.dsn + c0, gv);
    const float s = sg[n * p.H];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = fmaf(s, gv[v], acc[v]);
  }
  float* dst = p.cpf == 1 ? p.dhagg + (b * p.G + f) * p.P : p.part_h + (b * p.nch + chunk) * p.P;
#pragma unroll
  for (int v = 0; v < V; ++v) dst[c0 + v] = acc[v];
}

// dhagg = sum of each group's chunk partials (cpf > 1); dbias[h] = sum of the
// workgroup partials, one workgroup per head: strided per-thread sums, then a
// fixed tree over the threads.
static __global__ void __launch_bounds__(kThreads) heads_bwd_finalize(const HeadsParams p, int64_t nparts) {
  __shared__ float red[kThreads];
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (p.cpf > 1 && idx < p.B * p.G * p.P) {
    const int64_t c = idx % p.P, bf = idx / p.P, b = bf / p.G, f = bf - b * p.G;
    float s = 0.0f;
    for (int64_t k = 0; k < p.cpf; ++k) s += p.part_h[(b * p.nch + f * p.cpf + k) * p.P + c];
    p.dhagg[idx] = s;
  }
  if (p.dbias.ptr && blockIdx.x < p.H) {
    const int64_t h = blockIdx.x;
    float s = 0.0f;
    for (int64_t r = threadIdx.x; r < nparts; r += kThreads) s += p.part_b[r * p.H + h];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
      if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
      __syncthreads();
    }
    if (threadIdx.x == 0) param_set(p.dbias, h, red[0]);
  }
}

template <typename T, int V>
hipError_t heads_fwd_v(const HeadsParams& p, hipStream_t st) {
  const int64_t total = p.B * p.N * (p.P / V);
  int64_t nb = (total + kThreads - 1) / kThreads;
  if (nb > 16384) nb = 16384;
  const dim3 grid((unsigned)nb), block(kThreads);
  switch (p.mode) {
    case MODE_PLAIN: hipLaunchKernelGGL((heads_fwd_kernel<T, V, MODE_PLAIN>), grid, block, 0, st, p); break;
    case MODE_ROPE1D: hipLaunchKernelGGL((heads_fwd_kernel<T, V, MODE_ROPE1D>), grid, block, 0, st, p); break;
    case MODE_ROPE2D: hipLaunchKernelGGL((heads_fwd_kernel<T, V, MODE_ROPE2D>), grid, block, 0, st, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int V>
hipError_t heads_bwd_v(const HeadsParams& p, hipStream_t st) {
  const dim3 block(kThreads);
  const dim3 tgrid((unsigned)p.tok_wgs);
  const size_t smem = heads_token_smem_bytes(p.P / V, p.H);
  switch (p.mode) {
    case MODE_PLAIN: hipLaunchKernelGGL((heads_bwd_token_kernel<T, V, MODE_PLAIN>), tgrid, block, smem, st, p); break;
    case MODE_ROPE1D: hipLaunchKernelGGL((heads_bwd_token_kernel<T, V, MODE_ROPE1D>), tgrid, block, smem, st, p); break;
    case MODE_ROPE2D: hipLaunchKernelGGL((heads_bwd_token_kernel<T, V, MODE_ROPE2D>), tgrid, block, smem, st, p); break;
    default: return hipErrorInvalidValue;
  }
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  const dim3 hgrid((unsigned)((p.P / V + kThreads - 1) / kThreads), (unsigned)p.nch, (unsigned)p.B);
  hipLaunchKernelGGL((heads_bwd_hagg_kernel<T, V>), hgrid, block, 0, st, p);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  const int64_t flat = p.cpf > 1 ? (p.B * p.G * p.P + kThreads - 1) / kThreads : 0;
  const int64_t nb = flat > p.H ? flat : (p.dbias.ptr ? p.H : flat);
  if (nb > 0) hipLaunchKernelGGL(heads_bwd_finalize, dim3((unsigned)nb), block, 0, st, p, p.tok_wgs);
  return hipGetLastError();
}

#define POM_V_SWITCH(T_, V_, FN, ...)                                       \
  switch (V_) {                                                             \
    case 8: if constexpr (sizeof(T_) == 2) return FN<T_, 8>(__VA_ARGS__); else break; \
    case 4: return FN<T_, 4>(__VA_ARGS__);                                  \
    case 2: return FN<T_, 2>(__VA_ARGS__);                                  \
    case 1: return FN<T_, 1>(__VA_ARGS__);                                  \
    default: break;                                                         \
  }                                                                         \
  return hipErrorInvalidValue;

template <typename T>
hipError_t heads_fwd_t(const HeadsParams& p, hipStream_t st) {
  POM_V_SWITCH(T, p.V, heads_fwd_v, p, st)
}

template <typename T>
hipError_t heads_bwd_t(const HeadsParams& p, hipStream_t st) {
  POM_V_SWITCH(T, p.V, heads_bwd_v, p, st)
}

}  // namespace pom
