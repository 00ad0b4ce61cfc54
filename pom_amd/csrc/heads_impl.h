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
// Tile path (the common shapes): heads_fwd_tile / heads_bwd_tile below.
// General path: heads_bwd_token: one wave per token row forms the head sums
// from per-chunk dot products staged in LDS (fixed order), then dz, dY_s, s'
// (fp32 scratch) and workgroup bias partials.  heads_bwd_hagg:
// channel-parallel sums of s' * dsh over each group's tokens, in chunks;
// heads_bwd_finalize adds the chunk and bias partials in a fixed order.
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
  // every load (y_s and bias of the head and its rotation partner, the table
  // entries) is issued before any of them is used
  int64_t k[2] = {h, h};
  int blk = 0, table = 0;
  int64_t col = 0;
  if constexpr (MODE != MODE_PLAIN) head_pair<MODE>(p.H, h, blk, col, k[1], table);
  const T y0 = yrow[k[0]], y1 = yrow[k[1]];
  float bv[2] = {0.0f, 0.0f};
  if (p.bias.ptr) param_gather<2>(p.bias, [&](int q) { return k[q]; }, bv);
  const float s = hsig(to_f32<T>(y0) + bv[0]);
  if constexpr (MODE == MODE_PLAIN) {
    return s;
  } else {
    float cs, sn;
    table_cs(p.rope, table, n, col, cs, sn);
    const float sp = hsig(to_f32<T>(y1) + bv[1]);
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

// ---------------------------------------------------------------------------
// Tile kernels: a workgroup owns kTT tokens of one batch row x kCT channels.
// Used when P % 8 == 0 (8-element chunks), the operands admit 8-element
// vectors, and every tile lies in one hagg group (L % kTT == 0) or groups are
// single tokens (L == 1).  The gate values of the tile's tokens and heads are
// formed once per tile; the backward reads dsh once, forming both the
// per-head dot products (over the tile's channels) and the aggregate-gradient
// sums (over its tokens) from an LDS copy.
// Forward row walk (plain gate, no channel-major copy, head_dim % 8 == 0, one
// hagg row per batch row): 32 lanes x 8 channels of a token row, eight rows
// per workgroup step.  A lane's 8 channels lie in one head, so its hagg chunk
// and the head's bias are loaded once; each row then costs one gate load and
// one 16-byte store, the arithmetic of heads_fwd_tile (bit-identical sh).
template <typename T>
__global__ void __launch_bounds__(kThreads) heads_fwd_rows(const HeadsParams p) {
  constexpr int U = 4;                                   // rows per lane in flight
  constexpr int kSlots = kThreads / kFwdRowLanes;        // token rows per workgroup step
  const int tid = threadIdx.x, lc = tid % kFwdRowLanes, slot = tid / kFwdRowLanes;
  const int64_t b = blockIdx.z;
  const int64_t c0 = ((int64_t)blockIdx.x * kFwdRowLanes + lc) * 8;
  if (c0 >= p.P) return;   // no barriers below
  const int64_t n0 = (int64_t)blockIdx.y * p.fwd_rows;
  const int64_t n1 = n0 + p.fwd_rows < p.N ? n0 + p.fwd_rows : p.N;
  const int64_t h = c0 / p.hd;
  float hv[8];
  VecIO<T, 8>::load(reinterpret_cast<const T*>(p.hagg) + b * p.P + c0, hv);
  float bias = 0.0f;
  if (p.bias.ptr) {
    float bv[1];
    param_gather<1>(p.bias, [&](int) { return h; }, bv);
    bias = bv[0];
  }
  const T* yb = reinterpret_cast<const T*>(p.ys) + b * p.ysb + h;
  T* ob = reinterpret_cast<T*>(p.sh) + b * p.shb + c0;
  for (int64_t n = n0 + slot; n < n1; n += U * kSlots) {
    T yv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = n + (int64_t)u * kSlots;
      yv[u] = yb[(r < n1 ? r : n) * p.ysn];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t r = n + (int64_t)u * kSlots;
      if (r >= n1) break;
      const float g = hsig(to_f32<T>(yv[u]) + bias);
      float o[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) o[v] = g * hv[v];
      VecIO<T, 8>::store(ob + r * p.shn, o);
    }
  }
}

template <typename T>
hipError_t heads_rows_fwd(const HeadsParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.P / 8 + kFwdRowLanes - 1) / kFwdRowLanes), (unsigned)((p.N + p.fwd_rows - 1) / p.fwd_rows),
                  (unsigned)p.B);
  hipLaunchKernelGGL((heads_fwd_rows<T>), grid, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
constexpr int kTT = 64, kCT = 64;
constexpr int kGM = kCT / 8 + 1;   // heads a kCT-channel tile can touch (head_dim >= 8 on this path)

// Per-tile prologue: local head of each channel and the gate values s'[t][hi].
template <typename T, int MODE>
__device__ __forceinline__ void tile_gates(const HeadsParams& p, int64_t b, int64_t n0, int64_t c0, int nt, int nc,
                                           int64_t& h0, int& nh, int* hidx, float* gs) {
  h0 = c0 / p.hd;
  nh = (int)((c0 + nc - 1) / p.hd - h0) + 1;
  const int tid = threadIdx.x;
  if (tid < nc) hidx[tid] = (int)((c0 + tid) / p.hd - h0);
  const T* yb = reinterpret_cast<const T*>(p.ys) + b * p.ysb;
  for (int i = tid; i < nt * nh; i += kThreads) {
    const int t = i / nh, hi = i - t * nh;
    const int64_t n = n0 + t;
    gs[t * kGM + hi] = head_gate<T, MODE>(p, yb + n * p.ysn, n, h0 + hi);
  }
}

template <typename T, int MODE, bool TR>
__global__ void __launch_bounds__(kThreads) heads_fwd_tile(const HeadsParams p) {
  constexpr int PITCH = kTT + 8;   // [channel][token] rows of 16-byte multiples, staggered banks
  __shared__ float gs[kTT * kGM];
  __shared__ int hidx[kCT];
  __shared__ __attribute__((aligned(16))) T tt[TR ? kCT * PITCH : 8];
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.z, n0 = (int64_t)blockIdx.y * kTT, c0 = (int64_t)blockIdx.x * kCT;
  const int nt = (int)(p.N - n0 < kTT ? p.N - n0 : kTT), nc = (int)(p.P - c0 < kCT ? p.P - c0 : kCT);
  // this thread's two chunks (t, j) = (i >> 3, i & 7), i = tid and tid + 256:
  // their hagg rows are loaded before the gate values are formed, so the two
  // memory latencies overlap
  const int cj = nc / 8;
  const T* hb = reinterpret_cast<const T*>(p.hagg) + c0;
  constexpr int R = kTT * 8 / kThreads;
  Pack<T, 8> hp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid + r * kThreads, t = i >> 3, j = i & 7;
    if (t < nt && j < cj) hp[r].load(hb + (b * p.G + (n0 + t) / p.L) * p.P + j * 8);
  }
  int64_t h0;
  int nh;
  tile_gates<T, MODE>(p, b, n0, c0, nt, nc, h0, nh, hidx, gs);
  __syncthreads();
  T* ob = reinterpret_cast<T*>(p.sh) + b * p.shb + c0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = tid + r * kThreads, t = i >> 3, j = i & 7;
    if (t >= nt || j >= cj) continue;
    const int cc = j * 8;
    float o[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) o[v] = gs[t * kGM + hidx[cc + v]] * hp[r].get(v);
    VecIO<T, 8>::store(ob + (n0 + t) * p.shn + cc, o);
    if constexpr (TR) {
#pragma unroll
      for (int v = 0; v < 8; ++v) tt[(cc + v) * PITCH + t] = from_f32<T>(o[v]);
    }
  }
  if constexpr (TR) {
    __syncthreads();
    using Raw = typename RawVec<16>::type;
    T* base = reinterpret_cast<T*>(p.sht.data) + b * p.sht.sb + n0;
    const int tj = nt / 8;   // N % 8 == 0 on this path
    for (int i = tid; i < nc * 8; i += kThreads) {
      const int cc = i >> 3, k = i & 7;
      if (k >= tj) continue;
      *reinterpret_cast<Raw*>(base + (c0 + cc) * p.sht.ld + k * 8) =
          *reinterpret_cast<const Raw*>(tt + cc * PITCH + k * 8);
    }
  }
}

template <typename T, int MODE>
__global__ void __launch_bounds__(kThreads) heads_bwd_tile(const HeadsParams p) {
  constexpr int DP = kCT + 1;   // fp32 tile pitch: conflict-free columns
  __shared__ float gs[kTT * kGM];
  __shared__ float pr[kTT * DP];      // s' * dsh (groups of kTT or more tokens)
  __shared__ float cd[kTT * 8 * 2];   // per chunk: the dot product's parts on its first / second head
  __shared__ float red[4 * kCT];
  __shared__ int hidx[kCT];
  const int tid = threadIdx.x;
  // this workgroup walks p.tpw consecutive token tiles of one batch row (inside one group)
  const int64_t b = blockIdx.z, c0 = (int64_t)blockIdx.x * kCT;
  const int64_t n_first = (int64_t)blockIdx.y * p.tpw * kTT;
  const int nc = (int)(p.P - c0 < kCT ? p.P - c0 : kCT);
  const bool per_token = p.L == 1;
  const int cj = nc / 8;
  const T* gb = reinterpret_cast<const T*>(p.dsh) + b * p.dsb + c0;
  const T* hb = reinterpret_cast<const T*>(p.hagg) + b * p.G * p.P + c0;
  const int64_t nct = (p.P + kCT - 1) / kCT;
  constexpr int R = kTT * 8 / kThreads;
  Pack<T, 8> gp[R], hp[R];
  // loads of one tile's dsh (and hagg) chunks: (t, j) = (i >> 3, i & 7), i = tid + r * 256
  auto load_tile = [&](int64_t n0, int nt) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = tid + r * kThreads, t = i >> 3, j = i & 7;
      if (t < nt && j < cj) {
        gp[r].load(gb + (n0 + t) * p.dsn + j * 8);
        hp[r].load(hb + (per_token ? n0 + t : n0 / p.L) * p.P + j * 8);
      }
    }
  };
  const int ntiles = (int)((p.N - n_first + kTT - 1) / kTT) < p.tpw ? (int)((p.N - n_first + kTT - 1) / kTT) : p.tpw;
  float acc = 0.0f;   // this thread's quarter sum of s' * dsh (channel tid & 63), over the walk
  load_tile(n_first, (int)(p.N - n_first < kTT ? p.N - n_first : kTT));
  for (int k = 0; k < ntiles; ++k) {
    const int64_t n0 = n_first + (int64_t)k * kTT;
    const int nt = (int)(p.N - n0 < kTT ? p.N - n0 : kTT);
    int64_t h0;
    int nh;
    __syncthreads();   // the previous tile's readers of gs / cd / pr are done
    tile_gates<T, MODE>(p, b, n0, c0, nt, nc, h0, nh, hidx, gs);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = tid + r * kThreads, t = i >> 3, j = i & 7;
      if (t >= nt || j >= cj) continue;
      const int cc = j * 8, ha = hidx[cc];
      float pa = 0.0f, pb = 0.0f, o[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int hv = hidx[cc + v];
        const float g = gp[r].get(v), d = g * hp[r].get(v);
        if (hv == ha) pa += d;
        else pb += d;
        o[v] = gs[t * kGM + hv] * g;
      }
      cd[i * 2] = pa;
      cd[i * 2 + 1] = pb;
      if (per_token) {
        store_f32<8>(p.dhagg + (b * p.G + n0 + t) * p.P + c0 + cc, o);
      } else {
#pragma unroll
        for (int v = 0; v < 8; ++v) pr[t * DP + cc + v] = o[v];
      }
    }
    // the next tile's loads go out before this tile's reductions
    if (k + 1 < ntiles) {
      const int64_t n1 = n0 + kTT;
      load_tile(n1, (int)(p.N - n1 < kTT ? p.N - n1 : kTT));
    }
    __syncthreads();
    for (int i = tid; i < nt * nh; i += kThreads) {
      const int t = i / nh, hi = i - t * nh;
      float d = 0.0f;
      for (int j = 0; j < cj; ++j) {
        const int ha = hidx[j * 8], hz = hidx[j * 8 + 7];
        d += (ha == hi ? cd[(t * 8 + j) * 2] : 0.0f) + (hz == hi && hz != ha ? cd[(t * 8 + j) * 2 + 1] : 0.0f);
      }
      p.dpart[((b * p.N + n0 + t) * nct + blockIdx.x) * p.nhm + hi] = d;
    }
    if (!per_token) {
      const int c = tid & (kCT - 1), q = tid >> 6;
      if (c < nc) {
        const int te = (q + 1) * (kTT / 4) < nt ? (q + 1) * (kTT / 4) : nt;
        for (int t = q * (kTT / 4); t < te; ++t) acc += pr[t * DP + c];
      }
    }
  }
  if (!per_token) {
    // the walk's sum over its tokens: four token quarters, then a fixed sum
    red[tid] = acc;
    __syncthreads();
    if (tid < nc)
      p.part_h[(b * p.ntt + blockIdx.y) * p.P + c0 + tid] =
          ((red[tid] + red[kCT + tid]) + red[2 * kCT + tid]) + red[3 * kCT + tid];
  }
}

constexpr int kDzT = 16;   // tokens per workgroup of the dz kernel (= rows per bias partial)

template <typename T, int MODE>
__global__ void __launch_bounds__(kThreads) heads_bwd_dz(const HeadsParams p) {
  extern __shared__ float dzl[];   // [kDzT][H]
  const int64_t ntok = p.B * p.N, tok0 = (int64_t)blockIdx.x * kDzT;
  const int nt = (int)(ntok - tok0 < kDzT ? ntok - tok0 : kDzT);
  const int H = (int)p.H;
  const int64_t nct = (p.P + kCT - 1) / kCT;
  for (int i = threadIdx.x; i < nt * H; i += kThreads) {
    const int t = i / H, h = i - t * H;
    const int64_t tok = tok0 + t;
    const int64_t b = tok / p.N, n = tok - b * p.N;
    auto dsp = [&](int64_t hh) {
      const int64_t ca = hh * p.hd, cb = ca + p.hd - 1;
      float s = 0.0f;
      for (int64_t ct = ca / kCT; ct <= cb / kCT; ++ct)
        s += p.dpart[(tok * nct + ct) * p.nhm + (hh - (ct * kCT) / p.hd)];
      return s;
    };
    float ds = dsp(h);
    if constexpr (MODE != MODE_PLAIN) {
      int blk, table;
      int64_t col, partner;
      head_pair<MODE>(p.H, h, blk, col, partner, table);
      float cs, sn;
      table_cs(p.rope, table, n, col, cs, sn);
      const float dq = dsp(partner);
      ds = blk ? ds * cs - dq * sn : ds * cs + dq * sn;
    }
    const T* yrow = reinterpret_cast<const T*>(p.ys) + b * p.ysb + n * p.ysn;
    const float z = to_f32<T>(yrow[h]) + (p.bias.ptr ? param_get(p.bias, h) : 0.0f);
    const float dz = ds * hsig_grad(z);
    reinterpret_cast<T*>(p.dys)[b * p.dyb + n * p.dyn + h] = from_f32<T>(dz);
    dzl[i] = dz;
  }
  __syncthreads();
  for (int h = threadIdx.x; h < H; h += kThreads) {
    float s = 0.0f;
    for (int t = 0; t < nt; ++t) s += dzl[t * H + h];
    p.dzbuf[blockIdx.x * p.H + h] = s;
  }
}

// dhagg[b, g, c] = sum of the group's token-tile partials (groups of L >= kTT
// tokens); dbias[h] = sum over every token of dz (one workgroup per head,
// strided sums then a fixed tree).
static __global__ void __launch_bounds__(kThreads) heads_tile_finalize(const HeadsParams p) {
  __shared__ float red[kThreads];
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (p.L > 1 && idx < p.B * p.G * p.P) {
    const int64_t c = idx % p.P, bg = idx / p.P, b = bg / p.G, g = bg - b * p.G;
    // walks per group (a single group may end in a partial walk)
    const int64_t per = p.G == 1 ? p.ntt : p.L / (p.rows ? p.wt : kTT * p.tpw);
    const float* src = p.part_h + (b * p.ntt + g * per) * p.P + c;
    float s = 0.0f;
    int64_t k = 0;
    for (; k + 8 <= per; k += 8) {   // eight loads in flight, summed in order
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = src[(k + q) * p.P];
#pragma unroll
      for (int q = 0; q < 8; ++q) s += v[q];
    }
    for (; k < per; ++k) s += src[k * p.P];
    p.dhagg[idx] = s;
  }
  if (p.dbias.ptr && blockIdx.x < p.H) {
    // dz partial rows: one per walk (row path) or per 16 tokens (dz kernel)
    const int64_t h = blockIdx.x, rows = p.rows ? p.B * p.ntt : (p.B * p.N + kDzT - 1) / kDzT;
    float s = 0.0f;
    for (int64_t r = threadIdx.x; r < rows; r += kThreads) s += p.dzbuf[r * p.H + h];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int off = kThreads / 2; off > 0; off >>= 1) {
      if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
      __syncthreads();
    }
    if (threadIdx.x == 0) param_set(p.dbias, h, red[0]);
  }
}

// ---------------------------------------------------------------------------
// Row path of the backward (head_dim % 8 == 0, groups of more than one token).
// A workgroup walks p.wt tokens of one batch row over all P channels: thread j
// owns channels 8j..8j+7, which lie in one head.  Per step of kRowU tokens
// each thread adds s' * dsh into its dhagg partial (registers, whole walk) and
// writes its chunk's share of the head dot product into LDS; after one
// barrier, thread (t, h) sums head h's chunks for token t, applies R^T and
// hardsigmoid', writes dY_s and keeps its dz sum.  The dot products are
// double-buffered, so a step needs no second barrier.  dsh is read once and
// no partial leaves the workgroup except the walk's dhagg and dz sums.
// ---------------------------------------------------------------------------
constexpr int kRowU = kHeadsRowU;

template <typename T, int MODE>
__global__ void __launch_bounds__(1024) heads_bwd_rows(const HeadsParams p) {
  extern __shared__ float dots[];   // [2][kRowU][J]; reused for the dz sums at the end
  const int tid = threadIdx.x;
  const int J = (int)(p.P / 8), hd8 = (int)(p.hd / 8), H = (int)p.H;
  const int64_t b = blockIdx.y, w = blockIdx.x;
  const int64_t nbeg = w * p.wt, nend = nbeg + p.wt < p.N ? nbeg + p.wt : p.N;
  const int64_t grp = nbeg / p.L;
  const T* yb = reinterpret_cast<const T*>(p.ys) + b * p.ysb;

  // chunk role: channels c0..c0+7 of head hj
  const bool own = tid < J;
  const int j = own ? tid : 0;
  const int64_t c0 = (int64_t)j * 8, hj = j / hd8;
  int blk = 0, table = 0;
  int64_t col = 0, partner = hj;
  if constexpr (MODE != MODE_PLAIN) head_pair<MODE>(p.H, hj, blk, col, partner, table);
  float bj[2] = {0.0f, 0.0f};
  if (p.bias.ptr) param_gather<2>(p.bias, [&](int q) { return q ? partner : hj; }, bj);
  float hv[8];
  {
    Pack<T, 8> hp;
    hp.load(reinterpret_cast<const T*>(p.hagg) + (b * p.G + grp) * p.P + c0);
#pragma unroll
    for (int v = 0; v < 8; ++v) hv[v] = hp.get(v);
  }
  const T* gb = reinterpret_cast<const T*>(p.dsh) + b * p.dsb + c0;

  // reduction role: slot (rt, hr) for tid < kRowU * H
  const bool red = tid < kRowU * H;
  const int rt = red ? tid / H : 0, hr = red ? tid - rt * H : 0;
  int rblk = 0, rtable = 0;
  int64_t rcol = 0, rpartner = hr;
  if constexpr (MODE != MODE_PLAIN) head_pair<MODE>(p.H, hr, rblk, rcol, rpartner, rtable);
  const float bz = (red && p.bias.ptr) ? param_get(p.bias, hr) : 0.0f;
  float dzacc = 0.0f;

  float acc[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) acc[v] = 0.0f;
  Pack<T, 8> gp[kRowU];
  T y0[kRowU], y1[kRowU], yz = T();
  // one step's loads (the chunk rows and gate inputs, and the reduction slot's
  // y_s), all issued together: a load issued after them would wait for them
  // all; rows past the walk re-read its last row (never used)
  auto load = [&](int64_t n0) {
    if (own) {
#pragma unroll
      for (int u = 0; u < kRowU; ++u) {
        const int64_t n = n0 + u < nend ? n0 + u : nend - 1;
        gp[u].load(gb + n * p.dsn);
        y0[u] = yb[n * p.ysn + hj];
        if constexpr (MODE != MODE_PLAIN) y1[u] = yb[n * p.ysn + partner];
      }
    }
    if (red) yz = yb[(n0 + rt < nend ? n0 + rt : nend - 1) * p.ysn + hr];
  };
  load(nbeg);
  int buf = 0;
  for (int64_t n0 = nbeg; n0 < nend; n0 += kRowU, buf ^= 1) {
    float* d = dots + buf * kRowU * J;
    const float zy = to_f32<T>(yz);   // this step's reduction-slot y_s
    if (own) {
#pragma unroll
      for (int u = 0; u < kRowU; ++u) {
        const int64_t n = n0 + u;
        float s = hsig(to_f32<T>(y0[u]) + bj[0]);
        if constexpr (MODE != MODE_PLAIN) {
          float cs, sn;
          table_cs(p.rope, table, n < nend ? n : nend - 1, col, cs, sn);
          const float sp = hsig(to_f32<T>(y1[u]) + bj[1]);
          s = blk ? s * cs + sp * sn : s * cs - sp * sn;
        }
        const bool in = n < nend;
        float dot = 0.0f;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const float g = gp[u].get(v);
          dot = fmaf(g, hv[v], dot);
          acc[v] = fmaf(g, in ? s : 0.0f, acc[v]);
        }
        d[u * J + j] = in ? dot : 0.0f;
      }
    }
    if (n0 + kRowU < nend) load(n0 + kRowU);   // in flight during the reduction below
    __syncthreads();   // the step's dot products are in LDS
    if (red && n0 + rt < nend) {
      const int64_t n = n0 + rt;
      const float* dr = d + rt * J;
      float ds = 0.0f;
      for (int k = 0; k < hd8; ++k) ds += dr[hr * hd8 + k];
      if constexpr (MODE != MODE_PLAIN) {
        float dq = 0.0f;
        for (int k = 0; k < hd8; ++k) dq += dr[rpartner * hd8 + k];
        float cs, sn;
        table_cs(p.rope, rtable, n, rcol, cs, sn);
        ds = rblk ? ds * cs - dq * sn : ds * cs + dq * sn;
      }
      const float z = zy + bz;
      const float dz = ds * hsig_grad(z);
      reinterpret_cast<T*>(p.dys)[b * p.dyb + n * p.dyn + hr] = from_f32<T>(dz);
      dzacc += dz;
    }
  }
  const int64_t walk = b * p.ntt + w;
  if (own) store_f32<8>(p.part_h + walk * p.P + c0, acc);
  __syncthreads();   // every step's readers of the dot products are done
  if (red) dots[tid] = dzacc;   // [rt][hr]
  __syncthreads();
  if (tid < H) {
    float sum = 0.0f;
    for (int t = 0; t < kRowU; ++t) sum += dots[t * H + tid];
    p.dzbuf[walk * H + tid] = sum;
  }
}

template <typename T, int MODE>
hipError_t heads_rows_bwd_m(const HeadsParams& p, hipStream_t st) {
  const dim3 grid((unsigned)p.ntt, (unsigned)p.B);
  hipLaunchKernelGGL((heads_bwd_rows<T, MODE>), grid, dim3(heads_rows_threads(p.P, p.H)),
                     heads_rows_smem(p.P, p.H), st, p);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  const int64_t flat = (p.B * p.G * p.P + kThreads - 1) / kThreads;
  const int64_t fb = flat > p.H ? flat : (p.dbias.ptr ? p.H : flat);
  hipLaunchKernelGGL(heads_tile_finalize, dim3((unsigned)fb), dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <typename T>
hipError_t heads_rows_bwd(const HeadsParams& p, hipStream_t st) {
  switch (p.mode) {
    case MODE_PLAIN: return heads_rows_bwd_m<T, MODE_PLAIN>(p, st);
    case MODE_ROPE1D: return heads_rows_bwd_m<T, MODE_ROPE1D>(p, st);
    case MODE_ROPE2D: return heads_rows_bwd_m<T, MODE_ROPE2D>(p, st);
    default: return hipErrorInvalidValue;
  }
}

template <typename T, int MODE>
hipError_t heads_tile_fwd_m(const HeadsParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.P + kCT - 1) / kCT), (unsigned)((p.N + kTT - 1) / kTT), (unsigned)p.B);
  if constexpr (sizeof(T) == 2) {
    if (p.sht.data) {
      hipLaunchKernelGGL((heads_fwd_tile<T, MODE, true>), grid, dim3(kThreads), 0, st, p);
      return hipGetLastError();
    }
  } else {
    if (p.sht.data) return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((heads_fwd_tile<T, MODE, false>), grid, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <typename T, int MODE>
hipError_t heads_tile_bwd_m(const HeadsParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.P + kCT - 1) / kCT), (unsigned)p.ntt, (unsigned)p.B);
  hipLaunchKernelGGL((heads_bwd_tile<T, MODE>), grid, dim3(kThreads), 0, st, p);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  const int64_t nb = (p.B * p.N + kDzT - 1) / kDzT;
  hipLaunchKernelGGL((heads_bwd_dz<T, MODE>), dim3((unsigned)nb), dim3(kThreads),
                     sizeof(float) * kDzT * (size_t)p.H, st, p);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  const int64_t flat = p.L > 1 ? (p.B * p.G * p.P + kThreads - 1) / kThreads : 0;
  const int64_t fb = flat > p.H ? flat : (p.dbias.ptr ? p.H : flat);
  if (fb > 0) hipLaunchKernelGGL(heads_tile_finalize, dim3((unsigned)fb), dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <typename T>
hipError_t heads_tile_fwd(const HeadsParams& p, hipStream_t st) {
  switch (p.mode) {
    case MODE_PLAIN: return heads_tile_fwd_m<T, MODE_PLAIN>(p, st);
    case MODE_ROPE1D: return heads_tile_fwd_m<T, MODE_ROPE1D>(p, st);
    case MODE_ROPE2D: return heads_tile_fwd_m<T, MODE_ROPE2D>(p, st);
    default: return hipErrorInvalidValue;
  }
}

template <typename T>
hipError_t heads_tile_bwd(const HeadsParams& p, hipStream_t st) {
  switch (p.mode) {
    case MODE_PLAIN: return heads_tile_bwd_m<T, MODE_PLAIN>(p, st);
    case MODE_ROPE1D: return heads_tile_bwd_m<T, MODE_ROPE1D>(p, st);
    case MODE_ROPE2D: return heads_tile_bwd_m<T, MODE_ROPE2D>(p, st);
    default: return hipErrorInvalidValue;
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
  if (p.fwd_rows > 0) return heads_rows_fwd<T>(p, st);
  if (p.tile) return heads_tile_fwd<T>(p, st);
  if (p.sht.data) return hipErrorInvalidValue;
  POM_V_SWITCH(T, p.V, heads_fwd_v, p, st)
}

template <typename T>
hipError_t heads_bwd_t(const HeadsParams& p, hipStream_t st) {
  if (p.rows) return heads_rows_bwd<T>(p, st);
  if (p.tile) return heads_tile_bwd<T>(p, st);
  POM_V_SWITCH(T, p.V, heads_bwd_v, p, st)
}

}  // namespace pom
