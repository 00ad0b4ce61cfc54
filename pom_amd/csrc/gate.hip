// Gating / selection path of the Polynomial Mixer for gfx950.
//
// Forward (pom/pom.py:207 + :103-122, with RoPE pom/pom_rope.py:522-525):
//   z  = y_s + se_bias
//   s  = hardsigmoid(z)                       (relu6(z + 3) / 6)
//   s' = R(pos_query) s                       (RoPE variants only)
//   sh = s' * hagg[b, group(token)]           (hagg fp32, group = token / Lg)
// One streaming pass: reads y_s, writes sh; everything in between stays in
// registers (the reference makes three passes: add, hardsigmoid, multiply).
//
// Backward:
//   d s' = dsh * hagg,  ds = R^T d s',  dz = ds * hardsigmoid'(z)  -> dY_s (strided)
//   dhagg[b, g] = sum_{tokens of g} dsh * s'                        (fp32)
//   dbias       = sum_{all tokens} dz                               (fp32)
// Reductions use the same chunk/slab decomposition and last-workgroup
// election as the aggregation kernels (deterministic, no float atomics).
#include "common.h"
#include "pom_internal.h"
#include "lanes.h"

namespace pom {

template <typename T, int CPT, int MODE>
__global__ void __launch_bounds__(kThreads)
gate_fwd_kernel(const GateParams p) {
  using Map = LaneMap<CPT, MODE>;
  constexpr int CPT2 = Map::CPT2;
  constexpr bool ROPE = (MODE == MODE_ROPE1D || MODE == MODE_ROPE2D);
  constexpr int U = 4;

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

  const int64_t vcol = slab * lpr + lcol;
  if (vcol >= p.nvec) return;   // no cross-lane work in the forward
  Map map;
  map.init(vcol, p.P);

  float bias[CPT2];
#pragma unroll
  for (int i = 0; i < CPT2; ++i) bias[i] = p.bias ? p.bias[map.chan(i)] : 0.0f;

  const int64_t n0 = chunk * p.RC;
  const bool row_groups = p.Lg < p.RC;   // group changes inside the chunk (Lg == 1)
  float hv[CPT2];
  if (!row_groups) {
    const int64_t g = n0 / p.Lg;
#pragma unroll
    for (int i = 0; i < CPT2; ++i) hv[i] = p.hagg[(b * p.G + g) * p.P + map.chan(i)];
  }

  const T* yb = reinterpret_cast<const T*>(p.ys) + b * p.ysb;
  T* ob = reinterpret_cast<T*>(p.sh) + b * p.shb;
  const int row0 = wave * rpw + lrow;

  for (int64_t r = row0; r < p.RC; r += (int64_t)rs * U) {
    float yv[U][CPT2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t rr = r + (int64_t)u * rs;
      if (rr < p.RC) {
        const T* row = yb + (n0 + rr) * p.ysn;
        float tmp[CPT];
        VecIO<T, CPT>::load(row + map.c1, tmp);
#pragma unroll
        for (int i = 0; i < CPT; ++i) yv[u][i] = tmp[i];
        if constexpr (ROPE) {
          VecIO<T, CPT>::load(row + map.c2, tmp);
#pragma unroll
          for (int i = 0; i < CPT; ++i) yv[u][CPT + i] = tmp[i];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t rr = r + (int64_t)u * rs;
      if (rr >= p.RC) continue;
      const int64_t n = n0 + rr;
      float s[CPT2];
#pragma unroll
      for (int i = 0; i < CPT2; ++i) s[i] = hsig(yv[u][i] + bias[i]);
      if constexpr (ROPE) {
        float cs[CPT], sn[CPT];
        load_table<CPT>(p.rope, map.table, n, map.tcol, cs, sn);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const float a = s[i], bb = s[CPT + i];
          s[i] = a * cs[i] - bb * sn[i];
          s[CPT + i] = bb * cs[i] + a * sn[i];
        }
      }
      if (row_groups) {
        const int64_t g = n / p.Lg;
#pragma unroll
        for (int i = 0; i < CPT2; ++i) hv[i] = p.hagg[(b * p.G + g) * p.P + map.chan(i)];
      }
      float o[CPT];
      T* orow = ob + n * p.shn;
#pragma unroll
      for (int i = 0; i < CPT; ++i) o[i] = s[i] * hv[i];
      VecIO<T, CPT>::store(orow + map.c1, o);
      if constexpr (ROPE) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) o[i] = s[CPT + i] * hv[CPT + i];
        VecIO<T, CPT>::store(orow + map.c2, o);
      }
    }
  }
}

template <typename T, int CPT, int MODE>
__global__ void __launch_bounds__(kThreads)
gate_bwd_kernel(const GateParams p) {
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

  const int64_t vcol = slab * lpr + lcol;
  const bool active = vcol < p.nvec;
  Map map;
  map.init(active ? vcol : 0, p.P);

  float bias[CPT2], hv[CPT2], dh[CPT2], db[CPT2];
  const int64_t n0 = chunk * p.RC;
  const bool row_groups = p.Lg < p.RC;
  const int64_t g0 = n0 / p.Lg;
#pragma unroll
  for (int i = 0; i < CPT2; ++i) {
    bias[i] = (active && p.bias) ? p.bias[map.chan(i)] : 0.0f;
    hv[i] = (active && !row_groups) ? p.hagg[(b * p.G + g0) * p.P + map.chan(i)] : 0.0f;
    dh[i] = 0.0f;
    db[i] = 0.0f;
  }

  const T* yb = reinterpret_cast<const T*>(p.ys) + b * p.ysb;
  const T* gb = reinterpret_cast<const T*>(p.dsh) + b * p.dsb;
  T* dyb = reinterpret_cast<T*>(p.dys) + b * p.dyb;
  const int row0 = wave * rpw + lrow;

  if (active) {
    for (int64_t r = row0; r < p.RC; r += (int64_t)rs * U) {
      float yv[U][CPT2], gv[U][CPT2];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t rr = r + (int64_t)u * rs;
        if (rr < p.RC) {
          const T* yrow = yb + (n0 + rr) * p.ysn;
          const T* grow = gb + (n0 + rr) * p.dsn;
          float tmp[CPT];
          VecIO<T, CPT>::load(yrow + map.c1, tmp);
#pragma unroll
          for (int i = 0; i < CPT; ++i) yv[u][i] = tmp[i];
          VecIO<T, CPT>::load(grow + map.c1, tmp);
#pragma unroll
          for (int i = 0; i < CPT; ++i) gv[u][i] = tmp[i];
          if constexpr (ROPE) {
            VecIO<T, CPT>::load(yrow + map.c2, tmp);
#pragma unroll
            for (int i = 0; i < CPT; ++i) yv[u][CPT + i] = tmp[i];
            VecIO<T, CPT>::load(grow + map.c2, tmp);
#pragma unroll
            for (int i = 0; i < CPT; ++i) gv[u][CPT + i] = tmp[i];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t rr = r + (int64_t)u * rs;
        if (rr >= p.RC) continue;
        const int64_t n = n0 + rr;
        if (row_groups) {
          const int64_t g = n / p.Lg;
#pragma unroll
          for (int i = 0; i < CPT2; ++i) hv[i] = p.hagg[(b * p.G + g) * p.P + map.chan(i)];
        }
        float z[CPT2], s[CPT2], dsr[CPT2], dcon[CPT2];
#pragma unroll
        for (int i = 0; i < CPT2; ++i) {
          z[i] = yv[u][i] + bias[i];
          s[i] = hsig(z[i]);
          dsr[i] = gv[u][i] * hv[i];   // gradient w.r.t. the (rotated) gate
        }
        float ds[CPT2];
        if constexpr (ROPE) {
          float cs[CPT], sn[CPT];
          load_table<CPT>(p.rope, map.table, n, map.tcol, cs, sn);
#pragma unroll
          for (int i = 0; i < CPT; ++i) {
            const float a = s[i], bb = s[CPT + i];
            const float r1 = a * cs[i] - bb * sn[i], r2 = bb * cs[i] + a * sn[i];
            dcon[i] = gv[u][i] * r1;
            dcon[CPT + i] = gv[u][CPT + i] * r2;
            ds[i] = dsr[i] * cs[i] + dsr[CPT + i] * sn[i];
            ds[CPT + i] = dsr[CPT + i] * cs[i] - dsr[i] * sn[i];
          }
        } else {
#pragma unroll
          for (int i = 0; i < CPT2; ++i) {
            dcon[i] = gv[u][i] * s[i];
            ds[i] = dsr[i];
          }
        }
        float dz[CPT2];
#pragma unroll
        for (int i = 0; i < CPT2; ++i) {
          dz[i] = ds[i] * hsig_grad(z[i]);
          db[i] += dz[i];
        }
        if (row_groups) {
          // one token per group: the gradient of hagg is the contribution itself
          const int64_t g = n / p.Lg;
#pragma unroll
          for (int i = 0; i < CPT2; ++i) p.dhagg[(b * p.G + g) * p.P + map.chan(i)] = dcon[i];
        } else {
#pragma unroll
          for (int i = 0; i < CPT2; ++i) dh[i] += dcon[i];
        }
        T* drow = dyb + n * p.dyn;
        float tmp[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) tmp[i] = dz[i];
        VecIO<T, CPT>::store(drow + map.c1, tmp);
        if constexpr (ROPE) {
#pragma unroll
          for (int i = 0; i < CPT; ++i) tmp[i] = dz[CPT + i];
          VecIO<T, CPT>::store(drow + map.c2, tmp);
        }
      }
    }
  }

  const int width = lpr * CPT2;
  const int rslot = wave * rpw + lrow;
  const int64_t slot0 = slab * (int64_t)width;
  const int64_t nslot = p.nvec * CPT2;
  const int64_t prow = b * p.nchunks + chunk;

  // Chunk partials: dhagg (unless per-token groups) then dbias.
  if (!row_groups) {
#pragma unroll
    for (int i = 0; i < CPT2; ++i) red[rslot * width + lcol * CPT2 + i] = dh[i];
    __syncthreads();
    for (int col = tid; col < width; col += kThreads) {
      float t = 0.0f;
      for (int q = 0; q < rs; ++q) t += red[q * width + col];
      if (slot0 + col < nslot) p.part_h[prow * p.P + slot0 + col] = t;
    }
    __syncthreads();
  }
  if (p.dbias) {
#pragma unroll
    for (int i = 0; i < CPT2; ++i) red[rslot * width + lcol * CPT2 + i] = db[i];
    __syncthreads();
    for (int col = tid; col < width; col += kThreads) {
      float t = 0.0f;
      for (int q = 0; q < rs; ++q) t += red[q * width + col];
      if (slot0 + col < nslot) p.part_b[prow * p.P + slot0 + col] = t;
    }
  }

  // dhagg: last chunk of the group sums the group's chunks.
  if (!row_groups) {
    const int64_t g = g0;
    if (elect_last(p.cnt_h + (b * p.G + g) * p.nslabs + slab, (int)p.cpg, &flag)) {
      for (int col = tid; col < width; col += kThreads) {
        const int64_t s = slot0 + col;
        if (s >= nslot) continue;
        float t = 0.0f;
        for (int64_t k = 0; k < p.cpg; ++k) t += p.part_h[(b * p.nchunks + g * p.cpg + k) * p.P + s];
        p.dhagg[(b * p.G + g) * p.P + slot_chan<CPT, MODE>(s, p.P)] = t;
      }
    }
  }
  if (!p.dbias) return;
  // dbias: per (batch row, slab) over chunks, then per slab over the batch.
  if (!elect_last(p.cnt_b1 + b * p.nslabs + slab, (int)p.nchunks, &flag)) return;
  for (int col = tid; col < width; col += kThreads) {
    const int64_t s = slot0 + col;
    if (s >= nslot) continue;
    float t = 0.0f;
    for (int64_t k = 0; k < p.nchunks; ++k) t += p.part_b[(b * p.nchunks + k) * p.P + s];
    p.part_bb[b * p.P + s] = t;
  }
  if (!elect_last(p.cnt_b2 + slab, (int)p.B, &flag)) return;
  for (int col = tid; col < width; col += kThreads) {
    const int64_t s = slot0 + col;
    if (s >= nslot) continue;
    float t = 0.0f;
    for (int64_t bb = 0; bb < p.B; ++bb) t += p.part_bb[bb * p.P + s];
    p.dbias[slot_chan<CPT, MODE>(s, p.P)] = t;
  }
}

template <typename T, int CPT>
static hipError_t launch_gate_cpt(const GateParams& p, bool bwd, hipStream_t st) {
  const dim3 grid((unsigned)(p.B * p.nchunks * p.nslabs)), block(kThreads);
  switch (p.mode) {
#define POM_CASE(M)                                                                  \
  case M:                                                                            \
    if (bwd) hipLaunchKernelGGL((gate_bwd_kernel<T, CPT, M>), grid, block, 0, st, p); \
    else hipLaunchKernelGGL((gate_fwd_kernel<T, CPT, M>), grid, block, 0, st, p);     \
    break;
    POM_CASE(MODE_PLAIN)
    POM_CASE(MODE_ROPE1D)
    POM_CASE(MODE_ROPE2D)
#undef POM_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_gate_t(const GateParams& p, bool bwd, hipStream_t st) {
  switch (p.cpt) {
    case 8: if constexpr (sizeof(T) == 2) return launch_gate_cpt<T, 8>(p, bwd, st); else break;
    case 4: return launch_gate_cpt<T, 4>(p, bwd, st);
    case 2: return launch_gate_cpt<T, 2>(p, bwd, st);
    case 1: return launch_gate_cpt<T, 1>(p, bwd, st);
    default: break;
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gate(const GateParams& p, bool bwd, hipStream_t st) {
  switch (p.dtype) {
    case DT_F32: return launch_gate_t<float>(p, bwd, st);
    case DT_BF16: return launch_gate_t<__hip_bfloat16>(p, bwd, st);
    case DT_F16: return launch_gate_t<__half>(p, bwd, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pom
