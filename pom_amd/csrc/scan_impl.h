// Token-causal aggregation (prefix mean per token) as a chunked scan, forward
// and backward — replaces pom/pom_triton_causal.py:68-344 and the causal
// RoPE kernels pom/pom_triton_rope.py:483-873 (whose single program walks all
// N tokens serially).
//
// Forward, out[n] = (1/(n+1)) * sum_{m <= n} R_m p(act(x_m)):
//   1. chunk sums of the (rotated) features: the aggregation chunk kernel
//      with one frame and chunks of RC rows, partials only;
//   2. exclusive prefix of the chunk sums along the sequence (one thread per
//      (batch row, channel), fixed order);
//   3. every chunk re-reads its rows and runs the running sum from its
//      prefix: one lane per vector column walks the chunk's rows in order.
// Backward, with sw[m] = sum_{n >= m} go[n] / (n+1):
//   1. chunk sums of go[n] / (n+1);  2. exclusive suffix over chunks;
//   3. every chunk walks its rows backwards: d(R_m p_m) = sw[m],
//      grad_x = (R_m^T sw[m]) p'(h) act'(x), grad_coeff partial per lane.
// All sums in fp32, fixed order: deterministic.
#pragma once

#include "agg_impl.h"

namespace pom {

// Exclusive prefix (forward) or suffix (backward) over the chunk axis, in place.
static __global__ void __launch_bounds__(kThreads) chunk_exclusive_scan(float* __restrict__ cs, int64_t B, int64_t nch,
                                                                 int64_t P, int reverse) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= B * P) return;
  const int64_t b = idx / P, c = idx - b * P;
  float* base = cs + b * nch * P + c;
  // eight chunks loaded before any is rewritten (in place: the loads would
  // otherwise each wait for the previous store), then scanned in order
  constexpr int KB = 8;
  float run = 0.0f;
  for (int64_t j0 = 0; j0 < nch; j0 += KB) {
    float v[KB];
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      const int64_t k = reverse ? nch - 1 - (j0 + q) : j0 + q;
      v[q] = j0 + q < nch ? base[k * P] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      if (j0 + q >= nch) break;
      const int64_t k = reverse ? nch - 1 - (j0 + q) : j0 + q;
      base[k * P] = run;
      run += v[q];
    }
  }
}

// SUMS: the first pass, which only sums each chunk's (rotated) features into
// csum, in the same thread layout as the scan itself.
template <typename T, int CPT, int KM, int MODE, bool SUMS>
__global__ void __launch_bounds__(kThreads) scan_fwd_kernel(const ScanParams p) {
  using Map = LaneMap<CPT, MODE>;
  constexpr int CPT2 = Map::CPT2;
  constexpr bool ROPE = Mode_<MODE>::rope;
  constexpr int U = 4;
  const int64_t vcol = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (vcol >= p.nvec) return;   // no cross-lane work in this kernel
  const int64_t chunk = blockIdx.y, b = blockIdx.z;
  Map map;
  map.init(vcol, p.P);

  float c[CPT2][KM], acc[CPT2];
  const float* pre = p.csum + (b * p.nch + chunk) * p.P;
  {
    float flat[CPT2 * KM];
    param_gather<CPT2 * KM>(p.coeff, [&](int q) {
      const int j = q % KM;
      return map.chan(q / KM) * p.K + (j < p.K ? j : p.K - 1);
    }, flat);
#pragma unroll
    for (int i = 0; i < CPT2; ++i) {
#pragma unroll
      for (int j = 0; j < KM; ++j) c[i][j] = j < p.K ? flat[i * KM + j] : 0.0f;
      acc[i] = SUMS ? 0.0f : pre[map.chan(i)];
    }
  }
  const int64_t rbeg = chunk * p.RC;
  const int64_t rend = rbeg + p.RC < p.N ? rbeg + p.RC : p.N;
  const T* xb = reinterpret_cast<const T*>(p.x) + b * p.sxb;
  T* ob = reinterpret_cast<T*>(p.out) + b * p.N * p.P;
  for (int64_t r = rbeg; r < rend; r += U) {
    Pack<T, CPT> v1[U], v2[ROPE ? U : 1];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (r + u < rend) {
        const T* row = xb + (r + u) * p.sxn;
        v1[u].load_stream(row + map.c1);
        if constexpr (ROPE) v2[u].load_stream(row + map.c2);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t n = r + u;
      if (n >= rend) break;
      const float cnt = (float)(n + 1);
      float o1[CPT], o2[CPT];
      if constexpr (ROPE) {
        float cs[CPT], sn[CPT];
        load_table<CPT>(p.rope, map.table, n, map.tcol, cs, sn);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const float p1 = poly<KM>(act(v1[u].get(i)), c[i]);
          const float p2 = poly<KM>(act(v2[u].get(i)), c[CPT + i]);
          acc[i] += p1 * cs[i] - p2 * sn[i];
          acc[CPT + i] += p2 * cs[i] + p1 * sn[i];
          o1[i] = acc[i] / cnt;
          o2[i] = acc[CPT + i] / cnt;
        }
        if constexpr (!SUMS) {
          VecIO<T, CPT>::store(ob + n * p.P + map.c1, o1);
          VecIO<T, CPT>::store(ob + n * p.P + map.c2, o2);
        }
      } else {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          acc[i] += poly<KM>(act(v1[u].get(i)), c[i]);
          o1[i] = acc[i] / cnt;
        }
        if constexpr (!SUMS) VecIO<T, CPT>::store(ob + n * p.P + map.c1, o1);
      }
    }
  }
  if constexpr (SUMS) {
    float* cs = p.csum + (b * p.nch + chunk) * p.P;
#pragma unroll
    for (int i = 0; i < CPT2; ++i) cs[map.chan(i)] = acc[i];
  }
}

// Backward step 1: chunk sums of go[n] / (n+1) (plain channel columns).
template <int V>
__global__ void __launch_bounds__(kThreads) scan_go_chunk_sums(const ScanParams p) {
  const int64_t vcol = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (vcol * V >= p.P) return;
  const int64_t chunk = blockIdx.y, b = blockIdx.z;
  const int64_t rbeg = chunk * p.RC;
  const int64_t rend = rbeg + p.RC < p.N ? rbeg + p.RC : p.N;
  const float* gb = p.go + b * p.N * p.P + vcol * V;
  float s[V];
#pragma unroll
  for (int i = 0; i < V; ++i) s[i] = 0.0f;
  for (int64_t n = rbeg; n < rend; ++n) {
    float v[V];
    load_f32<V>(gb + n * p.P, v);
    const float cnt = (float)(n + 1);
#pragma unroll
    for (int i = 0; i < V; ++i) s[i] += v[i] / cnt;
  }
  store_f32<V>(p.csum + (b * p.nch + chunk) * p.P + vcol * V, s);
}

template <typename T, int CPT, int KM, int MODE>
__global__ void __launch_bounds__(kThreads) scan_bwd_kernel(const ScanParams p) {
  using Map = LaneMap<CPT, MODE>;
  constexpr int CPT2 = Map::CPT2;
  constexpr bool ROPE = Mode_<MODE>::rope;
  constexpr int U = 4;
  const int64_t vcol = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (vcol >= p.nvec) return;
  const int64_t chunk = blockIdx.y, b = blockIdx.z;
  Map map;
  map.init(vcol, p.P);

  float c[CPT2][KM], g[CPT2][KM], sw[CPT2];
  const float* suf = p.csum + (b * p.nch + chunk) * p.P;
  {
    float flat[CPT2 * KM];
    param_gather<CPT2 * KM>(p.coeff, [&](int q) {
      const int j = q % KM;
      return map.chan(q / KM) * p.K + (j < p.K ? j : p.K - 1);
    }, flat);
#pragma unroll
    for (int i = 0; i < CPT2; ++i) {
#pragma unroll
      for (int j = 0; j < KM; ++j) {
        c[i][j] = j < p.K ? flat[i * KM + j] : 0.0f;
        g[i][j] = 0.0f;
      }
      sw[i] = suf[map.chan(i)];
    }
  }
  const int64_t rbeg = chunk * p.RC;
  const int64_t rend = rbeg + p.RC < p.N ? rbeg + p.RC : p.N;
  const T* xb = reinterpret_cast<const T*>(p.x) + b * p.sxb;
  const float* gob = p.go + b * p.N * p.P;
  T* gxb = reinterpret_cast<T*>(p.gx) + b * p.sgb;
  for (int64_t r = rend - 1; r >= rbeg; r -= U) {
    Pack<T, CPT> v1[U], v2[ROPE ? U : 1];
    float g1[U][CPT], g2[ROPE ? U : 1][CPT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t n = r - u;
      if (n >= rbeg) {
        const T* row = xb + n * p.sxn;
        v1[u].load_stream(row + map.c1);
        load_f32<CPT>(gob + n * p.P + map.c1, g1[u]);
        if constexpr (ROPE) {
          v2[u].load_stream(row + map.c2);
          load_f32<CPT>(gob + n * p.P + map.c2, g2[u]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t n = r - u;
      if (n < rbeg) break;
      const float cnt = (float)(n + 1);
      float o1[CPT], o2[CPT];
      if constexpr (ROPE) {
        float cs[CPT], sn[CPT];
        load_table<CPT>(p.rope, map.table, n, map.tcol, cs, sn);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          sw[i] += g1[u][i] / cnt;
          sw[CPT + i] += g2[u][i] / cnt;
          const float w1 = sw[i] * cs[i] + sw[CPT + i] * sn[i];
          const float w2 = sw[CPT + i] * cs[i] - sw[i] * sn[i];
          const float x1 = v1[u].get(i), x2 = v2[u].get(i);
          o1[i] = w1 * poly_grad_acc<KM>(act(x1), w1, c[i], g[i]) * act_grad(x1);
          o2[i] = w2 * poly_grad_acc<KM>(act(x2), w2, c[CPT + i], g[CPT + i]) * act_grad(x2);
        }
        VecIO<T, CPT>::store(gxb + n * p.sgn + map.c1, o1);
        VecIO<T, CPT>::store(gxb + n * p.sgn + map.c2, o2);
      } else {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          sw[i] += g1[u][i] / cnt;
          const float xx = v1[u].get(i);
          o1[i] = sw[i] * poly_grad_acc<KM>(act(xx), sw[i], c[i], g[i]) * act_grad(xx);
        }
        VecIO<T, CPT>::store(gxb + n * p.sgn + map.c1, o1);
      }
    }
  }
  float* part = p.part + (b * p.nch + chunk) * p.K * p.P;
#pragma unroll
  for (int i = 0; i < CPT2; ++i)
#pragma unroll
    for (int j = 0; j < KM; ++j)
      if (j < p.K) part[j * p.P + map.chan(i)] = g[i][j];
}

template <typename T, int CPT, int KM, bool SUMS>
hipError_t scan_fwd_mode(const ScanParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.nvec + kThreads - 1) / kThreads), (unsigned)p.nch, (unsigned)p.B);
  switch (p.mode) {
    case MODE_PLAIN:
      hipLaunchKernelGGL((scan_fwd_kernel<T, CPT, KM, MODE_PLAIN, SUMS>), grid, dim3(kThreads), 0, st, p);
      break;
    case MODE_ROPE1D:
      hipLaunchKernelGGL((scan_fwd_kernel<T, CPT, KM, MODE_ROPE1D, SUMS>), grid, dim3(kThreads), 0, st, p);
      break;
    case MODE_ROPE2D:
      hipLaunchKernelGGL((scan_fwd_kernel<T, CPT, KM, MODE_ROPE2D, SUMS>), grid, dim3(kThreads), 0, st, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int CPT, int KM>
hipError_t scan_bwd_mode(const ScanParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.nvec + kThreads - 1) / kThreads), (unsigned)p.nch, (unsigned)p.B);
  switch (p.mode) {
    case MODE_PLAIN: hipLaunchKernelGGL((scan_bwd_kernel<T, CPT, KM, MODE_PLAIN>), grid, dim3(kThreads), 0, st, p); break;
    case MODE_ROPE1D: hipLaunchKernelGGL((scan_bwd_kernel<T, CPT, KM, MODE_ROPE1D>), grid, dim3(kThreads), 0, st, p); break;
    case MODE_ROPE2D: hipLaunchKernelGGL((scan_bwd_kernel<T, CPT, KM, MODE_ROPE2D>), grid, dim3(kThreads), 0, st, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T, int CPT>
hipError_t scan_sums_cpt(const ScanParams& p, hipStream_t st) {
  POM_K_SWITCH(p.K, return (scan_fwd_mode<T, CPT, KM, true>(p, st)))
}

template <typename T, int CPT>
hipError_t scan_fwd_cpt(const ScanParams& p, hipStream_t st) {
  POM_K_SWITCH(p.K, return (scan_fwd_mode<T, CPT, KM, false>(p, st)))
}

template <typename T, int CPT>
hipError_t scan_bwd_cpt(const ScanParams& p, hipStream_t st) {
  POM_K_SWITCH(p.K, return (scan_bwd_mode<T, CPT, KM>(p, st)))
}

template <typename T>
hipError_t scan_fwd_t(const ScanParams& p, hipStream_t st) {
  {
    auto sums = [&]() -> hipError_t { POM_CPT_SWITCH(T, p.cpt, scan_sums_cpt, p, st) };
    if (hipError_t e = sums()) return e;
  }
  hipLaunchKernelGGL(chunk_exclusive_scan, flat_grid(p.B * p.P), dim3(kThreads), 0, st, p.csum, p.B, p.nch, p.P, 0);
  if (hipError_t e = hipGetLastError()) return e;
  POM_CPT_SWITCH(T, p.cpt, scan_fwd_cpt, p, st)
}

template <typename T>
hipError_t scan_bwd_t(const ScanParams& p, hipStream_t st) {
  // go is fp32 and contiguous: 4 channels per lane when P allows it
  const bool v4 = (p.P % 4) == 0 && (reinterpret_cast<uintptr_t>(p.go) % 16) == 0;
  const int64_t cols = v4 ? p.P / 4 : p.P;
  const dim3 g1((unsigned)((cols + kThreads - 1) / kThreads), (unsigned)p.nch, (unsigned)p.B);
  if (v4) hipLaunchKernelGGL(scan_go_chunk_sums<4>, g1, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL(scan_go_chunk_sums<1>, g1, dim3(kThreads), 0, st, p);
  if (hipError_t e = hipGetLastError()) return e;
  hipLaunchKernelGGL(chunk_exclusive_scan, flat_grid(p.B * p.P), dim3(kThreads), 0, st, p.csum, p.B, p.nch, p.P, 1);
  if (hipError_t e = hipGetLastError()) return e;
  hipError_t e;
  {
    auto run = [&]() -> hipError_t { POM_CPT_SWITCH(T, p.cpt, scan_bwd_cpt, p, st) };
    e = run();
  }
  if (e != hipSuccess) return e;
  return launch_coeff_grad_finalize(p.part, p.B * p.nch, p.P, p.K, p.gc, st);
}

}  // namespace pom
