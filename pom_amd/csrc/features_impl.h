// Per-token polynomial features for gfx950: the operand of the dense-mask
// route (full_mask_mixer, pom/pom.py:41-45), whose mixing is a batched GEMM.
//
// Forward (pom/pom.py:83-88):  p[b,n,c] = sum_{j<K} coeff[c,j] act(x[b,n,c])^(j+1)
// Backward, for an upstream gradient dp (B, N, P):
//   dx[b,n,c]    = dp * p'(h) * act'(x)
//   dcoeff[c, j] = sum_{b,n} dp * h^(j+1)     (chunk partials + fixed-order finalize)
// One thread per V-element channel chunk walks the rows of one token chunk
// (a wave reads 64 consecutive chunks of a row: contiguous segments).
#pragma once

#include "agg_impl.h"

namespace pom {

template <typename T, int V, int KM>
__global__ void __launch_bounds__(kThreads) features_fwd_kernel(const FeatParams p) {
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= p.P / V) return;   // no barriers below
  const int64_t chunk = blockIdx.y, b = blockIdx.z;
  const int64_t rbeg = chunk * p.RC, rend = rbeg + p.RC < p.N ? rbeg + p.RC : p.N;
  const int64_t c0 = j * V;
  float c[V][KM];
  {
    float flat[V * KM];
    param_gather<V * KM>(p.coeff, [&](int q) {
      const int k = q % KM;
      return (c0 + q / KM) * p.K + (k < p.K ? k : p.K - 1);
    }, flat);
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
      for (int k = 0; k < KM; ++k) c[v][k] = k < p.K ? flat[v * KM + k] : 0.0f;
  }
  const T* xb = reinterpret_cast<const T*>(p.x) + b * p.sxb + c0;
  T* ob = reinterpret_cast<T*>(p.out) + b * p.sob + c0;
  for (int64_t n = rbeg; n < rend; ++n) {
    float xv[V], o[V];
    VecIO<T, V>::load(xb + n * p.sxn, xv);
#pragma unroll
    for (int v = 0; v < V; ++v) o[v] = poly<KM>(act(xv[v]), c[v]);
    VecIO<T, V>::store(ob + n * p.son, o);
  }
}

template <typename T, int V, int KM>
__global__ void __launch_bounds__(kThreads) features_bwd_kernel(const FeatParams p) {
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= p.P / V) return;   // no barriers below
  const int64_t chunk = blockIdx.y, b = blockIdx.z;
  const int64_t rbeg = chunk * p.RC, rend = rbeg + p.RC < p.N ? rbeg + p.RC : p.N;
  const int64_t c0 = j * V;
  float d[V][KM], g[V][KM];
  {
    float flat[V * KM];
    param_gather<V * KM>(p.coeff, [&](int q) {
      const int k = q % KM;
      return (c0 + q / KM) * p.K + (k < p.K ? k : p.K - 1);
    }, flat);
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        d[v][k] = k < p.K ? flat[v * KM + k] * (float)(k + 1) : 0.0f;
        g[v][k] = 0.0f;
      }
  }
  const T* xb = reinterpret_cast<const T*>(p.x) + b * p.sxb + c0;
  const T* gb = reinterpret_cast<const T*>(p.go) + b * p.sgob + c0;
  T* dxb = reinterpret_cast<T*>(p.gx) + b * p.sgxb + c0;
  for (int64_t n = rbeg; n < rend; ++n) {
    float xv[V], gv[V], dx[V];
    VecIO<T, V>::load(xb + n * p.sxn, xv);
    VecIO<T, V>::load(gb + n * p.sgon, gv);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float l = leaky(xv[v]), h = clamp_act(l);
      dx[v] = weighted_act_grad(xv[v], l, h, gv[v], 0.01f * gv[v]) * poly_d<KM>(h, d[v]);
      pow_acc<KM>(h, gv[v], g[v]);
    }
    VecIO<T, V>::store(dxb + n * p.sgxn, dx);
  }
  // chunk partial, laid out as the aggregation's: part[((b * nch + chunk) * K + k) * P + c]
  float* part = p.part + (b * p.nch + chunk) * p.K * p.P + c0;
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    if (k >= p.K) break;
#pragma unroll
    for (int v = 0; v < V; ++v) part[k * p.P + v] = g[v][k];
  }
}

template <typename T, int V>
hipError_t features_v(const FeatParams& p, bool bwd, hipStream_t st) {
  const dim3 grid((unsigned)((p.P / V + kThreads - 1) / kThreads), (unsigned)p.nch, (unsigned)p.B), block(kThreads);
  POM_K_SWITCH(p.K, {
    if (bwd) hipLaunchKernelGGL((features_bwd_kernel<T, V, KM>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((features_fwd_kernel<T, V, KM>), grid, block, 0, st, p);
    return hipGetLastError();
  })
}

template <typename T>
hipError_t features_fwd_t(const FeatParams& p, hipStream_t st) {
  switch (p.V) {
    case 8: if constexpr (sizeof(T) == 2) return features_v<T, 8>(p, false, st); else break;
    case 4: return features_v<T, 4>(p, false, st);
    case 2: return features_v<T, 2>(p, false, st);
    case 1: return features_v<T, 1>(p, false, st);
    default: break;
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t features_bwd_t(const FeatParams& p, hipStream_t st) {
  hipError_t e = hipErrorInvalidValue;
  switch (p.V) {
    case 8: if constexpr (sizeof(T) == 2) e = features_v<T, 8>(p, true, st); break;
    case 4: e = features_v<T, 4>(p, true, st); break;
    case 2: e = features_v<T, 2>(p, true, st); break;
    case 1: e = features_v<T, 1>(p, true, st); break;
    default: break;
  }
  if (e != hipSuccess) return e;
  return launch_coeff_grad_finalize(p.part, p.B * p.nch, p.P, p.K, p.gc, st);
}

}  // namespace pom
