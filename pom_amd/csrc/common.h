// Shared device helpers for the PoM HIP kernels (gfx950 / CDNA4).
//
// Element types: float, __hip_bfloat16, __half.  All arithmetic is fp32;
// loads widen to fp32, stores round to nearest-even.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

namespace pom {

constexpr int kWave = 64;          // CDNA wavefront width
constexpr int kWaves = 4;          // waves per workgroup in the streaming kernels
constexpr int kThreads = kWave * kWaves;
constexpr int kMaxLpr = kWave;      // lanes per token row: 2^lpr_log2 <= one wave
constexpr int kMaxK = 16;          // highest polynomial degree supported

// ---------------------------------------------------------------------------
// Scalar conversions
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<__hip_bfloat16>(__hip_bfloat16 v) {
  return __bfloat162float(v);
}
template <> __device__ __forceinline__ float to_f32<__half>(__half v) { return __half2float(v); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float v) {
  return __float2bfloat16(v);
}
template <> __device__ __forceinline__ __half from_f32<__half>(float v) { return __float2half(v); }

// Round an fp32 value to T and back: the value a T tensor would hold.
template <typename T> __device__ __forceinline__ float round_to(float v) {
  return to_f32<T>(from_f32<T>(v));
}

// ---------------------------------------------------------------------------
// Vector loads / stores of V consecutive elements, widened to fp32.
// The caller guarantees alignment of V * sizeof(T) bytes (checked on host).
// ---------------------------------------------------------------------------
template <int BYTES> struct RawVec;
template <> struct RawVec<2> { using type = uint16_t; };
template <> struct RawVec<4> { using type = uint32_t; };
template <> struct RawVec<8> { using type = uint2; };
template <> struct RawVec<16> { using type = uint4; };

template <typename T, int V>
struct VecIO {
  static constexpr int kBytes = V * (int)sizeof(T);
  static constexpr int kChunk = kBytes > 16 ? 16 : kBytes;   // bytes per memory op
  static constexpr int kOps = kBytes / kChunk;
  static constexpr int kPer = kChunk / (int)sizeof(T);       // elements per memory op
  using Raw = typename RawVec<kChunk>::type;

  __device__ __forceinline__ static void load(const T* __restrict__ p, float (&o)[V]) {
#pragma unroll
    for (int op = 0; op < kOps; ++op) {
      Raw r = *reinterpret_cast<const Raw*>(p + op * kPer);
      const T* e = reinterpret_cast<const T*>(&r);
#pragma unroll
      for (int i = 0; i < kPer; ++i) o[op * kPer + i] = to_f32<T>(e[i]);
    }
  }
  __device__ __forceinline__ static void store(T* __restrict__ p, const float (&v)[V]) {
#pragma unroll
    for (int op = 0; op < kOps; ++op) {
      Raw r;
      T* e = reinterpret_cast<T*>(&r);
#pragma unroll
      for (int i = 0; i < kPer; ++i) e[i] = from_f32<T>(v[op * kPer + i]);
      *reinterpret_cast<Raw*>(p + op * kPer) = r;
    }
  }
};

template <int V>
__device__ __forceinline__ void load_f32(const float* __restrict__ p, float (&o)[V]) {
  VecIO<float, V>::load(p, o);
}
template <int V>
__device__ __forceinline__ void store_f32(float* __restrict__ p, const float (&v)[V]) {
  VecIO<float, V>::store(p, v);
}

// ---------------------------------------------------------------------------
// PoM activation and its derivative, with torch autograd's conventions:
//   act(x)  = clamp(leaky_relu(x, 0.01), -0.1, 6)
//   act'(x) = (x > 0 ? 1 : 0.01) * [-0.1 <= leaky(x) <= 6]
// leaky_relu's backward uses x > 0, clamp's backward keeps both bounds.
// ---------------------------------------------------------------------------
// leaky_relu(x, 0.01) == max(x, 0.01 x) for every x (slope below 1).
__device__ __forceinline__ float leaky(float x) { return fmaxf(x, 0.01f * x); }

// clamp(l, -0.1, 6) as one median-of-three.
__device__ __forceinline__ float clamp_act(float l) { return __builtin_amdgcn_fmed3f(l, -0.1f, 6.0f); }

__device__ __forceinline__ float act(float x) { return clamp_act(leaky(x)); }

__device__ __forceinline__ float act_grad(float x) {
  const float l = leaky(x);
  const float slope = x > 0.0f ? 1.0f : 0.01f;
  return (clamp_act(l) == l) ? slope : 0.0f;
}

// w * act'(x) given l = leaky(x), h = clamp_act(l), w1 = w and w01 = 0.01 w:
// leaky_relu's backward picks the slope by x > 0 and clamp's backward passes
// the gradient where l lies inside [-0.1, 6] (h == l).
__device__ __forceinline__ float weighted_act_grad(float x, float l, float h, float w1, float w01) {
  const float s = x > 0.0f ? w1 : w01;
  return h == l ? s : 0.0f;
}

// p(h) / h = c0 + h (c1 + h (c2 + ...)) in Horner form, so p(h) = h * poly_q(h).
template <int K>
__device__ __forceinline__ float poly_q(float h, const float (&c)[K]) {
  float t = c[K - 1];
#pragma unroll
  for (int j = K - 2; j >= 0; --j) t = fmaf(t, h, c[j]);
  return t;
}

// p(h) = sum_{j<K} c[j] h^(j+1).
template <int K>
__device__ __forceinline__ float poly(float h, const float (&c)[K]) {
  return poly_q<K>(h, c) * h;
}

// p'(h) = sum_j d[j] h^j with d[j] = (j+1) c[j] precomputed.
template <int K>
__device__ __forceinline__ float poly_d(float h, const float (&d)[K]) {
  return poly_q<K>(h, d);
}

// g[j] += w h^(j+1) for j < K (the last term as one fma).
template <int K>
__device__ __forceinline__ void pow_acc(float h, float w, float (&g)[K]) {
  float t = w;   // w h^j
#pragma unroll
  for (int j = 0; j < K; ++j) {
    if (j + 1 == K) {
      g[j] = fmaf(t, h, g[j]);
    } else {
      t *= h;
      g[j] += t;
    }
  }
}

// g[j] += h^(j+1) for j < K (unweighted power sums).
template <int K>
__device__ __forceinline__ void pow_sum(float h, float (&g)[K]) {
  float t = h;   // h^(j+1)
#pragma unroll
  for (int j = 0; j < K; ++j) {
    if (j + 1 == K) {
      g[j] += t;
    } else if (j + 2 == K) {
      g[j] += t;
      g[j + 1] = fmaf(t, h, g[j + 1]);
      break;
    } else {
      g[j] += t;
      t *= h;
    }
  }
}

// Backward of p at h: returns p'(h) and accumulates w * h^(j+1) into g[j].
template <int K>
__device__ __forceinline__ float poly_grad_acc(float h, float w, const float (&c)[K], float (&g)[K]) {
  float d[K];
#pragma unroll
  for (int j = 0; j < K; ++j) d[j] = c[j] * (float)(j + 1);
  pow_acc<K>(h, w, g);
  return poly_d<K>(h, d);
}

// Hardsigmoid relu6(z + 3) / 6 and its derivative (torch: 1/6 on (-3, 3)).
// The division by 6 is a product with RN(1/6) plus one fma correction
// (q = x r, e = x - 6 q exactly, q' = q + e r), three instructions where an
// IEEE division expands to about ten.  q' equals RN(x / 6) for every x in
// [2^-122, 6] (checked exhaustively over all fp32 values) and for x = 0; the
// argument relu6(z + 3) never lies strictly between: z + 3 is 0 or at least
// ulp(3) / 2 = 2^-23 in magnitude (Sterbenz), so hsig matches torch's
// relu6(z + 3) / 6 bit for bit.
__device__ __forceinline__ float hsig(float z) {
  const float x = fminf(fmaxf(z + 3.0f, 0.0f), 6.0f);
  constexpr float r = 1.0f / 6.0f;
  const float q = x * r;
  return __builtin_fmaf(__builtin_fmaf(-q, 6.0f, x), r, q);
}
__device__ __forceinline__ float hsig_grad(float z) {
  return (z > -3.0f && z < 3.0f) ? (1.0f / 6.0f) : 0.0f;
}

// ---------------------------------------------------------------------------
// Raw vector of V elements of T held in registers as loaded (16-byte or
// narrower memory operations), widened to fp32 one element at a time.
// ---------------------------------------------------------------------------
// Loads of data read once per launch (token rows) carry the non-temporal
// hint: the line is not kept in the caches at the expense of others, so a
// stream does not evict (and force the write-back of) the dirty lines the
// previous kernel left behind.  Set POM_STREAM_NT=0 to compile plain loads.
#ifndef POM_STREAM_NT
#define POM_STREAM_NT 1
#endif
template <typename R>
__device__ __forceinline__ R load_stream_raw(const R* __restrict__ p) {
#if POM_STREAM_NT
  if constexpr (sizeof(R) == 16) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    R r;
    __builtin_memcpy(&r, &v, 16);
    return r;
  } else if constexpr (sizeof(R) == 8) {
    typedef unsigned int v2u __attribute__((ext_vector_type(2)));
    const v2u v = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(p));
    R r;
    __builtin_memcpy(&r, &v, 8);
    return r;
  } else {
    return __builtin_nontemporal_load(p);
  }
#else
  return *p;
#endif
}

template <typename T, int V>
struct Pack {
  using IO = VecIO<T, V>;
  typename IO::Raw r[IO::kOps];

  __device__ __forceinline__ void load(const T* __restrict__ p) {
#pragma unroll
    for (int op = 0; op < IO::kOps; ++op) r[op] = *reinterpret_cast<const typename IO::Raw*>(p + op * IO::kPer);
  }
  // the same for data read once (see load_stream_raw)
  __device__ __forceinline__ void load_stream(const T* __restrict__ p) {
#pragma unroll
    for (int op = 0; op < IO::kOps; ++op)
      r[op] = load_stream_raw(reinterpret_cast<const typename IO::Raw*>(p + op * IO::kPer));
  }
  __device__ __forceinline__ float get(int i) const {
    return to_f32<T>(reinterpret_cast<const T*>(r)[i]);
  }
};

// ---------------------------------------------------------------------------
// Cross-lane sums inside one 64-lane wavefront: lanes whose ids differ only in
// bits >= lo_bits (the lanes that share a column) are added, fixed order.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float xor_sum_rows(float v, int lo_bits) {
  for (int off = 1 << lo_bits; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// ---------------------------------------------------------------------------
// The running-mean step of PoM.state_forward (pom/pom.py:255-259) as the
// reference evaluates it on the GPU in the element type T:
//   a = T(n * h)              (scalar multiply in fp32, rounded)
//   c = T(a + m)              (the n_current = 1 term is m itself)
//   h = T(c * fp32(1/(n+1)))  (division by a scalar is a multiply by its
//                              fp32 reciprocal in torch's GPU kernels)
// Contraction is off in this function: an fma of n * h + m would round once
// where the reference rounds twice.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float running_mean_step(float h, float m, float n) {
#pragma clang fp contract(off)
  const float a = round_to<T>(n * h);
  const float c = round_to<T>(a + m);
  const float inv = 1.0f / (n + 1.0f);   // correctly rounded (no fast-math)
  return round_to<T>(c * inv);
}

}  // namespace pom
