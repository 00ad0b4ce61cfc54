// Shared device helpers for the PoM HIP kernels (gfx950 / CDNA4).
//
// Element types: float, __hip_bfloat16, __half.  All arithmetic is fp32;
// loads widen to fp32, stores round to nearest-even.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace pom {

constexpr int kWave = 64;          // CDNA wavefront width
constexpr int kWaves = 4;          // waves per workgroup in the streaming kernels
constexpr int kThreads = kWave * kWaves;
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
__device__ __forceinline__ float leaky(float x) { return x > 0.0f ? x : x * 0.01f; }

__device__ __forceinline__ float act(float x) {
  return fminf(fmaxf(leaky(x), -0.1f), 6.0f);
}

__device__ __forceinline__ float act_grad(float x) {
  const float l = leaky(x);
  const float slope = x > 0.0f ? 1.0f : 0.01f;
  return (l >= -0.1f && l <= 6.0f) ? slope : 0.0f;
}

// p(h) = sum_{j<K} c[j] h^(j+1), with powers built by repeated products.
template <int K>
__device__ __forceinline__ float poly(float h, const float (&c)[K]) {
  float hp = h, acc = c[0] * h;
#pragma unroll
  for (int j = 1; j < K; ++j) {
    hp *= h;
    acc += c[j] * hp;
  }
  return acc;
}

// Backward of p at h: returns p'(h) and accumulates w * h^(j+1) into g[j].
template <int K>
__device__ __forceinline__ float poly_grad_acc(float h, float w, const float (&c)[K], float (&g)[K]) {
  float hp = 1.0f, dp = 0.0f;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const float hph = hp * h;
    dp += c[j] * (float)(j + 1) * hp;
    g[j] += w * hph;
    hp = hph;
  }
  return dp;
}

// Hardsigmoid relu6(z + 3) / 6 and its derivative (torch: 1/6 on (-3, 3)).
__device__ __forceinline__ float hsig(float z) {
  return fminf(fmaxf(z + 3.0f, 0.0f), 6.0f) / 6.0f;
}
__device__ __forceinline__ float hsig_grad(float z) {
  return (z > -3.0f && z < 3.0f) ? (1.0f / 6.0f) : 0.0f;
}

// ---------------------------------------------------------------------------
// Device-scope "last workgroup done" election.
//
// Every workgroup of a group publishes its partial results, then calls
// elect_last(); exactly one workgroup (the last to arrive) gets true and may
// read all partials of the group.  The counter is reset by the winner so the
// workspace is reusable by the next launch on the stream without a memset.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool elect_last(int* counter, int expected, int* lds_flag) {
  __threadfence();   // every thread releases its own partial stores at agent scope
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = (prev == expected - 1);
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = last ? 1 : 0;
  }
  __syncthreads();
  const bool last = *lds_flag != 0;
  if (last) __threadfence();  // acquire: partials of the other workgroups are visible
  return last;
}

}  // namespace pom
