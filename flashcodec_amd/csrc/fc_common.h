// Shared device helpers for the flashcodec_amd kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flashcodec_amd.h"

namespace fc {

// bf16 storage word. Arithmetic always happens in fp32.
struct bf16_t {
  uint16_t bits;
};
typedef _Float16 f16_t;

template <typename T>
struct dtype_code;
template <>
struct dtype_code<float> {
  static constexpr int value = FC_F32;
};
template <>
struct dtype_code<f16_t> {
  static constexpr int value = FC_F16;
};
template <>
struct dtype_code<bf16_t> {
  static constexpr int value = FC_BF16;
};

// Workgroup barrier ordering LDS accesses only: global loads in flight
// stay in flight, where __syncthreads() first waits for every outstanding
// load (and store).  For barriers that only hand LDS data between threads.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) {
  return __uint_as_float((uint32_t)x.bits << 16);
}
__device__ __forceinline__ float to_f32(int8_t x) { return (float)(int)x; }

// Round-to-nearest-even conversions from fp32 (the rounding torch's CPU
// casts perform; bf16 NaN becomes the canonical 0x7FC0 like c10::BFloat16).
template <typename T>
__device__ __forceinline__ T from_f32(float f);
template <>
__device__ __forceinline__ float from_f32<float>(float f) {
  return f;
}
// The empty asm pins f as an fp32 value: without it the backend may fold
// the fma / multiply that produced f and this conversion into one
// mixed-precision instruction (v_fma_mixlo_f16), which rounds the exact
// result to f16 once instead of fp32-then-f16, and the two differ when the
// fp32 value lands on an f16 halfway point.
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float f) {
  __asm__("" : "+v"(f));
  return (f16_t)f;
}
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16_t{0x7fc0};
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16_t{(uint16_t)(u >> 16)};
}

// Vector of N elements of T moved as one aligned memory operation.
template <typename T, int N>
struct alignas(sizeof(T) * N) vec_t {
  T v[N];
};

template <typename T, int N>
__device__ __forceinline__ void load_f32(const T* __restrict__ p, float (&out)[N]) {
  vec_t<T, N> t = *reinterpret_cast<const vec_t<T, N>*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = to_f32(t.v[i]);
}

template <typename T, int N>
__device__ __forceinline__ void store_from_f32(T* __restrict__ p, const float (&in)[N]) {
  vec_t<T, N> t;
#pragma unroll
  for (int i = 0; i < N; ++i) t.v[i] = from_f32<T>(in[i]);
  *reinterpret_cast<vec_t<T, N>*>(p) = t;
}

// Butterfly reductions over aligned groups of `width` lanes (power of two,
// <= 64) inside a wavefront.
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int m = 1; m < WIDTH; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < WIDTH; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float group_max_rt(float v, int width) {
  for (int m = 1; m < width; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// element `idx` of a float tensor of dtype `dt` (FC_F32 / FC_F16 / FC_BF16)
__device__ __forceinline__ float load_q(const void* q, int dt, int64_t idx) {
  switch (dt) {
    case FC_F16: return to_f32(static_cast<const f16_t*>(q)[idx]);
    case FC_BF16: return to_f32(static_cast<const bf16_t*>(q)[idx]);
    default: return static_cast<const float*>(q)[idx];
  }
}

// store v (round to nearest even) as element `idx` of a tensor of dtype `dt`
__device__ __forceinline__ void store_any(void* p, int dt, int64_t idx, float v) {
  switch (dt) {
    case FC_F16: static_cast<f16_t*>(p)[idx] = from_f32<f16_t>(v); break;
    case FC_BF16: static_cast<bf16_t*>(p)[idx] = from_f32<bf16_t>(v); break;
    default: static_cast<float*>(p)[idx] = v; break;
  }
}

// (used by the archive kernels and by the fused decode step's in-kernel
// archive of a completed block)
// clamp(rint(fl(c / s)), -127, 127) for a quantizer row with scale s and
// rs = fl(1 / s), where fl(c / s) is the IEEE single-precision quotient.
// For |c / s| < 128: x = fl(c * rs) is within |c/s| 2^-23 <= 2^-16 of c / s
// and fl(c / s) within 2^-17 of it, so they round to the same integer unless
// a half-integer lies within 2^-15 of x; only then is the quotient computed
// exactly.  (Scales are fl(amax / 127) rounded to the stream dtype, so
// |c / s| <= 127 (1 + 2^-8) < 128.)
// A NaN quotient gets code 0 (the reference's int8 cast of NaN is
// undefined; 0 is what x86's truncating conversion gives).
__device__ __forceinline__ float quant_code(float c, float s, float rs) {
  const float x = c * rs;
  float q = __builtin_rintf(x);
  if (!(0.5f - fabsf(x - q) > 0x1p-15f)) q = __builtin_rintf(c / s);
  return q == q ? fminf(fmaxf(q, -127.f), 127.f) : 0.f;
}

}  // namespace fc
