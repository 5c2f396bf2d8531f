// Pieces shared by the matrix-core attention passes over int8 jpeg archives
// (fc_attn_mfma.hip: decode, one query token per sequence; fc_prefill.hip:
// causal prefill, many query tokens).
#pragma once

#include <hip/hip_runtime.h>

namespace fc {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kPassRowsW = 64;         // max rows per wavefront pass
constexpr int kSPad = kPassRowsW + 4;  // float stride of a score row in LDS
constexpr int kWPad = kPassRowsW + 8;  // half stride of a weight row in LDS
constexpr float kLazyMax = 8.f;        // exponentials may reach 2^8 before a rescale
// fp32-weight split w = hi + lo / kLoScale into two f16 operands: |w| stays
// below 2^13 (16 taps of 2^8 times a V headroom of 2), so |lo| <= 2 |w| fits
constexpr float kLoScale = 4096.f;
constexpr int kTapsUnrolled = 16;      // softmax taps unrolled (block sizes up to 16)
constexpr int kCachePolicyNt = 2;      // buffer load cache policy: nontemporal (streaming)

// Orders this wavefront's LDS writes before its later LDS reads (lanes of a
// wavefront exchange data through its private LDS region).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// exponent e with x * 2^-e in [2^(target-1), 2^target) for x > 0; 0 for x == 0
__device__ __forceinline__ int pow2_exp_for(float x, int target) {
  if (!(x > 0.f)) return 0;
  int e;
  frexpf(x, &e);
  return e - target;
}

}  // namespace fc
