// Block-archive and reconstruction kernels of the KV codec (gfx950).
//
// Work decomposition shared by every kernel here: one "item" is one block
// of r tokens of one (batch, head) sequence.  An item is handled by LPI
// consecutive lanes of a wavefront (LPI = power of two <= 64); lane i of the
// item owns features [i*VEC, i*VEC + VEC) and walks the r tokens of the
// block, so the token-axis transform (DCT, deltas, running sums) is
// lane-local and every global access is a coalesced VEC-wide vector of a
// token row.  Per-row reductions over the feature axis (int8 absmax) are
// butterfly shuffles inside the item's lane group.
//
// Bit-exactness against the reference's CPU arithmetic:
//   * DCT encode: coefficient = fma chain over the r taps starting from 0,
//     rounded once to the stream dtype (the CPU GEMM's accumulation order).
//   * DCT decode: same chain over the k coefficients.
//   * int8: scale = dtype(absmax / 127) in fp32, 1 when not > 0, codes =
//     round-half-even(c / scale) clamped to [-127, 127] (0 for a NaN quotient).
//   * png cumsum: fp64 running sum rounded to fp32 per step (CPU cumsum
//     accumulates float in double), anchor + sum in fp32, then the anchor
//     dtype.
// The file is compiled with -ffp-contract=off so no other multiply-add is
// fused behind our back.
#include <initializer_list>
#include <type_traits>
#include <utility>

#include "fc_common.h"
#include "fc_topm.h"

namespace fc {

constexpr int kThreads = 256;

struct ItemMap {
  int64_t item;
  int lane;  // lane index inside the item group
};

// lpi_log2: log2 of the lanes per item.
__device__ __forceinline__ ItemMap item_of_thread(int lpi_log2) {
  ItemMap m;
  m.item = (int64_t)blockIdx.x * (kThreads >> lpi_log2) + (threadIdx.x >> lpi_log2);
  m.lane = threadIdx.x & ((1 << lpi_log2) - 1);
  return m;
}


// ---------------------------------------------------------------- jpeg encode

template <typename T, int VEC, int RMAX, bool QUANT, bool GATED = false>
__global__ __launch_bounds__(kThreads) void jpeg_encode_kernel(
    const T* __restrict__ x, int64_t sb, int64_t sh, int64_t ss, int64_t H, int64_t m,
    int64_t D, int64_t s_valid, int r, int k, const float* __restrict__ basis,
    void* __restrict__ out, float* __restrict__ scales, int64_t cap, int64_t n0,
    int64_t items, int lpi_log2, const int64_t* __restrict__ gate = nullptr, int group = 0) {
  if constexpr (GATED) {
    // gate = device (n_blocks, n_tail) of a decode step: the block is
    // archived only when the tail completes it, at block n_blocks
    if (gate[1] != r - 1) return;
    n0 = gate[0];
    if (n0 < 0 || n0 + m > cap) return;
  }
  const ItemMap im = item_of_thread(lpi_log2);
  // Dead lanes still take part in the group shuffles below; they work on
  // item 0 and store nothing.
  const bool live = im.item < items;
  const int64_t item = live ? im.item : 0;
  const int64_t bh = item / m, blk = item - bh * m;
  const int64_t b = bh / H, h = bh - b * H;
  const int64_t d0 = (int64_t)im.lane * VEC;
  const bool active = live && d0 < D;
  const T* src = x + b * sb + h * sh + (active ? d0 : 0);
  const int64_t tok0 = blk * r;

  float xr[RMAX > 0 ? RMAX : 1][VEC];
  if constexpr (RMAX > 0) {
#pragma unroll
    for (int t = 0; t < RMAX; ++t) {
      if (t < r && active && tok0 + t < s_valid) {
        load_f32<T, VEC>(src + (tok0 + t) * ss, xr[t]);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) xr[t][v] = 0.f;
      }
    }
  }

  const int64_t out_row0 = (bh * cap + n0 + blk) * k;
  for (int j = 0; j < k; ++j) {
    const float* mj = basis + (int64_t)j * r;
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
    if constexpr (RMAX > 0) {
#pragma unroll
      for (int t = 0; t < RMAX; ++t) {
        if (t < r) {
          const float w = mj[t];
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[v] = __builtin_fmaf(xr[t][v], w, acc[v]);
        }
      }
    } else {
      for (int t = 0; t < r; ++t) {
        float xv[VEC];
        if (active && tok0 + t < s_valid) {
          load_f32<T, VEC>(src + (tok0 + t) * ss, xv);
        } else {
#pragma unroll
          for (int v = 0; v < VEC; ++v) xv[v] = 0.f;
        }
        const float w = mj[t];
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = __builtin_fmaf(xv[v], w, acc[v]);
      }
    }
    // round once to the stream dtype (dct_compress returns x.dtype)
    float c[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) c[v] = to_f32(from_f32<T>(acc[v]));

    if constexpr (!QUANT) {
      if (active) store_from_f32<T, VEC>(static_cast<T*>(out) + (out_row0 + j) * D + d0, c);
    } else {
      // one scale per row, or per `group` features of the row (the lanes
      // of a group are aligned runs of group / VEC lanes)
      const int glanes = group ? group / VEC : 1 << lpi_log2;
      float amax = 0.f;
#pragma unroll
      for (int v = 0; v < VEC; ++v) amax = fmaxf(amax, fabsf(c[v]));
      amax = group_max_rt(amax, glanes);
      float s = to_f32(from_f32<T>(amax / 127.0f));
      if (!(s > 0.f)) s = 1.0f;
      const float rs = 1.0f / s;
      if (active) {
        vec_t<int8_t, VEC> qv;
#pragma unroll
        for (int v = 0; v < VEC; ++v) qv.v[v] = (int8_t)(int)quant_code(c[v], s, rs);
        *reinterpret_cast<vec_t<int8_t, VEC>*>(static_cast<int8_t*>(out) + (out_row0 + j) * D +
                                               d0) = qv;
        if ((im.lane & (glanes - 1)) == 0) {
          if (group)
            scales[(out_row0 + j) * (D / group) + d0 / group] = s;
          else
            scales[out_row0 + j] = s;
        }
      }
    }
  }
}

// ------------------------------------------------- jpeg int8 archive, r = 8

// Max over aligned groups of `width` lanes of non-negative, non-NaN floats
// (compared as integers, which orders them the same way): DPP row permutes
// inside 16 lanes (quad swaps, half-row and row mirrors), shuffles beyond.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t v) {
  return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float group_amax(float v, int width) {
  uint32_t u = __float_as_uint(v);
  if (width > 1) u = dpp_umax<0xB1>(u);   // quad_perm [1,0,3,2]
  if (width > 2) u = dpp_umax<0x4E>(u);   // quad_perm [2,3,0,1]
  if (width > 4) u = dpp_umax<0x141>(u);  // row_half_mirror
  if (width > 8) u = dpp_umax<0x140>(u);  // row_mirror
  if (width > 16) u = max(u, (uint32_t)__shfl_xor((int)u, 16, 64));
  if (width > 32) u = max(u, (uint32_t)__shfl_xor((int)u, 32, 64));
  return __uint_as_float(u);
}

// fl(a / 127) for every finite a >= 0: y0 = fl(a R) with R = fl(1/127) is
// within an ulp of the quotient, the residual a - 127 y0 is exact in one
// fma, and one correction step rounds correctly (checked exhaustively over
// all 2^31 non-negative finite floats by tests/test_quant_shortcut.py).
__device__ __forceinline__ float div127(float a) {
  constexpr float R = 1.0f / 127.0f;
  const float y0 = a * R;
  const float e = __builtin_fmaf(-y0, 127.0f, a);
  return __builtin_fmaf(e, R, y0);
}

// stream-dtype rounding of a value that is only used again as fp32 (NaN
// stays NaN; the payload is irrelevant here)
template <typename T>
__device__ __forceinline__ float round_trip(float f) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    return (float)(__bf16)f;
  } else {
    return to_f32(from_f32<T>(f));
  }
}

// Smallest normal scale of the stream dtype: with a normal scale the
// row's quotients stay below 127.5 in magnitude (the scale is absmax / 127
// rounded with relative error <= 2^-8), so their rounded values need no
// clamp.
template <typename T>
__device__ __forceinline__ constexpr float min_normal_scale() {
  return std::is_same<T, f16_t>::value ? 0x1p-14f : 0x1p-126f;
}

// Codes of 8 coefficients of one quantizer row with scale s, packed into
// two dwords; the same codes as quant_code.  rs is the hardware reciprocal
// (relative error <= 2^-23): for |c / s| < 128, x = fl(c rs) lies within
// 1.5 * 2^-16 of c / s and fl(c / s) within 2^-18, so both round to the
// same integer unless x is within 2^-14 of a half-integer.  x + 1.5 * 2^23
// rounds x to an integer held in the low mantissa bits (two's complement
// in the low byte), so one add gives rint(x) and the code byte.  Rows with a
// tie candidate or a scale outside the normal range take the IEEE quotient
// for all 8 elements (a few rows in a thousand).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ u32x2 quantize8(const float (&c)[8], float s) {
  constexpr float kMagic = 0x1.8p23f;
  const bool normal = s >= min_normal_scale<T>() && s <= 0x1p126f;
  const float rs = __builtin_amdgcn_rcpf(s);
  float y[8];
  float dm = 0.f;
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const float x = c[v] * rs;
    y[v] = x + kMagic;
    dm = fmaxf(dm, fabsf(x - (y[v] - kMagic)));
  }
  // NaN elements (dropped by the max) have NaN y and code 0, as below
  if (!normal || !(dm < 0.5f - 0x1p-14f)) {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float q = __builtin_rintf(c[v] / s);
      y[v] = (q == q ? fminf(fmaxf(q, -127.f), 127.f) : 0.f) + kMagic;
    }
  }
  uint32_t u[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) u[v] = __float_as_uint(y[v]);
  const uint32_t lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(u[3], u[2], 0x0c0c0400u),
                                            __builtin_amdgcn_perm(u[1], u[0], 0x0c0c0400u),
                                            0x05040100u);
  const uint32_t hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(u[7], u[6], 0x0c0c0400u),
                                            __builtin_amdgcn_perm(u[5], u[4], 0x0c0c0400u),
                                            0x05040100u);
  return u32x2{lo, hi};
}

// jpeg int8 archive of complete 8-token blocks, 8 features per lane: the
// jpeg_encode_kernel<T, 8, 8, true> computation (same fma chain, dtype
// rounding, scale and codes) with the block loads unconditional, the row
// absmax on DPP, the divisions replaced by exact shortcuts and KT (the
// kept frequencies, 0 = runtime k) unrolled.
template <typename T, int KT, bool GATED = false>
__global__ __launch_bounds__(kThreads) void jpeg_encode_r8q_kernel(
    const T* __restrict__ x, int64_t sb, int64_t sh, int64_t ss, int64_t H, int64_t m,
    int64_t D, int k_rt, const float* __restrict__ basis, int8_t* __restrict__ out,
    float* __restrict__ scales, int64_t cap, int64_t n0, int64_t items, int lpi_log2,
    const int64_t* __restrict__ gate = nullptr) {
  constexpr int R = 8, VEC = 8;
  if constexpr (GATED) {
    // gate = device (n_blocks, n_tail): archive only a completed tail
    if (gate[1] != R - 1) return;
    n0 = gate[0];
    if (n0 < 0 || n0 + m > cap) return;
  }
  const int k = KT > 0 ? KT : k_rt;
  const ItemMap im = item_of_thread(lpi_log2);
  const bool live = im.item < items;
  const int64_t item = live ? im.item : 0;
  const int64_t bh = item / m, blk = item - bh * m;
  const int64_t b = bh / H, h = bh - b * H;
  const int64_t d0 = (int64_t)im.lane * VEC;
  const bool active = live && d0 < D;
  const T* src = x + b * sb + h * sh + blk * R * ss + (active ? d0 : 0);

  // All R token loads are issued before any of them is consumed (the
  // scheduling barrier keeps the backend from waiting on the first load to
  // widen it while the others are still unissued).
  vec_t<T, VEC> raw[R];
  if (active) {
#pragma unroll
    for (int t = 0; t < R; ++t) raw[t] = *reinterpret_cast<const vec_t<T, VEC>*>(src + t * ss);
  } else {
#pragma unroll
    for (int t = 0; t < R; ++t)
#pragma unroll
      for (int v = 0; v < VEC; ++v) raw[t].v[v] = from_f32<T>(0.f);
  }
  __builtin_amdgcn_sched_barrier(0);
  float xr[R][VEC];
#pragma unroll
  for (int t = 0; t < R; ++t)
#pragma unroll
    for (int v = 0; v < VEC; ++v) xr[t][v] = to_f32(raw[t].v[v]);

  int8_t* dst = out + (bh * cap + n0 + blk) * k * D + d0;
  float* sdst = scales + (bh * cap + n0 + blk) * k;
  const int width = 1 << lpi_log2;
#pragma unroll
  for (int j = 0; j < k; ++j) {
    const float* mj = basis + j * R;
    float c[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) c[v] = 0.f;
#pragma unroll
    for (int t = 0; t < R; ++t) {
      const float w = mj[t];
#pragma unroll
      for (int v = 0; v < VEC; ++v) c[v] = __builtin_fmaf(xr[t][v], w, c[v]);
    }
    float amax = 0.f;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      c[v] = round_trip<T>(c[v]);
      amax = fmaxf(amax, fabsf(c[v]));
    }
    amax = group_amax(amax, width);
    float s = round_trip<T>(amax <= 0x1.fffffep127f ? div127(amax) : amax / 127.0f);
    if (!(s > 0.f)) s = 1.0f;
    const u32x2 qv = quantize8<T>(c, s);
    if (active) {
      // nontemporal stores: this write-once stream runs measurably faster
      // when it does not allocate in the caches
      __builtin_nontemporal_store(qv, reinterpret_cast<u32x2*>(dst + (int64_t)j * D));
      if (im.lane == 0) __builtin_nontemporal_store(s, sdst + j);
    }
  }
}

// ---------------------------------------------------------------- jpeg decode

template <typename TI, typename TO, int VEC, int RMAX, bool QUANT>
__global__ __launch_bounds__(kThreads) void jpeg_decode_kernel(
    const TI* __restrict__ store, const float* __restrict__ scales, int64_t H, int64_t cap,
    int64_t a, int64_t nblk, int64_t D, int r, int k, const float* __restrict__ basis,
    TO* __restrict__ out, int64_t osb, int64_t osh, int64_t oss, int64_t out_len,
    int64_t items, int lpi_log2, int group = 0) {
  const ItemMap im = item_of_thread(lpi_log2);
  if (im.item >= items) return;
  const int64_t bh = im.item / nblk, blk = a + (im.item - bh * nblk);
  const int64_t b = bh / H, h = bh - b * H;
  const int64_t d0 = (int64_t)im.lane * VEC;
  if (d0 >= D) return;
  const int64_t row0 = (bh * cap + blk) * k;
  TO* dst = out + b * osb + h * osh + d0;
  const int64_t tok0 = blk * r;

  if constexpr (RMAX > 0) {
    float acc[RMAX][VEC];
#pragma unroll
    for (int t = 0; t < RMAX; ++t)
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[t][v] = 0.f;
    for (int j = 0; j < k; ++j) {
      float c[VEC];
      load_f32<TI, VEC>(store + (row0 + j) * D + d0, c);
      if constexpr (QUANT) {
        const float s =
            group ? scales[(row0 + j) * (D / group) + d0 / group] : scales[row0 + j];
#pragma unroll
        for (int v = 0; v < VEC; ++v) c[v] = c[v] * s;
      }
      const float* mj = basis + (int64_t)j * r;
#pragma unroll
      for (int t = 0; t < RMAX; ++t) {
        if (t < r) {
          const float w = mj[t];
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[t][v] = __builtin_fmaf(c[v], w, acc[t][v]);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < RMAX; ++t)
      if (t < r && tok0 + t < out_len) store_from_f32<TO, VEC>(dst + (tok0 + t) * oss, acc[t]);
  } else {
    for (int t = 0; t < r; ++t) {
      if (tok0 + t >= out_len) break;
      float acc[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
      for (int j = 0; j < k; ++j) {
        float c[VEC];
        load_f32<TI, VEC>(store + (row0 + j) * D + d0, c);
        if constexpr (QUANT) {
          const float s =
              group ? scales[(row0 + j) * (D / group) + d0 / group] : scales[row0 + j];
#pragma unroll
          for (int v = 0; v < VEC; ++v) c[v] = c[v] * s;
        }
        const float w = basis[(int64_t)j * r + t];
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = __builtin_fmaf(c[v], w, acc[v]);
      }
      store_from_f32<TO, VEC>(dst + (tok0 + t) * oss, acc);
    }
  }
}

// ---------------------------------------- jpeg int8 reconstruct, r = 8

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 8 consecutive outputs of one token row, rounded to TO and written with
// nontemporal stores (16 B for f16 / bf16, 2 x 16 B for f32)
template <typename TO>
__device__ __forceinline__ void nt_store8(TO* p, const float (&v)[8]) {
  vec_t<TO, 8> o;
#pragma unroll
  for (int i = 0; i < 8; ++i) o.v[i] = from_f32<TO>(v[i]);
  if constexpr (sizeof(TO) == 2) {
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), reinterpret_cast<u32x4*>(p));
  } else {
    struct Two { u32x4 a, b; };
    const Two t = __builtin_bit_cast(Two, o);
    __builtin_nontemporal_store(t.a, reinterpret_cast<u32x4*>(p));
    __builtin_nontemporal_store(t.b, reinterpret_cast<u32x4*>(p) + 1);
  }
}

// jpeg_decode_kernel<int8_t, TO, 8, 8, true> for r = 8 (same products,
// same fma order): the k code rows and scales of an item are all requested
// before the first is used, KT (0 = runtime k <= 8) is unrolled, and the
// reconstructed rows go out with nontemporal stores.
template <typename TO, int KT>
__global__ __launch_bounds__(kThreads) void jpeg_decode_r8q_kernel(
    const int8_t* __restrict__ store, const float* __restrict__ scales, int64_t H, int64_t cap,
    int64_t a, int64_t nblk, int64_t D, int k_rt, const float* __restrict__ basis,
    TO* __restrict__ out, int64_t osb, int64_t osh, int64_t oss, int64_t out_len,
    int64_t items, int lpi_log2) {
  constexpr int R = 8, VEC = 8, KMAX = KT > 0 ? KT : 8;
  const int k = KT > 0 ? KT : k_rt;
  const ItemMap im = item_of_thread(lpi_log2);
  if (im.item >= items) return;
  const int64_t bh = im.item / nblk, blk = a + (im.item - bh * nblk);
  const int64_t b = bh / H, h = bh - b * H;
  const int64_t d0 = (int64_t)im.lane * VEC;
  if (d0 >= D) return;
  const int64_t row0 = (bh * cap + blk) * k;
  const int8_t* src = store + row0 * D + d0;

  u32x2 q[KMAX];
  float s[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < k) {
      q[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src + (int64_t)j * D));
      s[j] = scales[row0 + j];
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  float acc[R][VEC];
#pragma unroll
  for (int t = 0; t < R; ++t)
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[t][v] = 0.f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j < k) {
      float c[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const int code = (int)(int8_t)(q[j][v >> 2] >> (8 * (v & 3)));
        c[v] = (float)code * s[j];
      }
      const float* mj = basis + j * R;
#pragma unroll
      for (int t = 0; t < R; ++t) {
        const float w = mj[t];
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[t][v] = __builtin_fmaf(c[v], w, acc[t][v]);
      }
    }
  }
  TO* dst = out + b * osb + h * osh + d0 + blk * R * oss;
  const int64_t tok0 = blk * R;
#pragma unroll
  for (int t = 0; t < R; ++t)
    if (tok0 + t < out_len) nt_store8<TO>(dst + t * oss, acc[t]);
}

// ------------------------------------------------------------ quantize rows

template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void quantize_rows_kernel(
    const T* __restrict__ c, int64_t n_rows, int64_t rs, int64_t D, int8_t* __restrict__ codes,
    float* __restrict__ scales, int lpi_log2) {
  const ItemMap im = item_of_thread(lpi_log2);
  const bool live = im.item < n_rows;
  const int64_t row = live ? im.item : 0;
  const int64_t d0 = (int64_t)im.lane * VEC;
  const bool active = live && d0 < D;
  float v[VEC];
  if (active) {
    load_f32<T, VEC>(c + row * rs + d0, v);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = 0.f;
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = group_max_rt(amax, 1 << lpi_log2);
  float s = to_f32(from_f32<T>(amax / 127.0f));
  if (!(s > 0.f)) s = 1.0f;
  const float inv_s = 1.0f / s;
  if (!active) return;
  vec_t<int8_t, VEC> q;
#pragma unroll
  for (int i = 0; i < VEC; ++i) q.v[i] = (int8_t)(int)quant_code(v[i], s, inv_s);
  *reinterpret_cast<vec_t<int8_t, VEC>*>(codes + row * D + d0) = q;
  if (im.lane == 0) scales[row] = s;
}

template <typename TO>
__global__ __launch_bounds__(kThreads) void dequantize_rows_kernel(
    const int8_t* __restrict__ codes, const float* __restrict__ scales, int64_t n, int64_t D,
    TO* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  // q.to(dtype) * scale.to(dtype): both operands rounded to the output
  // dtype first, product rounded once.
  const float qv = to_f32(from_f32<TO>((float)(int)codes[i]));
  const float sv = to_f32(from_f32<TO>(scales[i / D]));
  out[i] = from_f32<TO>(qv * sv);
}

// ----------------------------------------------------------------- png encode

typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));

// PACK: the packed Top-M layout (fc_png_encode_packed) instead of dense
// deltas: `deltas` is the value store (B*H, cap, keep_m, D), `masks` the
// mask words (B*H, cap, D); 2 <= r <= 16, 1 <= keep_m <= r - 1.
template <typename T, int VEC, int RMAX, bool GATED = false, bool PACK = false>
__global__ __launch_bounds__(kThreads) void png_encode_kernel(
    const T* __restrict__ x, int64_t sb, int64_t sh, int64_t ss, int64_t H, int64_t m,
    int64_t D, int64_t s_valid, int r, int keep_m, float* __restrict__ deltas,
    T* __restrict__ anchors, int64_t cap, int64_t n0, int64_t items, int lpi_log2,
    const int64_t* __restrict__ gate = nullptr, uint32_t* __restrict__ masks = nullptr) {
  if constexpr (GATED) {
    // gate = device (n_blocks, n_tail): archive only a completed tail, as
    // block n_blocks
    if (gate[1] != r - 1) return;
    n0 = gate[0];
    if (n0 < 0 || n0 + m > cap) return;
  }
  const ItemMap im = item_of_thread(lpi_log2);
  if (im.item >= items) return;
  const int64_t bh = im.item / m, blk = im.item - bh * m;
  const int64_t b = bh / H, h = bh - b * H;
  const int64_t d0 = (int64_t)im.lane * VEC;
  if (d0 >= D) return;
  const T* src = x + b * sb + h * sh + d0;
  const int64_t tok0 = blk * r;
  const int64_t slot = bh * cap + n0 + blk;

  // anchor: token 0 of the block, copied in the stream dtype
  {
    vec_t<T, VEC> av;
    if (tok0 < s_valid) {
      av = *reinterpret_cast<const vec_t<T, VEC>*>(src + tok0 * ss);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) av.v[v] = from_f32<T>(0.f);
    }
    *reinterpret_cast<vec_t<T, VEC>*>(anchors + slot * D + d0) = av;
  }

  float xd[RMAX][VEC];
#pragma unroll
  for (int t = 0; t < RMAX; ++t) {
    if (t < r && tok0 + t < s_valid) {
      load_f32<T, VEC>(src + (tok0 + t) * ss, xd[t]);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) xd[t][v] = 0.f;
    }
  }
  // deltas in fp32, in place: xd[i] <- x_{i+1} - x_i
#pragma unroll
  for (int i = 0; i + 1 < RMAX; ++i)
#pragma unroll
    for (int v = 0; v < VEC; ++v) xd[i][v] = xd[i + 1][v] - xd[i][v];

  const int n = r - 1;
  if constexpr (PACK) {
    // kept steps: the Top-M survivors that are not +-0, then the
    // lowest-index +-0 steps until keep_m; the signs of the others (their
    // png_filter value is delta * 0) go to bits 16 + i of the mask word
    uint32_t kept[VEC], word[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      uint32_t key[RMAX];
      uint32_t nzm = 0;
#pragma unroll
      for (int i = 0; i < RMAX; ++i) {
        key[i] = i < n ? topm_key(__float_as_uint(xd[i][v])) : 0u;
        if (key[i] != 0u) nzm |= 1u << i;
      }
      uint32_t km = (uint32_t)topm_mask<RMAX>(key, n, keep_m) & nzm;
      int cnt = __builtin_popcount(km);
      uint32_t sg = 0;
#pragma unroll
      for (int i = 0; i < RMAX; ++i) {
        if (i < n && !((nzm >> i) & 1u) && cnt < keep_m) {
          km |= 1u << i;
          ++cnt;
        }
      }
#pragma unroll
      for (int i = 0; i < RMAX; ++i)
        if (i < n && !((km >> i) & 1u)) sg |= (__float_as_uint(xd[i][v]) >> 31) << i;
      kept[v] = km;
      word[v] = km | (sg << 16);
    }
    uint32_t* mdst = masks + slot * D + d0;
#pragma unroll
    for (int v = 0; v < VEC; ++v) mdst[v] = word[v];
    // slot j of a feature: its j-th kept step, in step order (popcount of
    // every kept word is keep_m, so the lowest remaining bit always exists)
    float* vdst = deltas + slot * (int64_t)keep_m * D + d0;
    for (int j = 0; j < keep_m; ++j) {
      float o[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const int i = __builtin_ctz(kept[v]);
        kept[v] &= kept[v] - 1u;
        float val = xd[0][v];
#pragma unroll
        for (int t = 1; t + 1 < RMAX; ++t) val = i == t ? xd[t][v] : val;
        o[v] = val;
      }
      store_from_f32<float, VEC>(vdst + (int64_t)j * D, o);
    }
    return;
  }
  if (keep_m > 0 && keep_m < n) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      uint32_t key[RMAX];
#pragma unroll
      for (int i = 0; i < RMAX; ++i) key[i] = i < n ? topm_key(__float_as_uint(xd[i][v])) : 0u;
      const uint64_t mask = topm_mask<RMAX>(key, n, keep_m);
#pragma unroll
      for (int i = 0; i + 1 < RMAX; ++i)
        if (!((mask >> i) & 1)) xd[i][v] = xd[i][v] * 0.0f;
    }
  }
  // 16-byte delta rows go out with nontemporal stores (write-once stream:
  // 45.2 -> 40.9 us for the keep-1.0 archive of a 2 x 8 x 16384 x 128 fp32
  // stream; a 32-byte-per-lane decode store measured no better)
  float* dst = deltas + slot * (int64_t)n * D + d0;
#pragma unroll
  for (int i = 0; i + 1 < RMAX; ++i)
    if (i < n) {
      if constexpr (VEC == 4) {
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4_nt, xd[i]),
                                    reinterpret_cast<u32x4_nt*>(dst + i * D));
      } else {
        store_from_f32<float, VEC>(dst + i * D, xd[i]);
      }
    }
}

// ----------------------------------------------------------------- png decode

// The delta rows of a block are requested kPngDecodeBatch at a time before
// any is used (a thread has that many loads in flight instead of one).  The
// C4 read's rate depends on where the anchors sit relative to the deltas:
// with one row per load-use step 43.3 us when both start 128 MB apart in
// one allocation, 52.7-56.9 us at the other offsets tried (so 4.7 to 6.2
// TB/s between runs and boxes, with the allocator's placement); 4 rows per
// batch: 43.2 us and 50.4-52.3 us; 8 rows: 46.6 us and 49.7-51.1 us (the
// registers of 8 rows lower the occupancy).
constexpr int kPngDecodeBatch = 4;

template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void png_decode_kernel(
    const float* __restrict__ deltas, const T* __restrict__ anchors, int64_t H, int64_t cap,
    int64_t a, int64_t nblk, int64_t D, int r, T* __restrict__ out, int64_t osb, int64_t osh,
    int64_t oss, int64_t out_len, int64_t items, int lpi_log2) {
  const ItemMap im = item_of_thread(lpi_log2);
  if (im.item >= items) return;
  const int64_t bh = im.item / nblk, blk = a + (im.item - bh * nblk);
  const int64_t b = bh / H, h = bh - b * H;
  const int64_t d0 = (int64_t)im.lane * VEC;
  if (d0 >= D) return;
  const int64_t slot = bh * cap + blk;
  T* dst = out + b * osb + h * osh + d0;
  const int64_t tok0 = blk * r;
  // rows 1 .. n-1 of the block are written (the output may end inside it)
  const int n = (int)min<int64_t>(r, max<int64_t>(out_len - tok0, 0));
  const float* src = deltas + slot * (int64_t)(r - 1) * D + d0;
  float base[VEC];
  load_f32<T, VEC>(anchors + slot * D + d0, base);
  double run[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) run[v] = 0.0;
  for (int i0 = 1; i0 < n; i0 += kPngDecodeBatch) {
    float dv[kPngDecodeBatch][VEC];
#pragma unroll
    for (int c = 0; c < kPngDecodeBatch; ++c)
      if (i0 + c < n) load_f32<float, VEC>(src + (int64_t)(i0 + c - 1) * D, dv[c]);
#pragma unroll
    for (int c = 0; c < kPngDecodeBatch; ++c) {
      if (i0 + c >= n) break;
      float o[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        run[v] += (double)dv[c][v];
        o[v] = base[v] + (float)run[v];
      }
      store_from_f32<T, VEC>(dst + (tok0 + i0 + c) * oss, o);
    }
  }
  if (n > 0) store_from_f32<T, VEC>(dst + tok0 * oss, base);
}

constexpr int kPackMaxKept = 8;  // kept deltas the packed read holds in registers

// Reconstruction from a packed archive: the dense decoder's fp64 running sum
// over the unpacked deltas (step i: the feature's next slot value when bit i
// of its mask word is set, else a zero with sign bit 16 + i).
template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void png_decode_packed_kernel(
    const float* __restrict__ vals, const uint32_t* __restrict__ masks,
    const T* __restrict__ anchors, int64_t H, int64_t cap, int64_t a, int64_t nblk, int64_t D,
    int r, int keep_m, T* __restrict__ out, int64_t osb, int64_t osh, int64_t oss,
    int64_t out_len, int64_t items, int lpi_log2) {
  const ItemMap im = item_of_thread(lpi_log2);
  if (im.item >= items) return;
  const int64_t bh = im.item / nblk, blk = a + (im.item - bh * nblk);
  const int64_t b = bh / H, h = bh - b * H;
  const int64_t d0 = (int64_t)im.lane * VEC;
  if (d0 >= D) return;
  const int64_t slot = bh * cap + blk;
  T* dst = out + b * osb + h * osh + d0;
  const int64_t tok0 = blk * r;
  float base[VEC];
  load_f32<T, VEC>(anchors + slot * D + d0, base);
  if (tok0 < out_len) store_from_f32<T, VEC>(dst + tok0 * oss, base);
  uint32_t w[VEC];
  int cur[VEC];
  double run[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    w[v] = masks[slot * D + d0 + v];
    cur[v] = 0;
    run[v] = 0.0;
  }
  const float* src = vals + slot * (int64_t)keep_m * D + d0;
  if (keep_m <= kPackMaxKept) {
    // the item's kept values once, as VEC-wide loads, then taken in step
    // order from registers (a gather per step fetched each line ~3x)
    float kv[kPackMaxKept][VEC];
#pragma unroll
    for (int m = 0; m < kPackMaxKept; ++m) {
      if (m < keep_m) {
        load_f32<float, VEC>(src + (int64_t)m * D, kv[m]);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) kv[m][v] = 0.f;
      }
    }
    for (int i = 1; i < r; ++i) {
      if (tok0 + i >= out_len) break;
      float o[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        float dv = __uint_as_float(((w[v] >> (15 + i)) & 1u) << 31);
        if ((w[v] >> (i - 1)) & 1u) {
          const int ci = min(cur[v]++, keep_m - 1);
          float sel = kv[0][v];
#pragma unroll
          for (int m = 1; m < kPackMaxKept; ++m) sel = ci == m ? kv[m][v] : sel;
          dv = sel;
        }
        run[v] += (double)dv;
        o[v] = base[v] + (float)run[v];
      }
      store_from_f32<T, VEC>(dst + (tok0 + i) * oss, o);
    }
    return;
  }
  for (int i = 1; i < r; ++i) {
    if (tok0 + i >= out_len) break;
    float o[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      float dv = __uint_as_float(((w[v] >> (15 + i)) & 1u) << 31);
      if ((w[v] >> (i - 1)) & 1u) dv = src[(int64_t)min(cur[v]++, keep_m - 1) * D + v];
      run[v] += (double)dv;
      o[v] = base[v] + (float)run[v];
    }
    store_from_f32<T, VEC>(dst + (tok0 + i) * oss, o);
  }
}

// Dense deltas (png_filter's layout) from a packed archive, one thread per
// (block, feature).
__global__ __launch_bounds__(kThreads) void png_unpack_kernel(
    const float* __restrict__ vals, const uint32_t* __restrict__ masks, int64_t cap, int64_t a,
    int64_t nblk, int64_t D, int r, int keep_m, float* __restrict__ deltas, int64_t d_cap,
    int64_t total) {
  const int64_t x = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (x >= total) return;
  const int64_t d = x % D, it = x / D;
  const int64_t bh = it / nblk, blk = a + (it - bh * nblk);
  const int64_t slot = bh * cap + blk;
  const uint32_t w = masks[slot * D + d];
  const float* src = vals + slot * (int64_t)keep_m * D + d;
  float* dst = deltas + (bh * d_cap + blk) * (int64_t)(r - 1) * D + d;
  int cur = 0;
  for (int i = 0; i + 1 < r; ++i) {
    float dv = __uint_as_float(((w >> (16 + i)) & 1u) << 31);
    if ((w >> i) & 1u) dv = src[(int64_t)min(cur++, keep_m - 1) * D];
    dst[(int64_t)i * D] = dv;
  }
}

// ------------------------------------------------------------ host helpers

thread_local int g_last_hip_error = 0;

int check_launch() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_last_hip_error = (int)e;
    return FC_ERR_HIP;
  }
  return FC_OK;
}

int hip_status(hipError_t e) {
  if (e == hipSuccess) return FC_OK;
  g_last_hip_error = (int)e;
  return FC_ERR_HIP;
}

static bool aligned(const void* p, int64_t bytes) {
  return p == nullptr || ((uintptr_t)p % (uintptr_t)bytes) == 0;
}

int esize_of(int dt) {
  switch (dt) {
    case FC_F32: return 4;
    case FC_F16: return 2;
    case FC_BF16: return 2;
    case FC_I8: return 1;
    default: return 0;
  }
}

// Elements per lane: the widest of {8, 4, 1} (<= max_vec) that divides D
// and every stride, keeps every pointer aligned and needs <= 64 lanes.
// 0 if none fits.
static int pick_vec(int64_t D, int max_vec, std::initializer_list<int64_t> strides,
                    std::initializer_list<std::pair<const void*, int>> ptrs) {
  for (int vec : {8, 4, 1}) {
    if (vec > max_vec || D % vec || (D + vec - 1) / vec > 64) continue;
    bool ok = true;
    for (int64_t s : strides) ok = ok && (s % vec == 0);
    for (const auto& pp : ptrs) ok = ok && aligned(pp.first, (int64_t)vec * pp.second);
    if (ok) return vec;
  }
  return 0;
}

static int log2_lanes(int64_t D, int vec) {
  const int64_t need = (D + vec - 1) / vec;
  int l = 0;
  while ((int64_t(1) << l) < need) ++l;
  return l;
}

static dim3 grid_for(int64_t items, int lpi_log2) {
  const int64_t per = kThreads >> lpi_log2;
  return dim3((unsigned)((items + per - 1) / per));
}

// Register-resident block size bucket for r, or 0 for the streaming path.
// rmax*vec is kept <= 64 floats per lane.
static int rmax_for(int r) { return r <= 8 ? 8 : (r <= 16 ? 16 : 0); }
static int max_vec_for(int rmax) { return rmax == 8 ? 8 : (rmax == 16 ? 4 : 8); }

template <typename F>
int with_float_type(int dt, F&& f) {
  switch (dt) {
    case FC_F32: return f(float{});
    case FC_F16: return f(f16_t{});
    case FC_BF16: return f(bf16_t{});
    default: return FC_ERR_ARG;
  }
}

template <int... Vs, typename F>
int with_int(int v, F&& f) {
  int rc = FC_ERR_UNSUPPORTED;
  bool hit = false;
  ((v == Vs ? (rc = f(std::integral_constant<int, Vs>{}), hit = true) : false), ...);
  return hit ? rc : FC_ERR_UNSUPPORTED;
}

}  // namespace fc

using namespace fc;

extern "C" {

int fc_version(void) { return 100; }

const char* fc_status_string(int status) {
  switch (status) {
    case FC_OK: return "ok";
    case FC_ERR_ARG: return "invalid argument";
    case FC_ERR_UNSUPPORTED: return "unsupported by this build's kernels";
    case FC_ERR_HIP: return "HIP runtime error";
    case FC_ERR_SCRATCH:
      return "the call needs more scratch than fc_decode_attention_noalloc's static array "
             "holds (FC_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status";
  }
}

int fc_last_hip_error(void) { return g_last_hip_error; }

}  // extern "C"

namespace fc {

template <bool GATED>
static int jpeg_encode_launch(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb,
                              int64_t x_sh, int64_t x_ss, int64_t s_valid, int64_t m, int64_t D,
                              int r, int k, const float* basis, void* coeffs, float* scales,
                              int64_t cap, int64_t n0, int quant_bits, void* stream,
                              const int64_t* gate, int group = 0) {
  if (B < 0 || H < 0 || m < 0 || D <= 0 || r < 1 || k < 1 || k > r) return FC_ERR_ARG;
  if (quant_bits != 0 && quant_bits != 8) return FC_ERR_ARG;
  if (group && (group != 32 || quant_bits != 8 || D % group)) return FC_ERR_ARG;
  if (n0 < 0 || n0 + m > cap) return FC_ERR_ARG;
  const int64_t items = B * H * m;
  if (items == 0) return FC_OK;
  if (!x || !basis || !coeffs || (quant_bits && !scales)) return FC_ERR_ARG;
  if (r > FC_MAX_BLOCK || D > FC_MAX_HEAD_DIM) return FC_ERR_UNSUPPORTED;
  const int es = esize_of(x_dtype);
  if (es == 0 || x_dtype == FC_I8) return FC_ERR_ARG;
  const int rmax = rmax_for(r);
  const int vec = pick_vec(D, max_vec_for(rmax), {x_sb, x_sh, x_ss},
                           {{x, es}, {coeffs, quant_bits ? 1 : es}});
  if (!vec) return FC_ERR_UNSUPPORTED;
  const int lg = log2_lanes(D, vec);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = grid_for(items, lg);
  if (quant_bits && !group && r == 8 && vec == 8 && s_valid >= m * r) {
    const int rc = with_float_type(x_dtype, [&](auto tv) {
      using T = decltype(tv);
      return with_int<2, 4, 8, 0>(k == 2 || k == 4 || k == 8 ? k : 0, [&](auto kc) {
        constexpr int KT = decltype(kc)::value;
        jpeg_encode_r8q_kernel<T, KT, GATED><<<grid, kThreads, 0, st>>>(
            (const T*)x, x_sb, x_sh, x_ss, H, m, D, k, basis, (int8_t*)coeffs, scales, cap, n0,
            items, lg, gate);
        return FC_OK;
      });
    });
    return rc != FC_OK ? rc : check_launch();
  }
  const int rc = with_float_type(x_dtype, [&](auto tv) {
    using T = decltype(tv);
    return with_int<1, 4, 8>(vec, [&](auto vc) {
      constexpr int VEC = decltype(vc)::value;
      return with_int<8, 16, 0>(rmax, [&](auto rc_) {
        constexpr int RMAX = decltype(rc_)::value;
        if (quant_bits)
          jpeg_encode_kernel<T, VEC, RMAX, true, GATED><<<grid, kThreads, 0, st>>>(
              (const T*)x, x_sb, x_sh, x_ss, H, m, D, s_valid, r, k, basis, coeffs, scales, cap,
              n0, items, lg, gate, group);
        else
          jpeg_encode_kernel<T, VEC, RMAX, false, GATED><<<grid, kThreads, 0, st>>>(
              (const T*)x, x_sb, x_sh, x_ss, H, m, D, s_valid, r, k, basis, coeffs, scales, cap,
              n0, items, lg, gate);
        return FC_OK;
      });
    });
  });
  return rc != FC_OK ? rc : check_launch();
}

int jpeg_encode_gated(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb,
                      int64_t x_sh, int64_t x_ss, int64_t D, int r, int k, const float* basis,
                      void* coeffs, float* scales, int64_t cap, int quant_bits, void* stream,
                      const int64_t* gate, int group) {
  if (!gate || cap < 1) return FC_ERR_ARG;
  return jpeg_encode_launch<true>(x, x_dtype, B, H, x_sb, x_sh, x_ss, r, 1, D, r, k, basis,
                                  coeffs, scales, cap, 0, quant_bits, stream, gate, group);
}

// masks != NULL: the packed layout (deltas = the value store)
template <bool GATED>
static int png_encode_launch(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb,
                             int64_t x_sh, int64_t x_ss, int64_t s_valid, int64_t m, int64_t D,
                             int r, int keep_m, float* deltas, void* anchors, int64_t cap,
                             int64_t n0, void* stream, const int64_t* gate,
                             uint32_t* masks = nullptr) {
  if (B < 0 || H < 0 || m < 0 || D <= 0 || r < 2 || keep_m < 0) return FC_ERR_ARG;
  if (masks && (r > 16 || keep_m < 1 || keep_m > r - 1)) return FC_ERR_ARG;
  if (n0 < 0 || n0 + m > cap) return FC_ERR_ARG;
  const int64_t items = B * H * m;
  if (items == 0) return FC_OK;
  if (!x || !deltas || !anchors) return FC_ERR_ARG;
  if (r > FC_MAX_BLOCK || D > FC_MAX_HEAD_DIM) return FC_ERR_UNSUPPORTED;
  const int es = esize_of(x_dtype);
  if (!es || x_dtype == FC_I8) return FC_ERR_ARG;
  // register-resident block bucket; rmax*vec <= 64 floats per lane
  const int rmax = r <= 8 ? 8 : (r <= 16 ? 16 : (r <= 32 ? 32 : 64));
  const int max_vec = rmax == 8 ? 8 : (rmax == 16 ? 4 : 1);
  const int vec = pick_vec(D, max_vec, {x_sb, x_sh, x_ss},
                           {{x, es}, {anchors, es}, {deltas, 4}, {masks, 4}});
  if (!vec) return FC_ERR_UNSUPPORTED;
  const int lg = log2_lanes(D, vec);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = grid_for(items, lg);
  const int rc = with_float_type(x_dtype, [&](auto tv) {
    using T = decltype(tv);
    return with_int<1, 4, 8>(vec, [&](auto vc) {
      constexpr int VEC = decltype(vc)::value;
      return with_int<8, 16, 32, 64>(rmax, [&](auto rc_) {
        constexpr int RMAX = decltype(rc_)::value;
        if constexpr (RMAX * VEC <= 64) {
          if (masks) {
            if constexpr (RMAX <= 16) {
              png_encode_kernel<T, VEC, RMAX, GATED, true><<<grid, kThreads, 0, st>>>(
                  (const T*)x, x_sb, x_sh, x_ss, H, m, D, s_valid, r, keep_m, deltas,
                  (T*)anchors, cap, n0, items, lg, gate, masks);
              return FC_OK;
            } else {
              return FC_ERR_ARG;
            }
          }
          png_encode_kernel<T, VEC, RMAX, GATED><<<grid, kThreads, 0, st>>>(
              (const T*)x, x_sb, x_sh, x_ss, H, m, D, s_valid, r, keep_m, deltas, (T*)anchors,
              cap, n0, items, lg, gate);
          return FC_OK;
        } else {
          return FC_ERR_UNSUPPORTED;
        }
      });
    });
  });
  return rc != FC_OK ? rc : check_launch();
}


int png_encode_gated(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb,
                     int64_t x_sh, int64_t x_ss, int64_t D, int r, int keep_m, float* deltas,
                     void* anchors, int64_t cap, void* stream, const int64_t* gate,
                     uint32_t* masks) {
  if (!gate || cap < 1) return FC_ERR_ARG;
  return png_encode_launch<true>(x, x_dtype, B, H, x_sb, x_sh, x_ss, r, 1, D, r, keep_m, deltas,
                                 anchors, cap, 0, stream, gate, masks);
}

}  // namespace fc

extern "C" {

int fc_jpeg_encode(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb, int64_t x_sh,
                   int64_t x_ss, int64_t s_valid, int64_t m, int64_t D, int r, int k,
                   const float* basis, void* coeffs, float* scales, int64_t cap, int64_t n0,
                   int quant_bits, void* stream) {
  return jpeg_encode_launch<false>(x, x_dtype, B, H, x_sb, x_sh, x_ss, s_valid, m, D, r, k, basis,
                                   coeffs, scales, cap, n0, quant_bits, stream, nullptr);
}

int fc_jpeg_encode_grouped(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb,
                           int64_t x_sh, int64_t x_ss, int64_t s_valid, int64_t m, int64_t D,
                           int r, int k, const float* basis, int8_t* codes, float* scales,
                           int64_t cap, int64_t n0, int group, void* stream) {
  if (group != 32) return FC_ERR_ARG;
  return jpeg_encode_launch<false>(x, x_dtype, B, H, x_sb, x_sh, x_ss, s_valid, m, D, r, k, basis,
                                   codes, scales, cap, n0, 8, stream, nullptr, group);
}

}  // extern "C"

static int jpeg_decode_launch(const void* store, int store_dtype, const float* scales, int64_t B,
                              int64_t H, int64_t cap, int64_t a, int64_t nblk, int64_t D, int r,
                              int k, const float* basis, void* out, int out_dtype, int64_t o_sb,
                              int64_t o_sh, int64_t o_ss, int64_t out_len, void* stream,
                              int group) {
  if (B < 0 || H < 0 || a < 0 || nblk < 0 || a + nblk > cap || D <= 0 || r < 1 || k < 1 ||
      k > r)
    return FC_ERR_ARG;
  if (group && (group != 32 || store_dtype != FC_I8 || D % group)) return FC_ERR_ARG;
  const int64_t items = B * H * nblk;
  if (items == 0) return FC_OK;
  if (!store || !basis || !out) return FC_ERR_ARG;
  const bool quant = store_dtype == FC_I8;
  if (quant && !scales) return FC_ERR_ARG;
  if (r > FC_MAX_BLOCK || D > FC_MAX_HEAD_DIM) return FC_ERR_UNSUPPORTED;
  const int es_in = esize_of(store_dtype), es_out = esize_of(out_dtype);
  if (!es_in || !es_out || out_dtype == FC_I8) return FC_ERR_ARG;
  const int rmax = rmax_for(r);
  const int vec =
      pick_vec(D, max_vec_for(rmax), {o_sb, o_sh, o_ss}, {{store, es_in}, {out, es_out}});
  if (!vec) return FC_ERR_UNSUPPORTED;
  const int lg = log2_lanes(D, vec);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = grid_for(items, lg);
  auto launch = [&](auto ti, auto to) {
    using TI = decltype(ti);
    using TO = decltype(to);
    return with_int<1, 4, 8>(vec, [&](auto vc) {
      constexpr int VEC = decltype(vc)::value;
      return with_int<8, 16, 0>(rmax, [&](auto rc_) {
        constexpr int RMAX = decltype(rc_)::value;
        jpeg_decode_kernel<TI, TO, VEC, RMAX, std::is_same<TI, int8_t>::value>
            <<<grid, kThreads, 0, st>>>((const TI*)store, scales, H, cap, a, nblk, D, r, k,
                                        basis, (TO*)out, o_sb, o_sh, o_ss, out_len, items, lg,
                                        group);
        return FC_OK;
      });
    });
  };
  int rc;
  if (quant && !group && r == 8 && vec == 8) {
    rc = with_float_type(out_dtype, [&](auto to) {
      using TO = decltype(to);
      return with_int<2, 4, 8, 0>(k == 2 || k == 4 || k == 8 ? k : 0, [&](auto kc) {
        constexpr int KT = decltype(kc)::value;
        jpeg_decode_r8q_kernel<TO, KT><<<grid, kThreads, 0, st>>>(
            (const int8_t*)store, scales, H, cap, a, nblk, D, k, basis, (TO*)out, o_sb, o_sh,
            o_ss, out_len, items, lg);
        return FC_OK;
      });
    });
  } else if (quant) {
    rc = with_float_type(out_dtype, [&](auto to) { return launch(int8_t{}, to); });
  } else if (out_dtype == FC_F32) {
    rc = with_float_type(store_dtype, [&](auto ti) { return launch(ti, float{}); });
  } else if (out_dtype == store_dtype) {
    rc = with_float_type(store_dtype, [&](auto ti) { return launch(ti, ti); });
  } else {
    return FC_ERR_UNSUPPORTED;
  }
  return rc != FC_OK ? rc : check_launch();
}

extern "C" {

int fc_jpeg_decode(const void* store, int store_dtype, const float* scales, int64_t B,
                   int64_t H, int64_t cap, int64_t a, int64_t nblk, int64_t D, int r, int k,
                   const float* basis, void* out, int out_dtype, int64_t o_sb, int64_t o_sh,
                   int64_t o_ss, int64_t out_len, void* stream) {
  return jpeg_decode_launch(store, store_dtype, scales, B, H, cap, a, nblk, D, r, k, basis, out,
                            out_dtype, o_sb, o_sh, o_ss, out_len, stream, 0);
}

int fc_jpeg_decode_grouped(const int8_t* codes, const float* scales, int64_t B, int64_t H,
                           int64_t cap, int64_t a, int64_t nblk, int64_t D, int r, int k,
                           int group, const float* basis, void* out, int out_dtype, int64_t o_sb,
                           int64_t o_sh, int64_t o_ss, int64_t out_len, void* stream) {
  if (group != 32) return FC_ERR_ARG;
  return jpeg_decode_launch(codes, FC_I8, scales, B, H, cap, a, nblk, D, r, k, basis, out,
                            out_dtype, o_sb, o_sh, o_ss, out_len, stream, group);
}

int fc_quantize_rows(const void* c, int c_dtype, int64_t n_rows, int64_t c_rs, int64_t D,
                     int8_t* codes, float* scales, void* stream) {
  if (n_rows < 0 || D <= 0) return FC_ERR_ARG;
  if (n_rows == 0) return FC_OK;
  if (!c || !codes || !scales) return FC_ERR_ARG;
  const int es = esize_of(c_dtype);
  if (!es || c_dtype == FC_I8) return FC_ERR_ARG;
  if (D > FC_MAX_HEAD_DIM) return FC_ERR_UNSUPPORTED;
  const int vec = pick_vec(D, 8, {c_rs}, {{c, es}, {codes, 1}});
  if (!vec) return FC_ERR_UNSUPPORTED;
  const int lg = log2_lanes(D, vec);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = grid_for(n_rows, lg);
  const int rc = with_float_type(c_dtype, [&](auto tv) {
    using T = decltype(tv);
    return with_int<1, 4, 8>(vec, [&](auto vc) {
      constexpr int VEC = decltype(vc)::value;
      quantize_rows_kernel<T, VEC>
          <<<grid, kThreads, 0, st>>>((const T*)c, n_rows, c_rs, D, codes, scales, lg);
      return FC_OK;
    });
  });
  return rc != FC_OK ? rc : check_launch();
}

int fc_dequantize_rows(const int8_t* codes, const float* scales, int64_t n_rows, int64_t D,
                       void* out, int out_dtype, void* stream) {
  if (n_rows < 0 || D <= 0) return FC_ERR_ARG;
  const int64_t n = n_rows * D;
  if (n == 0) return FC_OK;
  if (!codes || !scales || !out) return FC_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((n + kThreads - 1) / kThreads));
  const int rc = with_float_type(out_dtype, [&](auto to) {
    using TO = decltype(to);
    dequantize_rows_kernel<TO><<<grid, kThreads, 0, st>>>(codes, scales, n, D, (TO*)out);
    return FC_OK;
  });
  return rc != FC_OK ? rc : check_launch();
}

int fc_png_encode(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb, int64_t x_sh,
                  int64_t x_ss, int64_t s_valid, int64_t m, int64_t D, int r, int keep_m,
                  float* deltas, void* anchors, int64_t cap, int64_t n0, void* stream) {
  return png_encode_launch<false>(x, x_dtype, B, H, x_sb, x_sh, x_ss, s_valid, m, D, r, keep_m,
                                  deltas, anchors, cap, n0, stream, nullptr);
}

int fc_png_encode_packed(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb,
                         int64_t x_sh, int64_t x_ss, int64_t s_valid, int64_t m, int64_t D, int r,
                         int keep_m, float* vals, uint32_t* masks, void* anchors, int64_t cap,
                         int64_t n0, void* stream) {
  if (!masks && B * H * m > 0) return FC_ERR_ARG;
  return png_encode_launch<false>(x, x_dtype, B, H, x_sb, x_sh, x_ss, s_valid, m, D, r, keep_m,
                                  vals, anchors, cap, n0, stream, nullptr, masks);
}

int fc_png_decode_packed(const float* vals, const uint32_t* masks, const void* anchors,
                         int anchor_dtype, int64_t B, int64_t H, int64_t cap, int64_t a,
                         int64_t nblk, int64_t D, int r, int keep_m, void* out, int64_t o_sb,
                         int64_t o_sh, int64_t o_ss, int64_t out_len, void* stream) {
  if (B < 0 || H < 0 || a < 0 || nblk < 0 || a + nblk > cap || D <= 0 || r < 2 || r > 16 ||
      keep_m < 1 || keep_m > r - 1)
    return FC_ERR_ARG;
  const int64_t items = B * H * nblk;
  if (items == 0) return FC_OK;
  if (!vals || !masks || !anchors || !out) return FC_ERR_ARG;
  if (D > FC_MAX_HEAD_DIM) return FC_ERR_UNSUPPORTED;
  const int es = esize_of(anchor_dtype);
  if (!es || anchor_dtype == FC_I8) return FC_ERR_ARG;
  const int vec = pick_vec(D, 4, {o_sb, o_sh, o_ss}, {{anchors, es}, {out, es}, {vals, 4}});
  if (!vec) return FC_ERR_UNSUPPORTED;
  const int lg = log2_lanes(D, vec);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = grid_for(items, lg);
  const int rc = with_float_type(anchor_dtype, [&](auto tv) {
    using T = decltype(tv);
    return with_int<1, 4>(vec, [&](auto vc) {
      constexpr int VEC = decltype(vc)::value;
      png_decode_packed_kernel<T, VEC><<<grid, kThreads, 0, st>>>(
          vals, masks, (const T*)anchors, H, cap, a, nblk, D, r, keep_m, (T*)out, o_sb, o_sh,
          o_ss, out_len, items, lg);
      return FC_OK;
    });
  });
  return rc != FC_OK ? rc : check_launch();
}

int fc_png_unpack(const float* vals, const uint32_t* masks, int64_t B, int64_t H, int64_t cap,
                  int64_t a, int64_t nblk, int64_t D, int r, int keep_m, float* deltas,
                  int64_t d_cap, void* stream) {
  if (B < 0 || H < 0 || a < 0 || nblk < 0 || a + nblk > cap || a + nblk > d_cap || D <= 0 ||
      r < 2 || r > 16 || keep_m < 1 || keep_m > r - 1)
    return FC_ERR_ARG;
  const int64_t total = B * H * nblk * D;
  if (total == 0) return FC_OK;
  if (!vals || !masks || !deltas) return FC_ERR_ARG;
  const dim3 grid((unsigned)((total + kThreads - 1) / kThreads));
  png_unpack_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>(vals, masks, cap, a, nblk, D, r,
                                                                 keep_m, deltas, d_cap, total);
  return check_launch();
}

int fc_png_decode(const float* deltas, const void* anchors, int anchor_dtype, int64_t B,
                  int64_t H, int64_t cap, int64_t a, int64_t nblk, int64_t D, int r, void* out,
                  int64_t o_sb, int64_t o_sh, int64_t o_ss, int64_t out_len, void* stream) {
  if (B < 0 || H < 0 || a < 0 || nblk < 0 || a + nblk > cap || D <= 0 || r < 2)
    return FC_ERR_ARG;
  const int64_t items = B * H * nblk;
  if (items == 0) return FC_OK;
  if (!deltas || !anchors || !out) return FC_ERR_ARG;
  if (r > FC_MAX_BLOCK || D > FC_MAX_HEAD_DIM) return FC_ERR_UNSUPPORTED;
  const int es = esize_of(anchor_dtype);
  if (!es || anchor_dtype == FC_I8) return FC_ERR_ARG;
  const int vec =
      pick_vec(D, 8, {o_sb, o_sh, o_ss}, {{anchors, es}, {out, es}, {deltas, 4}});
  if (!vec) return FC_ERR_UNSUPPORTED;
  const int lg = log2_lanes(D, vec);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = grid_for(items, lg);
  const int rc = with_float_type(anchor_dtype, [&](auto tv) {
    using T = decltype(tv);
    return with_int<1, 4, 8>(vec, [&](auto vc) {
      constexpr int VEC = decltype(vc)::value;
      png_decode_kernel<T, VEC><<<grid, kThreads, 0, st>>>(
          deltas, (const T*)anchors, H, cap, a, nblk, D, r, (T*)out, o_sb, o_sh, o_ss, out_len,
          items, lg);
      return FC_OK;
    });
  });
  return rc != FC_OK ? rc : check_launch();
}

// Host restatement hook: the Top-M keep mask the png kernel computes for
// one column of n <= 63 deltas (same source as the device path).  Lets the
// CPU tests check the selection without a GPU.
uint64_t fc_png_topm_mask_host(const float* delta, int n, int keep_m) {
  const int m = keep_m;
  if (n <= 0 || n > 63 || m <= 0) return 0;
  if (m >= n) return n == 64 ? ~0ull : ((uint64_t)1 << n) - 1;
  uint32_t keys[64];
  for (int i = 0; i < n; ++i) {
    uint32_t bits;
    __builtin_memcpy(&bits, &delta[i], 4);
    keys[i] = topm_key(bits);
  }
  return topm_mask_exact(keys, n, m);
}

}  // extern "C"
