// Split 0's prologue of a fused png decode step (fc_decode_step on png
// archives, dense or packed): the rows the step adds to the attention and
// the group's partial over them.  Used by the png matrix-core pass
// (fc_attn_png_kernel.h) and the packed png pass (fc_attn_pngpk.h).
#pragma once

#include "fc_attn_mfma_kernel.h"
#include "fc_topm.h"

namespace fc {

// Where one stream's completed block goes: its anchor row (stream dtype),
// its deltas (dense: r - 1 fp32 rows; packed: keep_m fp32 value rows) and,
// packed, its mask words (one per feature).
struct PngStepDst {
  void* anch;
  float* del;
  uint32_t* mask;
};

// The step's rows, in LDS as fp32 (xk, xv: n rows of D, n returned), from
// the stream's tail rows 0..t-1 (T, r rows of D per tail) and the new token:
//   * t + 1 < r: the tail rows and the token; the token is written to tail
//     row t when `write`.
//   * t + 1 == r: the block of tail rows 0..r-2 and the token is archived
//     as png_encode_kernel does (anchor = token 0, fp32 deltas x_{i+1} - x_i,
//     the Top-M mask of the keep_m largest |delta|; dense: the others
//     multiplied by 0; PACK: the kept steps are the mask's non-zero
//     survivors, then the lowest-index zero steps until keep_m, their values
//     in step order and one mask word of kept steps and the others' sign
//     bits), stored when `write`, and its rows are left as png_decode_kernel
//     rebuilds them (anchor + the fp64 running sum of the deltas, rounded to
//     fp32).
// RMAX >= r; every thread of the workgroup takes part.
template <int D, int RMAX, typename T, bool PACK>
__device__ __forceinline__ int png_step_rows(int64_t t, int r, T* ktail, T* vtail, const T* ktok,
                                             const T* vtok, bool write, PngStepDst kd,
                                             PngStepDst vd, int keep_m, int tid, float* xk,
                                             float* xv) {
  const bool complete = t + 1 == r;
  const int n = complete ? r : (int)t + 1;
  for (int x = tid; x < n * D; x += kMThreads) {
    const int i = x / D, d = x - i * D;
    xk[x] = to_f32(i < t ? ktail[i * D + d] : ktok[d]);
    xv[x] = to_f32(i < t ? vtail[i * D + d] : vtok[d]);
  }
  if (write && !complete)
    for (int d = tid; d < D; d += kMThreads) {
      ktail[t * D + d] = ktok[d];
      vtail[t * D + d] = vtok[d];
    }
  __syncthreads();
  if (!complete) return n;
  // one (stream, feature) per thread
  const int n1 = r - 1;
  for (int x = tid; x < 2 * D; x += kMThreads) {
    const int sv = x / D, d = x - sv * D;
    float* xs = sv ? xv : xk;
    const PngStepDst& dst = sv ? vd : kd;
    float dl[RMAX];
#pragma unroll
    for (int i = 0; i < RMAX; ++i)
      dl[i] = i < n1 ? xs[(i + 1) * D + d] - xs[i * D + d] : 0.f;
    uint32_t kept = 0;  // PACK: the kept steps
    if (PACK || (keep_m > 0 && keep_m < n1)) {
      uint32_t key[RMAX];
      uint32_t nzm = 0;
#pragma unroll
      for (int i = 0; i < RMAX; ++i) {
        key[i] = i < n1 ? topm_key(__float_as_uint(dl[i])) : 0u;
        if (key[i] != 0u) nzm |= 1u << i;
      }
      const uint32_t mask = (uint32_t)topm_mask<RMAX>(key, n1, keep_m);
      if constexpr (PACK) {
        kept = mask & nzm;
        int cnt = __builtin_popcount(kept);
#pragma unroll
        for (int i = 0; i < RMAX; ++i)
          if (i < n1 && !((nzm >> i) & 1u) && cnt < keep_m) {
            kept |= 1u << i;
            ++cnt;
          }
      }
#pragma unroll
      for (int i = 0; i < RMAX; ++i)
        if (i < n1 && !(((PACK ? kept : mask) >> i) & 1u)) dl[i] = dl[i] * 0.0f;
    }
    const float a = xs[d];
    if (write) {
      static_cast<T*>(dst.anch)[d] = from_f32<T>(a);  // token 0 itself (a holds a value of T)
      if constexpr (PACK) {
        uint32_t sg = 0;
#pragma unroll
        for (int i = 0; i < RMAX; ++i)
          if (i < n1 && !((kept >> i) & 1u)) sg |= (__float_as_uint(dl[i]) >> 31) << i;
        dst.mask[d] = kept | (sg << 16);
        uint32_t rem = kept;
        for (int j = 0; j < keep_m; ++j) {
          const int i = __builtin_ctz(rem);
          rem &= rem - 1u;
          float v = dl[0];
#pragma unroll
          for (int u = 1; u < RMAX; ++u) v = i == u ? dl[u] : v;
          dst.del[j * D + d] = v;
        }
      } else {
#pragma unroll
        for (int i = 0; i < RMAX; ++i)
          if (i < n1) dst.del[i * D + d] = dl[i];
      }
    }
    double run = 0.0;
#pragma unroll
    for (int i = 0; i < RMAX; ++i)
      if (i < n1) {
        run += (double)dl[i];
        xs[(i + 1) * D + d] = a + (float)run;
      }
  }
  __syncthreads();
  return n;
}

// The partial of the group's G heads over the n rows (xk, xv) at full
// precision, as raw_tail_partial_t (etl: 16 * FC_MAX_BLOCK floats of
// scratch; acc: G rows of D; tm, tl: per head).  The query rows (QT) are
// q + qb + (h0 + h) * q_sh.
template <int D, typename QT>
__device__ __forceinline__ void png_step_attend(int n, const QT* q, int64_t qb, int64_t q_sh,
                                                int64_t h0, int G, float scale_log2, int tid,
                                                const float* xk, const float* xv, float* etl,
                                                float* acc, float* tm, float* tl) {
  const int lane = tid & 63, wave = tid >> 6;
  {
    const int grp = tid >> 4, gl = tid & 15;
    for (int u = grp; u < G * n; u += kMThreads / 16) {
      const int h = u / n, i = u - h * n;
      const QT* qr = q + qb + (h0 + h) * q_sh + gl;
      float a = 0.f;
      for (int c = 0; c < D / 16; ++c)
        a = __builtin_fmaf(to_f32(qr[16 * c]), xk[i * D + gl + 16 * c], a);
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) a += __shfl_xor(a, m, 16);
      if (gl == 0) etl[h * FC_MAX_BLOCK + i] = a * scale_log2;
    }
  }
  __syncthreads();
  for (int h = wave; h < G; h += kWaves) {
    float mx = -INFINITY;
    for (int i = lane; i < n; i += 64) mx = fmaxf(mx, etl[h * FC_MAX_BLOCK + i]);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    float l = 0.f;
    for (int i = lane; i < n; i += 64) {
      const float e = __builtin_amdgcn_exp2f(etl[h * FC_MAX_BLOCK + i] - mx);
      etl[h * FC_MAX_BLOCK + i] = e;
      l += e;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) l += __shfl_xor(l, m, 64);
    if (lane == 0) {
      tm[h] = mx;
      tl[h] = l;
    }
  }
  __syncthreads();
  for (int x = tid; x < G * D; x += kMThreads) {
    const int h = x / D, d = x - h * D;
    float o = 0.f;
    for (int i = 0; i < n; ++i) o = __builtin_fmaf(etl[h * FC_MAX_BLOCK + i], xv[i * D + d], o);
    acc[h * D + d] = o;
  }
}

}  // namespace fc
