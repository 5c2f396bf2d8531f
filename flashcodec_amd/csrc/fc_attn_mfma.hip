// Split pass of the decode attention for int8 jpeg archives on gfx950 matrix
// cores.
//
// With G query heads per kv head, a block's work is a skinny GEMM: scores
// S = K_rows . Q^T (M = rows, N = heads, K-dim = features) and output
// O = W . V_rows (M = heads, N = features, K-dim = rows).  On the vector ALU
// that costs ~4 fp32 FMAs per code byte per head group — as much VALU time
// as the HBM time of the bytes — so both products run as
// v_mfma_f32_16x16x32_f16 and the VALU only converts codes and runs the
// softmax.
//
// Codes convert to f16 exactly: for a code byte b, u = b ^ 0x80 = b + 128;
// the f16 with bits 0x6400 | u is 1024 + u, and one packed f16 add of -1152
// (exact) leaves b.  Queries enter as f16 scaled by a per-head power of two
// (exact for fp16 queries, and for bf16 queries in the normal f16 range);
// output weights enter as f16 scaled by a per-workgroup power of two.
// Products are exact in fp32 and the matrix cores accumulate in fp32.
//
// Workgroup = 4 wavefronts = one (batch, kv head, split, group of <= 16 query
// heads).  Each wavefront owns a contiguous run of 32-row slabs of the split
// and walks it in passes of up to 128 rows:
//   scores: per 16-row tile, lane (q, m) holds row m, features
//      [q*D/4, (q+1)*D/4) (any relabelling of the feature axis shared by both
//      operands is allowed), DK products of 32 features; lane (q, c < G) gets
//      the scores of rows 4q..4q+3 for head c and parks them in LDS.
//   softmax: (block, head) pairs over all 64 lanes (head = lane % GP): r
//      logits from the s scores, the pass maximum per head, exponentials and
//      s output weights w_j = sum_p 2^(logit_p - m) A[p][j] times the V row
//      scale, stored as f16 in LDS.
//   values: per 32-row slab, lane (q, c) loads rows 8q..8q+7, bytes
//      [8c, 8c+8) (16 lanes cover a 128-byte row) and transposes the 8x8
//      byte tile in registers, so matrix-core instance e of the slab sees
//      feature 8c + e in column c.
// The four wavefronts combine their (max, sum, acc) in LDS and write one
// partial per (query head, split) for the merge kernel.
#include <hip/hip_runtime.h>

#include "fc_common.h"

namespace fc {

int check_launch();

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct MfmaArgs {
  const void* q;
  int q_dtype;
  int64_t q_sb, q_sh;
  const int8_t* kcodes;
  const float* kscales;
  const int8_t* vcodes;
  const float* vscales;
  int64_t kcap, vcap;
  const float* A;  // r x s
  int64_t Hkv, G, nb;
  int r;
  float scale_log2;
  int64_t blocks_per_split;
  int n_splits;
  float* pm;
  float* pl;
  float* pacc;
};

constexpr int kMThreads = 256;
constexpr int kWaves = kMThreads / 64;
constexpr int kPassRowsW = 128;        // rows per wavefront pass
constexpr int kSPad = kPassRowsW + 4;  // float stride of a score row in LDS
constexpr int kWPad = kPassRowsW + 8;  // half stride of a weight row in LDS

// Orders this wavefront's LDS writes before its later LDS reads (lanes of a
// wavefront exchange data through its private LDS region).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t f16x2_sub1152(uint32_t v) {
  half2_t h = __builtin_bit_cast(half2_t, v);
  const half2_t off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  h = h + off;
  return __builtin_bit_cast(uint32_t, h);
}

// four int8 codes (one dword, already xor 0x80808080) -> f16 pairs
// (codes 0, 1) and (codes 2, 3)
__device__ __forceinline__ void biased_to_f16(uint32_t u, uint32_t& lo, uint32_t& hi) {
  lo = f16x2_sub1152(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
  hi = f16x2_sub1152(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
}

__device__ __forceinline__ half8_t as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const u32x4_t v = {a, b, c, d};
  return __builtin_bit_cast(half8_t, v);
}

// exponent e with x * 2^-e in [2^(target-1), 2^target) for x > 0; 0 for x == 0
__device__ __forceinline__ int pow2_exp_for(float x, int target) {
  if (!(x > 0.f)) return 0;
  int e;
  frexpf(x, &e);
  return e - target;
}

template <int SROWS, int DK, int GP>
__global__ __launch_bounds__(kMThreads) void attn_split_i8_mfma(MfmaArgs p) {
  constexpr int D = 32 * DK;
  constexpr int DV = (D + 127) / 128;  // 128-feature groups of the value product
  // rows per wavefront pass: its K codes (NT tiles) and V codes (NS slabs)
  // are in flight while the previous stage computes
  constexpr int PR = D == 256 ? 32 : 64;
  constexpr int NT = PR / 16;
  constexpr int NS = PR / 32;
  constexpr int KDW = 2 * DK;  // K dwords per lane per tile
  __shared__ float s_lds[kWaves][16][kSPad];
  __shared__ _Float16 w_lds[kWaves][16][kWPad];
  __shared__ float sc_lds[kWaves][2][PR];  // K and V row scales of the pass
  __shared__ float comb[kWaves][16][3];

  const int split = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int64_t g0 = (int64_t)blockIdx.z * 16;
  const int64_t b = bh / p.Hkv, hkv = bh - b * p.Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lq = lane >> 4, lc = lane & 15;
  const int G = (int)min<int64_t>(16, p.G - g0);  // heads of this group (<= GP)
  const int r = p.r;

  const int64_t nb_begin = (int64_t)split * p.blocks_per_split;
  const int64_t nb_end = min(p.nb, nb_begin + p.blocks_per_split);
  const int64_t row_begin = nb_begin * SROWS, row_end = nb_end * SROWS;
  const int64_t nslab = (row_end - row_begin + 31) / 32;
  const int64_t spw = (nslab + kWaves - 1) / kWaves;
  const int64_t wrow0 = min(row_end, row_begin + (int64_t)wave * spw * 32);
  const int64_t wrow1 = min(row_end, wrow0 + spw * 32);
  const int64_t last_row = row_end - 1;  // every load address is clamped to <= last_row

  const int8_t* kbase = p.kcodes + bh * p.kcap * SROWS * D;
  const int8_t* vbase = p.vcodes + bh * p.vcap * SROWS * D;
  const float* ksc = p.kscales + bh * p.kcap * SROWS;
  const float* vsc = p.vscales + bh * p.vcap * SROWS;

  // ---- queries: B operand of the score product.  Lane (q, c): head c,
  // features q*D/4 + 8*kc + i of product kc, scaled per head by a power of two
  const bool hq_ok = lc < G;
  const int64_t hq = hkv * p.G + g0 + (hq_ok ? lc : 0);
  const uint16_t* qrow =
      static_cast<const uint16_t*>(p.q) + b * p.q_sb + hq * p.q_sh + lq * (D / 4);
  const bool q_f16 = p.q_dtype == FC_F16;
  float qf[DK][8];
  float qmax = 0.f;
  // dtype branch outside the loops; fp16 lanes are read through a half8 view
  // (hipcc 7.2 reused dword 0's conversion for all dwords when each dword was
  // bit-cast to half2 inside an unrolled loop)
#pragma unroll
  for (int kc = 0; kc < DK; ++kc) {
    const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(qrow + 8 * kc);
    if (q_f16) {
      const half8_t h = __builtin_bit_cast(half8_t, raw);
#pragma unroll
      for (int i = 0; i < 8; ++i) qf[kc][i] = (float)h[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qf[kc][2 * i] = __uint_as_float(raw[i] << 16);
        qf[kc][2 * i + 1] = __uint_as_float(raw[i] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qf[kc][i] = hq_ok ? qf[kc][i] : 0.f;
      qmax = fmaxf(qmax, fabsf(qf[kc][i]));
    }
  }
  qmax = fmaxf(qmax, __shfl_xor(qmax, 16, 64));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
  const int qe = pow2_exp_for(qmax, 14);
  half8_t qop[DK];
#pragma unroll
  for (int kc = 0; kc < DK; ++kc)
#pragma unroll
    for (int i = 0; i < 8; ++i) qop[kc][i] = (_Float16)ldexpf(qf[kc][i], -qe);
  const float head_mul = ldexpf(p.scale_log2, qe);  // raw score -> base-2 logit / K scale

  float4_t acc[DV][8];
#pragma unroll
  for (int dv = 0; dv < DV; ++dv)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[dv][e] = (float4_t){0.f, 0.f, 0.f, 0.f};
  // running max / sum of head (lane % GP), identical in all lanes of a head;
  // the accumulators hold acc * 2^-sig_run
  const int myh = lane % GP;
  float m_run = -INFINITY, l_run = 0.f;
  int sig_run = -1000;

  // ---- loads of one pass (addresses clamped in range; values masked later)
  uint32_t kr[NT][KDW];
  float ks_r, vs_r;
  auto load_k = [&](int64_t pr0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t row = min(pr0 + 16 * t + lc, last_row);
      const int8_t* src = kbase + row * D + lq * (D / 4);
#pragma unroll
      for (int h = 0; h < DK / 2; ++h) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(src + 16 * h);
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[t][4 * h + i] = v[i];
      }
      if constexpr (DK & 1) {
        const u32x2_t v = *reinterpret_cast<const u32x2_t*>(src + 16 * (DK / 2));
        kr[t][KDW - 2] = v[0];
        kr[t][KDW - 1] = v[1];
      }
    }
    const int64_t srow = min(pr0 + (lane % PR), last_row);
    ks_r = ksc[srow];
    vs_r = vsc[srow];
  };
  uint32_t vr[NS][DV][16];
  auto load_v = [&](int64_t pr0) {
#pragma unroll
    for (int sl = 0; sl < NS; ++sl)
#pragma unroll
      for (int dv = 0; dv < DV; ++dv) {
        const int dcol = min(128 * dv + 8 * lc, D - 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int64_t row = min(pr0 + 32 * sl + 8 * lq + i, last_row);
          const u32x2_t v = *reinterpret_cast<const u32x2_t*>(vbase + row * D + dcol);
          vr[sl][dv][2 * i] = v[0];
          vr[sl][dv][2 * i + 1] = v[1];
        }
      }
  };

  if (wrow0 < wrow1) load_k(wrow0);
  for (int64_t pr0 = wrow0; pr0 < wrow1; pr0 += PR) {
    const int prow = (int)min<int64_t>(PR, wrow1 - pr0);  // multiple of SROWS
    const int rend = ((prow + 31) / 32) * 32;
    load_v(pr0);

    // ------------------------------------------------------------ scores
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool ok = 16 * t + lc < prow;
      float4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < DK; ++kc) {
        uint32_t a0, a1, a2, a3;
        biased_to_f16((ok ? kr[t][2 * kc] : 0u) ^ 0x80808080u, a0, a1);
        biased_to_f16((ok ? kr[t][2 * kc + 1] : 0u) ^ 0x80808080u, a2, a3);
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(a0, a1, a2, a3), qop[kc], sacc,
                                                      0, 0, 0);
      }
      if (lc < G) {
        const float4_t sv = sacc * head_mul;
        *reinterpret_cast<float4_t*>(&s_lds[wave][lc][16 * t + 4 * lq]) = sv;
      }
    }
    if (lane < PR) {
      sc_lds[wave][0][lane] = ks_r;
      sc_lds[wave][1][lane] = vs_r;
    }
    // V row scale exponent of this pass
    float smax = lane < prow ? vs_r : 0.f;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) smax = fmaxf(smax, __shfl_xor(smax, m, 64));
    const int sig_new = max(sig_run, pow2_exp_for(smax, 1));
    const float wmul = ldexpf(1.0f, -sig_new);
    // next pass's K codes and scales fly during the softmax and value stages
    if (pr0 + PR < wrow1) load_k(pr0 + PR);
    wave_lds_sync();

    // ------------------------------------------------------------ softmax
    const int nblk = prow / SROWS;
    const int npair = nblk * GP;
    float pmax = -INFINITY;
    for (int u = lane; u < npair; u += 64) {
      const int bl = u / GP;
      if (myh >= G) continue;
      float sv[SROWS];
#pragma unroll
      for (int j = 0; j < SROWS; ++j)
        sv[j] = s_lds[wave][myh][bl * SROWS + j] * sc_lds[wave][0][bl * SROWS + j];
      for (int t = 0; t < r; ++t) {
        float lg = 0.f;
#pragma unroll
        for (int j = 0; j < SROWS; ++j) lg = __builtin_fmaf(p.A[t * SROWS + j], sv[j], lg);
        pmax = fmaxf(pmax, lg);
      }
    }
#pragma unroll
    for (int m = GP; m < 64; m <<= 1) pmax = fmaxf(pmax, __shfl_xor(pmax, m, 64));
    const float m_new = fmaxf(m_run, pmax);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first pass
    m_run = m_new;
    float lsum = 0.f;
    for (int u = lane; u < npair; u += 64) {
      const int bl = u / GP;
      if (myh >= G) continue;
      float sv[SROWS], w[SROWS];
#pragma unroll
      for (int j = 0; j < SROWS; ++j) {
        sv[j] = s_lds[wave][myh][bl * SROWS + j] * sc_lds[wave][0][bl * SROWS + j];
        w[j] = 0.f;
      }
      for (int t = 0; t < r; ++t) {
        float lg = 0.f;
#pragma unroll
        for (int j = 0; j < SROWS; ++j) lg = __builtin_fmaf(p.A[t * SROWS + j], sv[j], lg);
        const float e = __builtin_amdgcn_exp2f(lg - m_new);
        lsum += e;
#pragma unroll
        for (int j = 0; j < SROWS; ++j) w[j] = __builtin_fmaf(e, p.A[t * SROWS + j], w[j]);
      }
#pragma unroll
      for (int j = 0; j < SROWS; ++j)
        w_lds[wave][myh][bl * SROWS + j] =
            (_Float16)(w[j] * (sc_lds[wave][1][bl * SROWS + j] * wmul));
    }
    // rows past the pass end inside the last slab carry zero weight
    if (prow < rend)
      for (int i = prow + lane; i < rend; i += 64)
        for (int h = 0; h < G; ++h) w_lds[wave][h][i] = (_Float16)0.f;
#pragma unroll
    for (int m = GP; m < 64; m <<= 1) lsum += __shfl_xor(lsum, m, 64);
    l_run = l_run * alpha + lsum;
    // rescale the accumulators: lane (q, c) register i holds head 4q + i
    const float sfix = ldexpf(1.0f, max(sig_run - sig_new, -126));
    sig_run = sig_new;
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * lq + i, 64) * sfix;
#pragma unroll
    for (int dv = 0; dv < DV; ++dv)
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[dv][e][i] *= al[i];
    wave_lds_sync();

    // ------------------------------------------------------------ values
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
      if (32 * sl >= rend) continue;
      u32x4_t wa = *reinterpret_cast<const u32x4_t*>(&w_lds[wave][lc][32 * sl + 8 * lq]);
      if (lc >= G) wa = (u32x4_t){0u, 0u, 0u, 0u};
      const half8_t wop = __builtin_bit_cast(half8_t, wa);
#pragma unroll
      for (int dv = 0; dv < DV; ++dv) {
        const bool dok = 128 * dv + 8 * lc < D;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          // row pair (a, b) = (2pp, 2pp+1): t0 = [a0 b0 a1 b1], t1 = [a2 b2 a3 b3]
          uint32_t t0[4], t1[4];
#pragma unroll
          for (int pp = 0; pp < 4; ++pp) {
            const bool oka = dok && 32 * sl + 8 * lq + 2 * pp < prow;
            const bool okb = dok && 32 * sl + 8 * lq + 2 * pp + 1 < prow;
            const uint32_t ra = (oka ? vr[sl][dv][2 * (2 * pp) + hh] : 0u) ^ 0x80808080u;
            const uint32_t rb = (okb ? vr[sl][dv][2 * (2 * pp + 1) + hh] : 0u) ^ 0x80808080u;
            t0[pp] = __builtin_amdgcn_perm(rb, ra, 0x05010400u);
            t1[pp] = __builtin_amdgcn_perm(rb, ra, 0x07030602u);
          }
#pragma unroll
          for (int ee = 0; ee < 4; ++ee) {
            uint32_t o[4];
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const uint32_t src = ee < 2 ? t0[pp] : t1[pp];
              const uint32_t sel = (ee & 1) ? 0x04030402u : 0x04010400u;
              o[pp] = f16x2_sub1152(__builtin_amdgcn_perm(0x64646464u, src, sel));
            }
            const int e = 4 * hh + ee;
            acc[dv][e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                wop, as_half8(o[0], o[1], o[2], o[3]), acc[dv][e], 0, 0, 0);
          }
        }
      }
    }
    wave_lds_sync();
  }

  // ---- combine the wavefronts.  Lane c < GP carries head c's (max, sum);
  // each wave's accumulators carry a factor 2^-sig_run.
  if (lane < GP) {
    comb[wave][lane][0] = m_run;
    comb[wave][lane][1] = l_run;
    comb[wave][lane][2] = ldexpf(1.0f, max(sig_run, -126));
  }
  float* obuf = &s_lds[0][0][0];  // [wave*4 + i][D] for the 4 heads of a lane group
  for (int h0 = 0; h0 < G; h0 += 4) {
    __syncthreads();
    if (lq == h0 / 4) {
#pragma unroll
      for (int dv = 0; dv < DV; ++dv)
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int d = 128 * dv + 8 * lc + e;
            if (d < D) obuf[(wave * 4 + i) * D + d] = acc[dv][e][i];
          }
    }
    __syncthreads();
    for (int x = tid; x < 4 * D; x += kMThreads) {
      const int i = x / D, d = x - i * D;
      const int h = h0 + i;
      if (h >= G) continue;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, comb[w][h][0]);
      float o = 0.f, l = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float mw = comb[w][h][0];
        const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        o = __builtin_fmaf(f * comb[w][h][2], obuf[(w * 4 + i) * D + d], o);
        l = __builtin_fmaf(f, comb[w][h][1], l);
      }
      const int64_t bq = b * (p.Hkv * p.G) + hkv * p.G + g0 + h;
      const int64_t slot = bq * p.n_splits + split;
      p.pacc[slot * D + d] = o;
      if (d == 0) {
        p.pm[slot] = M;
        p.pl[slot] = l;
      }
    }
  }
}

template <int... Vs, typename F>
int mfma_with_int(int v, F&& f) {
  int rc = FC_ERR_UNSUPPORTED;
  bool hit = false;
  ((v == Vs ? (rc = f(std::integral_constant<int, Vs>{}), hit = true) : false), ...);
  return hit ? rc : FC_ERR_UNSUPPORTED;
}

// Whether the matrix-core split pass handles this configuration.
// The pass reads 16 query bytes and 16 code bytes per load: the query rows
// and both code stores must be 16-byte aligned.
bool split_i8_mfma_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                             int s, const fc_stream_view* key, const fc_stream_view* value) {
  const auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  return (q_dtype == FC_F16 || q_dtype == FC_BF16) && (D == 64 || D == 128 || D == 256) &&
         (s == 1 || s == 2 || s == 4) && al16(q) && q_sb % 8 == 0 && q_sh % 8 == 0 &&
         al16(key->rows) && al16(value->rows);
}

int launch_split_i8_mfma(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t D, int r, int s, int64_t nb,
                         const fc_stream_view* key, const fc_stream_view* value, const float* A,
                         float scale_log2, float* pm, float* pl, float* pacc, int n_splits,
                         hipStream_t st) {
  MfmaArgs a;
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.kcodes = static_cast<const int8_t*>(key->rows);
  a.kscales = key->scales;
  a.vcodes = static_cast<const int8_t*>(value->rows);
  a.vscales = value->scales;
  a.kcap = key->cap;
  a.vcap = value->cap;
  a.A = A;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.nb = nb;
  a.r = r;
  a.scale_log2 = scale_log2;
  a.blocks_per_split = (nb + n_splits - 1) / n_splits;
  a.n_splits = n_splits;
  a.pm = pm;
  a.pl = pl;
  a.pacc = pacc;
  const int64_t G = Hq / Hkv;
  const int gg = (int)std::min<int64_t>(G, 16);
  const int gp = gg <= 1 ? 1 : gg <= 2 ? 2 : gg <= 4 ? 4 : gg <= 8 ? 8 : 16;
  const dim3 grid((unsigned)n_splits, (unsigned)(B * Hkv), (unsigned)((G + 15) / 16));
  const int rc = mfma_with_int<1, 2, 4>(s, [&](auto sc) {
    constexpr int SR = decltype(sc)::value;
    return mfma_with_int<2, 4, 8>((int)(D / 32), [&](auto dc) {
      constexpr int DKv = decltype(dc)::value;
      return mfma_with_int<1, 2, 4, 8, 16>(gp, [&](auto gc) {
        constexpr int GPv = decltype(gc)::value;
        attn_split_i8_mfma<SR, DKv, GPv><<<grid, kMThreads, 0, st>>>(a);
        return FC_OK;
      });
    });
  });
  if (rc != FC_OK) return rc;
  return check_launch();
}

}  // namespace fc
