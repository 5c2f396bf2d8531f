// Materialisation-free decode attention over a codec archive (gfx950).
//
// For one query token per sequence and an archive whose blocks store s rows
// S (s x D) with synthesis matrix A (r x s) — jpeg: A = M^T, png:
// A = tril(1) over (anchor, deltas) — the r tokens of a block are A S, so
//   logit[p] = scale * sum_j A[p][j] * (q . S_j)
//   out     += sum_j (sum_p prob[p] A[p][j]) * S_j
// (flashcodec/attention.py:1-22, 101-140).
//
// Kernel 1 (split): grid (split, batch*kv_head, query-head group).  A
// workgroup owns a contiguous range of blocks of one kv head and up to GM
// query heads of its group, so every archived row is read from HBM once per
// group of GM query heads (the reference's Triton kernel reads it once per
// query head).  The range is walked in passes of up to kPassRows rows:
//   A. scores: row tasks are spread over the workgroup, LPR lanes per row
//      with VEC features each; partial dots are reduced across the LPR
//      lanes (DPP inside 16-lane rows, shuffles beyond) and the per-row
//      int8 scale is applied once to the reduced dot;
//   B. softmax: every (block, head) pair turns its s scores into r logits
//      (base-2 domain, scale*log2(e) folded in), the pass maximum updates
//      the running maximum, and the pair writes its s output weights
//      w_j = sum_p 2^(logit_p - m) A[p][j] (times the V row scale) back in
//      place of its scores (png with r <= 16: one pair per 16-lane row,
//      DPP prefix / suffix sums); the first V rows are already requested;
//   C. values: the same row tasks accumulate acc[g][d] += w_j * S_j[d].
// The partial (m, l, acc[D]) of each (query head, split) goes to the
// workspace.  With the merge fused (fc_decode_attention), split 0 starts
// from the raw tail tokens (attended at full precision), and the last
// workgroup of each (batch, kv head, head group) to publish its partial
// combines all of them into out = acc / l in the query dtype.
// Kernel 2 (merge, for the two-pass entry points): one workgroup per query
// head combines the split partials with the raw tail tokens.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <type_traits>

#include "fc_attn_internal.h"
#include "fc_common.h"

namespace fc {

// Split pass selection: read from the environment once, when the library is
// loaded (FLASHCODEC_AMD_ATTN=valu forces the vector-ALU split pass, for A/B
// measurements), never on the call path.
static int g_attention_pass = [] {
  const char* v = getenv("FLASHCODEC_AMD_ATTN");
  return (v && v[0] == 'v') ? FC_PASS_VECTOR : FC_PASS_AUTO;
}();

bool mfma_split_allowed() { return g_attention_pass != FC_PASS_VECTOR; }
bool static_pass_order() { return g_attention_pass == FC_PASS_STATIC; }

constexpr int kAttnThreads = 256;
constexpr int kPassRows = 512;
constexpr int kMaxSplits = 256;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const void* q;
  int q_dtype;
  int64_t q_sb, q_sh;
  const void* krows;
  const float* kscales;
  const void* kanch;
  int64_t kcap;
  const void* vrows;
  const float* vscales;
  const void* vanch;
  int64_t vcap;
  const float* A;  // r x s
  int64_t Hkv, G, D, nb;
  int r, s;
  float scale_log2;  // attention scale * log2(e)
  int lpr_log2;
  int64_t blocks_per_split;
  int n_splits;
  float* pm;
  float* pl;
  float* pacc;
  // Fused merge (arrive != NULL): split 0 folds the raw tail into its
  // partial, every workgroup publishes its partial and counts its arrival
  // in its group's word (arrive + group * cstride, zero between calls), and
  // the last workgroup of the group merges the partials into `out`.
  // Otherwise n_raw is 0 here and the merge kernel runs afterwards.
  unsigned int* arrive;
  int64_t cstride;
  const void* kraw;
  const void* vraw;
  int raw_dtype;
  int64_t kr_sb, kr_sh, kr_st, vr_sb, vr_sh, vr_st;
  int64_t n_raw;
  void* out;
  int64_t o_sb, o_sh;
  // device (n_blocks, n_tail) before a decode step's token, or NULL: the
  // kernel then takes nb, the tail length and the split ranges from it
  const int64_t* state;
};

// v + (v from the lane selected by a DPP pattern); patterns stay inside a
// 16-lane row.
#define FC_DPP_ADD(v, CTRL)                                                          \
  ((v) + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (CTRL), 0xf, \
                                                    0xf, false)))

// Sum over aligned groups of `lpr` lanes (power of two <= 64); every lane of
// the group receives the group sum.
__device__ __forceinline__ float row_sum(float v, int lpr) {
  if (lpr >= 2) v = FC_DPP_ADD(v, 0xB1);   // quad_perm [1,0,3,2]
  if (lpr >= 4) v = FC_DPP_ADD(v, 0x4E);   // quad_perm [2,3,0,1]
  if (lpr >= 8) v = FC_DPP_ADD(v, 0x141);  // row_half_mirror
  if (lpr >= 16) v = FC_DPP_ADD(v, 0x140); // row_mirror
  if (lpr >= 32) v += __shfl_xor(v, 16, 64);
  if (lpr >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// DPP lane v + (v from `n` lanes below / above inside the 16-lane row;
// lanes without a source add 0)
#define FC_DPP_SHR(v, n) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + (n), 0xf, 0xf, true))
#define FC_DPP_SHL(v, n) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + (n), 0xf, 0xf, true))

// Inclusive prefix sum (lane t: sum of lanes <= t) and suffix sum (lane t:
// sum of lanes >= t) inside each 16-lane row.
__device__ __forceinline__ float row16_prefix(float v) {
  v += FC_DPP_SHR(v, 1);
  v += FC_DPP_SHR(v, 2);
  v += FC_DPP_SHR(v, 4);
  v += FC_DPP_SHR(v, 8);
  return v;
}
__device__ __forceinline__ float row16_suffix(float v) {
  v += FC_DPP_SHL(v, 1);
  v += FC_DPP_SHL(v, 2);
  v += FC_DPP_SHL(v, 4);
  v += FC_DPP_SHL(v, 8);
  return v;
}
// Maximum over the 16-lane row, in every lane of it.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false)));
  return v;
}

// Row `j` of block `n` of sequence `bh`, VEC features from d0, as fp32.
// Returns the row's scale (int8 stores) or 1.
template <typename TS, int KIND, int VEC>
__device__ __forceinline__ float load_row(const void* rows, const float* scales,
                                          const void* anch, int64_t cap, int64_t bh,
                                          int64_t n, int j, int s, int r, int64_t D,
                                          int64_t d0, bool dact, float (&x)[VEC]) {
  if (!dact) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = 0.f;
    return 1.f;
  }
  if constexpr (KIND == FC_STORE_JPEG_I8) {
    const int64_t row = (bh * cap + n) * s + j;
    load_f32<int8_t, VEC>(static_cast<const int8_t*>(rows) + row * D + d0, x);
    return scales[row];
  } else if constexpr (KIND == FC_STORE_JPEG_I8G) {
    // one scale per 32 features: the lane's VEC features share one, applied here
    const int64_t row = (bh * cap + n) * s + j;
    load_f32<int8_t, VEC>(static_cast<const int8_t*>(rows) + row * D + d0, x);
    const float sg = scales[row * (D / 32) + d0 / 32];
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] *= sg;
    return 1.f;
  } else if constexpr (KIND == FC_STORE_JPEG_FP) {
    const int64_t row = (bh * cap + n) * s + j;
    load_f32<TS, VEC>(static_cast<const TS*>(rows) + row * D + d0, x);
    return 1.f;
  } else {
    if (j == 0) {
      load_f32<TS, VEC>(static_cast<const TS*>(anch) + (bh * cap + n) * D + d0, x);
    } else {
      const int64_t row = (bh * cap + n) * (r - 1) + (j - 1);
      load_f32<float, VEC>(static_cast<const float*>(rows) + row * D + d0, x);
    }
    return 1.f;
  }
}

template <int GM>
__device__ __forceinline__ void wg_reduce(float (&v)[GM], float* red, bool is_max) {
  // v[g] is this thread's partial for head g; threads of a wavefront first
  // combine lane-wise, then the four wavefronts through LDS.  Every thread
  // ends with the workgroup result.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    float x = v[g];
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const float y = __shfl_xor(x, m, 64);
      x = is_max ? fmaxf(x, y) : x + y;
    }
    if (lane == 0) red[wave * GM + g] = x;
  }
  // LDS-only barriers: the V rows the pass requested before its softmax stay
  // in flight through the reductions
  lds_barrier();
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    float x = red[g];
#pragma unroll
    for (int w = 1; w < kAttnThreads / 64; ++w)
      x = is_max ? fmaxf(x, red[w * GM + g]) : x + red[w * GM + g];
    v[g] = x;
  }
  lds_barrier();
}


// ---- per-(block, head) softmax pieces.  `sc` points at the pair's s
// scores in LDS (stride `st`); logits live in the base-2 domain.
// SREG: s <= 8, scores and weights held in registers.

template <int KIND, bool SREG>
__device__ __forceinline__ float pair_max(const float* sc, int st, const float* A, int r, int s,
                                          float sl2) {
  float mx = -INFINITY;
  if constexpr (KIND == FC_STORE_PNG) {
    // A = tril(1): logit_t = prefix sum of the scores
    float run = 0.f;
    for (int t = 0; t < r; ++t) {
      run += sc[t * st];
      mx = fmaxf(mx, run * sl2);
    }
  } else if constexpr (SREG) {
    float sv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) sv[j] = j < s ? sc[j * st] : 0.f;
    for (int t = 0; t < r; ++t) {
      float lg = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < s) lg = __builtin_fmaf(A[t * s + j], sv[j], lg);
      mx = fmaxf(mx, lg * sl2);
    }
  } else {
    for (int t = 0; t < r; ++t) {
      float lg = 0.f;
      for (int j = 0; j < s; ++j) lg = __builtin_fmaf(A[t * s + j], sc[j * st], lg);
      mx = fmaxf(mx, lg * sl2);
    }
  }
  return mx;
}

// Writes the pair's output weights w_j (times the V row scale when `vsc` is
// given) over its scores (png, SREG) or to `wo` (generic s), and returns
// sum_t 2^(logit_t - m).
template <int KIND, bool SREG>
__device__ __forceinline__ float pair_weights(float* sc, float* wo, int st, const float* A, int r,
                                              int s, float sl2, float m, const float* vsc) {
  float es = 0.f;
  if constexpr (KIND == FC_STORE_PNG) {
    float run = 0.f;
    for (int t = 0; t < r; ++t) {
      run += sc[t * st];
      const float e = __builtin_amdgcn_exp2f(run * sl2 - m);
      es += e;
      sc[t * st] = e;
    }
    // w_j = sum_{t >= j} e_t
    float suf = 0.f;
    for (int j = r - 1; j >= 0; --j) {
      suf += sc[j * st];
      sc[j * st] = suf;
    }
  } else if constexpr (SREG) {
    float sv[8], w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sv[j] = j < s ? sc[j * st] : 0.f;
      w[j] = 0.f;
    }
    for (int t = 0; t < r; ++t) {
      float lg = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < s) lg = __builtin_fmaf(A[t * s + j], sv[j], lg);
      const float e = __builtin_amdgcn_exp2f(lg * sl2 - m);
      es += e;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < s) w[j] = __builtin_fmaf(e, A[t * s + j], w[j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < s) sc[j * st] = vsc ? w[j] * vsc[j] : w[j];
  } else {
    // generic s: weights go to a separate LDS region `wo`; token weights are
    // recomputed for every stored row
    for (int t = 0; t < r; ++t) {
      float lg = 0.f;
      for (int i = 0; i < s; ++i) lg = __builtin_fmaf(A[t * s + i], sc[i * st], lg);
      es += __builtin_amdgcn_exp2f(lg * sl2 - m);
    }
    for (int j = 0; j < s; ++j) {
      float wj = 0.f;
      for (int t = 0; t < r; ++t) {
        float lg = 0.f;
        for (int i = 0; i < s; ++i) lg = __builtin_fmaf(A[t * s + i], sc[i * st], lg);
        wj = __builtin_fmaf(__builtin_amdgcn_exp2f(lg * sl2 - m), A[t * s + j], wj);
      }
      wo[j * st] = vsc ? wj * vsc[j] : wj;
    }
  }
  return es;
}

// Merge of one (batch, kv head, group of ng <= GM query heads) by the last
// workgroup of the split pass to finish it: out = sum_s w_s acc_s /
// sum_s w_s l_s over the n_splits published partials, w_s = 2^(m_s - max m)
// (the raw tail is part of split 0's partial).  Partials and statistics are
// read with device-scope loads.  Each output task (head, 4 features) is
// shared by nsub adjacent lanes that take every nsub-th split, kPre partial
// loads per lane in flight at a time; the first sweep's first loads are
// requested together with the statistics, so a merge of up to kPre * nsub
// splits per task costs one round trip.  `lds` holds >= 2 * GM * kMaxSplits
// floats.
template <int GM>
__device__ void merge_group(const AttnArgs& p, int64_t b, int64_t hkv, int64_t g0, int ng, int tid,
                            float* lds) {
  constexpr int kPre = GM >= 4 ? 24 : 8;  // fewer heads: more lanes per task
  const int ns = p.n_splits;
  const int D = (int)p.D, C4 = D / 4;
  const int64_t bq0 = b * (p.Hkv * p.G) + hkv * p.G + g0;
  float* const wsp = lds;                    // [ng][ns] split maxima
  float* const plv = lds + GM * kMaxSplits;  // [ng][ns] split sums
  const __amdgpu_buffer_rsrc_t rp = buf_rsrc(p.pacc + bq0 * ns * D, ng * ns * D * 4);
  const __amdgpu_buffer_rsrc_t rm = buf_rsrc(p.pm + bq0 * ns, ng * ns * 4);
  const __amdgpu_buffer_rsrc_t rl = buf_rsrc(p.pl + bq0 * ns, ng * ns * 4);
  const int ntask = ng * C4;
  int lsub = 0;  // nsub = 2^lsub lanes per task, up to 16
  while (lsub < 4 && (ntask << (lsub + 1)) <= kAttnThreads) ++lsub;
  const int nsub = 1 << lsub;
  const int sub = tid & (nsub - 1);
  float4_t pre[kPre];
  auto fetch = [&](bool act, int h, int c, int sp0) {
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      const int sp = sp0 + j * nsub;
      pre[j] = (act && sp < ns)
                   ? __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rp, ((h * ns + sp) * C4 + c) * 16, 0,
                                                      kCachePolicySc1))
                   : (float4_t){0.f, 0.f, 0.f, 0.f};
    }
  };
  {
    const int task = tid >> lsub;
    const bool act = task < ntask;
    const int h = act ? task / C4 : 0;
    fetch(act, h, act ? task - h * C4 : 0, sub);
  }
  for (int u = tid; u < ng * ns; u += kAttnThreads) {
    wsp[u] = __builtin_bit_cast(float,
                                __builtin_amdgcn_raw_buffer_load_b32(rm, u * 4, 0, kCachePolicySc1));
    plv[u] = __builtin_bit_cast(float,
                                __builtin_amdgcn_raw_buffer_load_b32(rl, u * 4, 0, kCachePolicySc1));
  }
  __syncthreads();
  for (int t0 = 0; t0 < ntask; t0 += kAttnThreads >> lsub) {  // uniform trip count
    const int task = t0 + (tid >> lsub);
    const bool act = task < ntask;
    const int h = act ? task / C4 : 0, c = act ? task - h * C4 : 0;
    const float* wh = wsp + h * ns;
    const float* lh = plv + h * ns;
    float mx = -INFINITY;
    for (int sp = 0; sp < ns; ++sp) mx = fmaxf(mx, wh[sp]);
    float l = 0.f;
    float4_t o = {0.f, 0.f, 0.f, 0.f};
    for (int sp0 = sub; sp0 < ns; sp0 += kPre * nsub) {
      if (t0 > 0 || sp0 > sub) fetch(act, h, c, sp0);
#pragma unroll
      for (int j = 0; j < kPre; ++j) {
        const int sp = sp0 + j * nsub;
        if (sp < ns) {
          const float w = wh[sp] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(wh[sp] - mx);
          l = __builtin_fmaf(w, lh[sp], l);
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = __builtin_fmaf(w, pre[j][i], o[i]);
        }
      }
    }
    for (int m = 1; m < nsub; m <<= 1) {
      l += __shfl_xor(l, m, 64);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] += __shfl_xor(o[i], m, 64);
    }
    if (act && sub == 0) {
      const float iv = 1.0f / l;
      const int64_t ob = b * p.o_sb + (hkv * p.G + g0 + h) * p.o_sh + 4 * c;
#pragma unroll
      for (int i = 0; i < 4; ++i) store_any(p.out, p.q_dtype, ob + i, o[i] * iv);
    }
  }
}

// 3 waves per SIMD (12 per CU, 3 workgroups) up to 4 heads per workgroup,
// except the 16-bit png variants, which would spill at that register budget
template <typename TS, int KIND, bool SREG, int VEC, int GM>
constexpr int split_waves_per_eu() {
  return (GM >= 8 || (KIND == FC_STORE_PNG && sizeof(TS) == 2)) ? 2 : 3;
}

template <typename TS, int KIND, bool SREG, int VEC, int GM>
__global__ __launch_bounds__(kAttnThreads)
__attribute__((amdgpu_waves_per_eu(split_waves_per_eu<TS, KIND, SREG, VEC, GM>())))
void attn_split_kernel(AttnArgs p) {
  // scores, then weights, per (row, head); the generic-s variant keeps the
  // weights in a second region
  constexpr int kSwRegions = (KIND != FC_STORE_PNG && !SREG) ? 2 : 1;
  // rows whose loads one thread keeps in flight (fewer at 8 heads per
  // workgroup, whose accumulators already hold most registers)
  constexpr int kRB = GM >= 8 ? 2 : 4;
  // layout: block nl of the pass at nl * bst, row j of it at + j * GM, head
  // g at + g.  The block stride bst = (s | 1) * GM is an odd multiple of GM,
  // so the (block, head) pairs of phase B, which read their blocks' rows in
  // lockstep, fall in different LDS banks.  A pass of floor(kPassRows / s)
  // blocks then spans at most 1.5 * kPassRows * GM floats (at s = 2).
  constexpr int kRegion = kPassRows * GM * 3 / 2;
  static_assert(kRegion * kSwRegions >= 2 * GM * kMaxSplits, "merge statistics fit the region");
  static_assert(kRegion * kSwRegions >= 2 * 64 * GM, "tail logits fit the region");
  __shared__ float sw[kRegion * kSwRegions];
  float* const wts = sw + (kSwRegions - 1) * kRegion;
  __shared__ float red[(kAttnThreads / 64) * GM];
  __shared__ float qs[GM * FC_MAX_HEAD_DIM];

  const int split = blockIdx.x;
  const int64_t bh = blockIdx.y;  // b * Hkv + hkv
  const int64_t g0 = (int64_t)blockIdx.z * GM;
  const int64_t b = bh / p.Hkv, hkv = bh - b * p.Hkv;
  const int tid = threadIdx.x;
  const int lpr = 1 << p.lpr_log2;
  const int nslot = kAttnThreads >> p.lpr_log2;
  const int slot = tid >> p.lpr_log2;
  const int lir = tid & (lpr - 1);
  const int64_t d0 = (int64_t)lir * VEC;
  const bool dact = d0 < p.D;
  const int s = p.s, r = p.r;

  // query heads of this group, as fp32, for this lane's features.  Every
  // workgroup of a kv head reads the same few query rows, so the workgroup
  // stages them in LDS with one coalesced pass instead of letting each lane
  // fetch its own features (which crowds the L2 lines that hold them).
  {
    const int64_t qb = b * p.q_sb + (hkv * p.G + g0) * p.q_sh;
    for (int64_t i = tid; i < GM * p.D; i += kAttnThreads) {
      const int64_t g = i / p.D, d = i - g * p.D;
      qs[i] = (g0 + g) < p.G ? load_q(p.q, p.q_dtype, qb + g * p.q_sh + d) : 0.f;
    }
  }
  __syncthreads();
  float qv[GM][VEC];
#pragma unroll
  for (int g = 0; g < GM; ++g)
#pragma unroll
    for (int v = 0; v < VEC; ++v) qv[g][v] = dact ? qs[g * p.D + d0 + v] : 0.f;

  float acc[GM][VEC];
#pragma unroll
  for (int g = 0; g < GM; ++g)
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[g][v] = 0.f;
  float m_run[GM], l_run[GM];
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
  }

  // block and tail counts: the arguments, or the decode-step state on the
  // device (tail after the step's token: t = n_tail + 1 tokens, archived as
  // block n_blocks when t == r; clamped to the archive capacity)
  int64_t nb = p.nb, n_raw = p.n_raw, bps = p.blocks_per_split;
  if (p.state) {
    const int64_t t = min(max(p.state[1], (int64_t)0), (int64_t)(r - 1)) + 1;
    nb = min(max(p.state[0], (int64_t)0) + (t == r ? 1 : 0), min(p.kcap, p.vcap));
    n_raw = t == r ? 0 : t;
    bps = (nb + p.n_splits - 1) / p.n_splits;  // trailing splits may be empty
  }

  // ---- raw tail (fused merge only): split 0 starts its partial with the
  // n_raw <= FC_MAX_BLOCK tail tokens at full precision
  if (split == 0 && n_raw > 0) {
    const int nt = (int)n_raw;
    const int lane = tid & 63;
    float* const tsc = sw;            // [nt][GM] base-2 logits
    float* const tex = sw + 64 * GM;  // [nt][GM] exponentials
    // VEC elements from d0 of tail row t (row 0 for lanes without one: a
    // valid address whose values are dropped), all loads in flight together.
    // The tail is in the stream dtype, which is TS except for int8 archives.
    auto raw_row = [&](const void* base, int64_t off0, int64_t st, int t, bool ok,
                       float (&x)[VEC]) {
      const int64_t off = ok ? off0 + t * st + d0 : off0;
      const int dt = (KIND == FC_STORE_JPEG_I8 || KIND == FC_STORE_JPEG_I8G) ? p.raw_dtype
                     : std::is_same_v<TS, f16_t> ? FC_F16
                     : std::is_same_v<TS, bf16_t> ? FC_BF16 : FC_F32;
      switch (dt) {
        case FC_F16: {
          const f16_t* ptr = static_cast<const f16_t*>(base) + off;
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[v] = to_f32(ptr[ok ? v : 0]);
        } break;
        case FC_BF16: {
          const bf16_t* ptr = static_cast<const bf16_t*>(base) + off;
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[v] = to_f32(ptr[ok ? v : 0]);
        } break;
        default: {
          const float* ptr = static_cast<const float*>(base) + off;
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[v] = ptr[ok ? v : 0];
        } break;
      }
#pragma unroll
      for (int v = 0; v < VEC; ++v) x[v] = ok ? x[v] : 0.f;
    };
    for (int t0 = 0; t0 < nt; t0 += nslot) {
      const int t = t0 + slot;
      float x[VEC];
      raw_row(p.kraw, b * p.kr_sb + hkv * p.kr_sh, p.kr_st, t, t < nt && dact, x);
      float pd[GM];
#pragma unroll
      for (int g = 0; g < GM; ++g) {
        float a = 0.f;
#pragma unroll
        for (int v = 0; v < VEC; ++v) a = __builtin_fmaf(qv[g][v], x[v], a);
        pd[g] = row_sum(a, lpr);
      }
      if (lir == 0 && t < nt) {
#pragma unroll
        for (int g = 0; g < GM; ++g) tsc[t * GM + g] = pd[g] * p.scale_log2;
      }
    }
    __syncthreads();
    // every wavefront: per head, lanes = tokens
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      const float lg = lane < nt ? tsc[lane * GM + g] : -INFINITY;
      float mx = lg;
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
      const float e = lane < nt ? __builtin_amdgcn_exp2f(lg - mx) : 0.f;
      float l = e;
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) l += __shfl_xor(l, m, 64);
      m_run[g] = mx;
      l_run[g] = l;
      if (tid < nt) tex[tid * GM + g] = e;
    }
    __syncthreads();
    for (int t0 = 0; t0 < nt; t0 += nslot) {
      const int t = t0 + slot;
      float x[VEC];
      raw_row(p.vraw, b * p.vr_sb + hkv * p.vr_sh, p.vr_st, t, t < nt && dact, x);
      if (t < nt) {
#pragma unroll
        for (int g = 0; g < GM; ++g) {
          const float w = tex[t * GM + g];
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[g][v] = __builtin_fmaf(w, x[v], acc[g][v]);
        }
      }
    }
    __syncthreads();  // sw is reused by the passes
  }

  const int64_t nb_begin = (int64_t)split * bps;
  const int64_t nb_end = min(nb, nb_begin + bps);
  const int cb_max = max(1, kPassRows / s);
  const int bst = (s | 1) * GM;
  // V rows rho0, rho0 + nslot, ... (kRB of them) of the pass at block nb0
  auto load_v_batch = [&](int rho0, int nrows, int64_t nb0, float (&x)[kRB][VEC]) {
#pragma unroll
    for (int u = 0; u < kRB; ++u) {
      const int rho = rho0 + u * nslot;
      const bool ok = rho < nrows;
      const int nl = ok ? rho / s : 0, j = ok ? rho - nl * s : 0;
      load_row<TS, KIND, VEC>(p.vrows, KIND == FC_STORE_JPEG_I8G ? p.vscales : nullptr,
                              p.vanch, p.vcap, bh, nb0 + nl, j, s, r, p.D, d0, dact && ok, x[u]);
    }
  };

  for (int64_t nb0 = nb_begin; nb0 < nb_end; nb0 += cb_max) {
    const int cb = (int)min((int64_t)cb_max, nb_end - nb0);
    const int nrows = cb * s;

    // ---- A: scores q . S_j for every row of the pass; each thread issues
    // the loads of kRB rows before it reduces any of them
    for (int rho0 = slot; rho0 < nrows; rho0 += kRB * nslot) {
      float x[kRB][VEC], rs[kRB];
#pragma unroll
      for (int u = 0; u < kRB; ++u) {
        const int rho = rho0 + u * nslot;
        const bool ok = rho < nrows;
        const int nl = ok ? rho / s : 0, j = ok ? rho - nl * s : 0;
        rs[u] = load_row<TS, KIND, VEC>(p.krows, p.kscales, p.kanch, p.kcap, bh, nb0 + nl, j, s,
                                        r, p.D, d0, dact && ok, x[u]);
      }
#pragma unroll
      for (int u = 0; u < kRB; ++u) {
        const int rho = rho0 + u * nslot;
        float pd[GM];
#pragma unroll
        for (int g = 0; g < GM; ++g) {
          float a = 0.f;
#pragma unroll
          for (int v = 0; v < VEC; ++v) a = __builtin_fmaf(qv[g][v], x[u][v], a);
          pd[g] = row_sum(a, lpr);
        }
        if (lir == 0 && rho < nrows) {
          const int nl = rho / s, so = nl * bst + (rho - nl * s) * GM;
#pragma unroll
          for (int g = 0; g < GM; ++g) sw[so + g] = pd[g] * rs[u];
        }
      }
    }
    __syncthreads();

    // the first batch of V rows is requested now, so that its loads are in
    // flight while phase B works on the scores
    float xv[kRB][VEC];
    load_v_batch(slot, nrows, nb0, xv);

    // ---- B: logits, running max, weights (in place of the scores)
    const int npairs = cb * GM;
    // png with r <= 16: one 16-lane row per (block, head) pair, lane t =
    // token t (prefix sums for the logits, suffix sums for the weights);
    // otherwise one thread per pair.  Either way every pair a thread
    // handles has head gsel.
    const bool rows16 = KIND == FC_STORE_PNG && r <= 16;
    const int gsel = rows16 ? (tid >> 4) % GM : tid % GM;
    const int l16 = tid & 15;
    float pmax[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) pmax[g] = -INFINITY;
    if (rows16) {
      for (int u = tid >> 4; u - (tid >> 4) < npairs; u += kAttnThreads / 16) {
        const bool ok = u < npairs && l16 < r;  // uniform loop bound over the row
        const float sc = ok ? sw[(u / GM) * bst + l16 * GM + gsel] : 0.f;
        // the row operations run in all 16 lanes (their DPP sources must be active)
        const float pre = row16_prefix(sc);
        const float mx = row16_max(ok ? pre * p.scale_log2 : -INFINITY);
#pragma unroll
        for (int g = 0; g < GM; ++g)
          if (g == gsel) pmax[g] = fmaxf(pmax[g], mx);
      }
    } else {
      for (int u = tid; u < npairs; u += kAttnThreads) {
        const float mx = pair_max<KIND, SREG>(sw + (u / GM) * bst + gsel, GM, p.A, r, s,
                                              p.scale_log2);
#pragma unroll
        for (int g = 0; g < GM; ++g)
          if (g == gsel) pmax[g] = fmaxf(pmax[g], mx);
      }
    }
    wg_reduce<GM>(pmax, red, true);
    float alpha[GM];
    float mg = 0.f;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      const float mn = fmaxf(m_run[g], pmax[g]);
      alpha[g] = __builtin_amdgcn_exp2f(m_run[g] - mn);
      m_run[g] = mn;
      if (g == gsel) mg = mn;
    }
    float psum[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) psum[g] = 0.f;
    if (rows16) {
      float es = 0.f;
      for (int u = tid >> 4; u - (tid >> 4) < npairs; u += kAttnThreads / 16) {
        const bool ok = u < npairs && l16 < r;
        float* const at = sw + (u / GM) * bst + l16 * GM + gsel;
        const float sc = ok ? *at : 0.f;
        const float lg = row16_prefix(sc) * p.scale_log2;
        const float e = ok ? __builtin_amdgcn_exp2f(lg - mg) : 0.f;
        es += e;
        const float w = row16_suffix(e);  // w_j = sum_{t >= j} e_t
        if (ok) *at = w;
      }
#pragma unroll
      for (int g = 0; g < GM; ++g)
        if (g == gsel) psum[g] = es;
    } else {
      for (int u = tid; u < npairs; u += kAttnThreads) {
        const int nl = u / GM;
        const float* vsc = KIND == FC_STORE_JPEG_I8 ? p.vscales + (bh * p.vcap + nb0 + nl) * s
                                                    : nullptr;
        const float es = pair_weights<KIND, SREG>(sw + nl * bst + gsel, wts + nl * bst + gsel,
                                                  GM, p.A, r, s, p.scale_log2, mg, vsc);
#pragma unroll
        for (int g = 0; g < GM; ++g)
          if (g == gsel) psum[g] += es;
      }
    }
    wg_reduce<GM>(psum, red, false);
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      l_run[g] = l_run[g] * alpha[g] + psum[g];
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[g][v] *= alpha[g];
    }
    // (wg_reduce ended with a barrier, so the weights are visible)

    // ---- C: values, kRB rows of loads in flight per thread (xv holds the
    // batch at rho0; the next batch is requested once it is consumed)
    for (int rho0 = slot; rho0 < nrows; rho0 += kRB * nslot) {
#pragma unroll
      for (int u = 0; u < kRB; ++u) {
        const int rho = rho0 + u * nslot;
        if (rho >= nrows) break;  // uniform over the lanes of a row
        const int nl = rho / s, so = nl * bst + (rho - nl * s) * GM;
#pragma unroll
        for (int g = 0; g < GM; ++g) {
          const float w = wts[so + g];
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[g][v] = __builtin_fmaf(w, xv[u][v], acc[g][v]);
        }
      }
      if (rho0 + kRB * nslot < nrows) load_v_batch(rho0 + kRB * nslot, nrows, nb0, xv);
    }
    __syncthreads();
  }

  // ---- combine the row slots: lanes of a wavefront with equal `lir` (all
  // GM * VEC exchanges of one distance in flight together), then the
  // wavefronts through LDS (reusing sw) over the flattened (head, feature)
  // range, in as few chunks as the LDS region allows (one at GM * D <= 768).
  for (int m = lpr; m < 64; m <<= 1) {
#pragma unroll
    for (int g = 0; g < GM; ++g)
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[g][v] += __shfl_xor(acc[g][v], m, 64);
  }
  const int lane = tid & 63, wave = tid >> 6;
  constexpr int nwave = kAttnThreads / 64;
  constexpr int kChunk = kRegion * kSwRegions / nwave;
  const int64_t ng = min((int64_t)GM, p.G - g0);  // heads of this group
  const int64_t total = ng * p.D;
  const int64_t bq0 = b * (p.Hkv * p.G) + hkv * p.G + g0;
  // with the fused merge the partials are stored at device scope (read back
  // by another workgroup of this kernel)
  const bool fused = p.arrive != nullptr;
  auto publish = [&](float* at, float v) {
    if (fused)
      __hip_atomic_store(at, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      *at = v;
  };
  for (int64_t c = 0; c < total; c += kChunk) {
    const int64_t span = min((int64_t)kChunk, total - c);
    if (c > 0) __syncthreads();  // the previous chunk's sums are read
    if (lane < lpr && dact) {
#pragma unroll
      for (int g = 0; g < GM; ++g)
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          const int64_t i = g * p.D + d0 + v - c;
          if (g < ng && i >= 0 && i < span) sw[wave * span + i] = acc[g][v];
        }
    }
    __syncthreads();
    for (int64_t i = tid; i < span; i += kAttnThreads) {
      float x = 0.f;
#pragma unroll
      for (int w = 0; w < nwave; ++w) x += sw[w * span + i];
      const int64_t g = (c + i) / p.D, d = (c + i) - g * p.D;
      publish(p.pacc + ((bq0 + g) * p.n_splits + split) * p.D + d, x);
    }
  }
  if (tid < ng) {
#pragma unroll
    for (int g = 0; g < GM; ++g)
      if (g == tid) {
        publish(p.pm + (bq0 + g) * p.n_splits + split, m_run[g]);
        publish(p.pl + (bq0 + g) * p.n_splits + split, l_run[g]);
      }
  }
  if (!fused) return;

  // ---- arrival: every thread's stores are complete before the workgroup
  // counts itself, so the workgroup that counts last finds every partial of
  // its group published; it returns the word to zero and merges.
  __shared__ int s_last;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0) {
    unsigned int* word = p.arrive + ((int64_t)blockIdx.y * gridDim.z + blockIdx.z) * p.cstride;
    const unsigned int old = atomicAdd(word, 1u);
    const bool last = old + 1 == (unsigned int)p.n_splits;
    if (last) __hip_atomic_store(word, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  merge_group<GM>(p, b, hkv, g0, (int)ng, tid, sw);
}

struct MergeArgs {
  const void* q;
  int q_dtype;
  int64_t q_sb, q_sh;
  const void* kraw;
  const void* vraw;
  int raw_dtype;
  int64_t kr_sb, kr_sh, kr_st, vr_sb, vr_sh, vr_st;
  int64_t n_raw;
  void* out;
  int64_t o_sb, o_sh;
  int64_t Hkv, G, D;
  float scale_log2;
  int n_splits;
  const float* pm;
  const float* pl;
  const float* pacc;
};

constexpr int kMergeMaxD = FC_MAX_HEAD_DIM / 64;

__global__ __launch_bounds__(kAttnThreads) void attn_merge_kernel(MergeArgs p) {
  __shared__ float wsplit[kAttnThreads / 64][kMaxSplits];
  __shared__ float wtail[kAttnThreads / 64][FC_MAX_BLOCK];
  const int64_t bh = blockIdx.x;
  const int64_t b = bh / p.Hkv, hkv = bh - b * p.Hkv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int nwave = kAttnThreads / 64;
  const int nd = (int)((p.D + 63) / 64);

  // wavefront `wave` handles query head gbase + wave of the kv group; the
  // loop trip count is uniform so the barriers are reached by everyone
  for (int64_t gbase = 0; gbase < p.G; gbase += nwave) {
    const int64_t g = gbase + wave;
    const bool act = g < p.G;
    const int64_t hq = hkv * p.G + (act ? g : 0);
    const int64_t bq = b * (p.Hkv * p.G) + hq;
    float qv[kMergeMaxD];
#pragma unroll
    for (int i = 0; i < kMergeMaxD; ++i) {
      const int64_t d = lane + 64 * i;
      qv[i] = (i < nd && d < p.D) ? load_q(p.q, p.q_dtype, b * p.q_sb + hq * p.q_sh + d) : 0.f;
    }
    // raw-tail logits (base-2 domain)
    float mx = -INFINITY;
    for (int64_t t = 0; t < p.n_raw; ++t) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < kMergeMaxD; ++i) {
        const int64_t d = lane + 64 * i;
        if (i < nd && d < p.D)
          a = __builtin_fmaf(
              qv[i], load_q(p.kraw, p.raw_dtype, b * p.kr_sb + hkv * p.kr_sh + t * p.kr_st + d),
              a);
      }
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) a += __shfl_xor(a, m, 64);
      const float lg = a * p.scale_log2;
      if (lane == 0) wtail[wave][t] = lg;
      mx = fmaxf(mx, lg);
    }
    // split maxima
    for (int sp = lane; sp < p.n_splits; sp += 64) mx = fmaxf(mx, p.pm[bq * p.n_splits + sp]);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    float l = 0.f;
    for (int sp = lane; sp < p.n_splits; sp += 64) {
      const float w = __builtin_amdgcn_exp2f(p.pm[bq * p.n_splits + sp] - mx);
      wsplit[wave][sp] = w;
      l = __builtin_fmaf(w, p.pl[bq * p.n_splits + sp], l);
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) l += __shfl_xor(l, m, 64);
    __syncthreads();
    for (int64_t t = 0; t < p.n_raw; ++t) l += __builtin_amdgcn_exp2f(wtail[wave][t] - mx);
    const float inv = 1.0f / l;
#pragma unroll
    for (int i = 0; i < kMergeMaxD; ++i) {
      const int64_t d = lane + 64 * i;
      if (!act || i >= nd || d >= p.D) continue;
      float o = 0.f;
      for (int sp = 0; sp < p.n_splits; ++sp)
        o = __builtin_fmaf(wsplit[wave][sp], p.pacc[(bq * p.n_splits + sp) * p.D + d], o);
      for (int64_t t = 0; t < p.n_raw; ++t) {
        const float e = __builtin_amdgcn_exp2f(wtail[wave][t] - mx);
        o = __builtin_fmaf(
            e, load_q(p.vraw, p.raw_dtype, b * p.vr_sb + hkv * p.vr_sh + t * p.vr_st + d), o);
      }
      store_any(p.out, p.q_dtype, b * p.o_sb + hq * p.o_sh + d, o * inv);
    }
    __syncthreads();
  }
}

// Merge pass, one workgroup per query head (D % 4 == 0): split maxima and
// raw-tail logits first, then every thread owns 4 features of one split
// group and keeps all of that group's partial loads in flight at once.
constexpr int kMerge2Threads = 128;

__global__ __launch_bounds__(kMerge2Threads) void attn_merge_head_kernel(MergeArgs p) {
  __shared__ float wsp[kMaxSplits];
  __shared__ float wtl[FC_MAX_BLOCK];
  __shared__ float red[kMerge2Threads / 64];
  __shared__ float4 part[kMerge2Threads];
  const int64_t bq = blockIdx.x;                 // b * Hq + hq
  const int64_t Hq = p.Hkv * p.G;
  const int64_t b = bq / Hq, hq = bq - b * Hq, hkv = hq / p.G;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int nwave = kMerge2Threads / 64;
  const int ns = p.n_splits;

  // raw-tail logits: wavefront w takes tokens w, w + nwave, ...
  float qv[kMergeMaxD];
#pragma unroll
  for (int i = 0; i < kMergeMaxD; ++i) {
    const int64_t d = lane + 64 * i;
    qv[i] = (p.n_raw > 0 && d < p.D) ? load_q(p.q, p.q_dtype, b * p.q_sb + hq * p.q_sh + d) : 0.f;
  }
  float mx = -INFINITY;
  for (int64_t t = wave; t < p.n_raw; t += nwave) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < kMergeMaxD; ++i) {
      const int64_t d = lane + 64 * i;
      if (d < p.D)
        a = __builtin_fmaf(
            qv[i], load_q(p.kraw, p.raw_dtype, b * p.kr_sb + hkv * p.kr_sh + t * p.kr_st + d), a);
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) a += __shfl_xor(a, m, 64);
    a *= p.scale_log2;
    if (lane == 0) wtl[t] = a;
    mx = fmaxf(mx, a);
  }
  for (int sp = tid; sp < ns; sp += kMerge2Threads) mx = fmaxf(mx, p.pm[bq * ns + sp]);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < nwave; ++w) mx = fmaxf(mx, red[w]);
  __syncthreads();
  float l = 0.f;
  for (int sp = tid; sp < ns; sp += kMerge2Threads) {
    const float w = __builtin_amdgcn_exp2f(p.pm[bq * ns + sp] - mx);
    wsp[sp] = w;
    l = __builtin_fmaf(w, p.pl[bq * ns + sp], l);
  }
  for (int64_t t = tid; t < p.n_raw; t += kMerge2Threads) {
    const float e = __builtin_amdgcn_exp2f(wtl[t] - mx);
    wtl[t] = e;
    l += e;
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) l += __shfl_xor(l, m, 64);
  __syncthreads();  // weights visible; red reusable
  if (lane == 0) red[wave] = l;
  __syncthreads();
  l = red[0];
#pragma unroll
  for (int w = 1; w < nwave; ++w) l += red[w];
  const float inv = 1.0f / l;

  // features: thread -> (group g, 4 features c*4..c*4+3); groups stride splits
  const int chunks = (int)(p.D / 4);
  const int ngroup = kMerge2Threads / chunks;    // >= 1 since D <= 512
  const int grp = tid / chunks, c = tid - grp * chunks;
  float4 o = {0.f, 0.f, 0.f, 0.f};
  if (grp < ngroup) {
    const float4* src = reinterpret_cast<const float4*>(p.pacc + bq * ns * p.D) + c;
    const int64_t stride = p.D / 4;
    int sp = grp;
    for (; sp + 3 * ngroup < ns; sp += 4 * ngroup) {
      const float4 a0 = src[(int64_t)sp * stride];
      const float4 a1 = src[(int64_t)(sp + ngroup) * stride];
      const float4 a2 = src[(int64_t)(sp + 2 * ngroup) * stride];
      const float4 a3 = src[(int64_t)(sp + 3 * ngroup) * stride];
      const float w0 = wsp[sp], w1 = wsp[sp + ngroup], w2 = wsp[sp + 2 * ngroup],
                  w3 = wsp[sp + 3 * ngroup];
      o.x = __builtin_fmaf(w0, a0.x, o.x); o.y = __builtin_fmaf(w0, a0.y, o.y);
      o.z = __builtin_fmaf(w0, a0.z, o.z); o.w = __builtin_fmaf(w0, a0.w, o.w);
      o.x = __builtin_fmaf(w1, a1.x, o.x); o.y = __builtin_fmaf(w1, a1.y, o.y);
      o.z = __builtin_fmaf(w1, a1.z, o.z); o.w = __builtin_fmaf(w1, a1.w, o.w);
      o.x = __builtin_fmaf(w2, a2.x, o.x); o.y = __builtin_fmaf(w2, a2.y, o.y);
      o.z = __builtin_fmaf(w2, a2.z, o.z); o.w = __builtin_fmaf(w2, a2.w, o.w);
      o.x = __builtin_fmaf(w3, a3.x, o.x); o.y = __builtin_fmaf(w3, a3.y, o.y);
      o.z = __builtin_fmaf(w3, a3.z, o.z); o.w = __builtin_fmaf(w3, a3.w, o.w);
    }
    for (; sp < ns; sp += ngroup) {
      const float4 a0 = src[(int64_t)sp * stride];
      const float w0 = wsp[sp];
      o.x = __builtin_fmaf(w0, a0.x, o.x); o.y = __builtin_fmaf(w0, a0.y, o.y);
      o.z = __builtin_fmaf(w0, a0.z, o.z); o.w = __builtin_fmaf(w0, a0.w, o.w);
    }
    // raw-tail values: group g takes tokens g, g + ngroup, ...
    for (int64_t t = grp; t < p.n_raw; t += ngroup) {
      const float e = wtl[t];
      const int64_t base = b * p.vr_sb + hkv * p.vr_sh + t * p.vr_st + 4 * c;
      o.x = __builtin_fmaf(e, load_q(p.vraw, p.raw_dtype, base + 0), o.x);
      o.y = __builtin_fmaf(e, load_q(p.vraw, p.raw_dtype, base + 1), o.y);
      o.z = __builtin_fmaf(e, load_q(p.vraw, p.raw_dtype, base + 2), o.z);
      o.w = __builtin_fmaf(e, load_q(p.vraw, p.raw_dtype, base + 3), o.w);
    }
  }
  part[tid] = o;
  __syncthreads();
  if (tid < chunks) {
    float4 s4 = part[tid];
    for (int g = 1; g < ngroup; ++g) {
      const float4 x = part[g * chunks + tid];
      s4.x += x.x; s4.y += x.y; s4.z += x.z; s4.w += x.w;
    }
    const int64_t ob = b * p.o_sb + hq * p.o_sh + 4 * tid;
    store_any(p.out, p.q_dtype, ob + 0, s4.x * inv);
    store_any(p.out, p.q_dtype, ob + 1, s4.y * inv);
    store_any(p.out, p.q_dtype, ob + 2, s4.z * inv);
    store_any(p.out, p.q_dtype, ob + 3, s4.w * inv);
  }
}

template <int... Vs, typename F>
int attn_with_int(int v, F&& f) {
  int rc = FC_ERR_UNSUPPORTED;
  bool hit = false;
  ((v == Vs ? (rc = f(std::integral_constant<int, Vs>{}), hit = true) : false), ...);
  return hit ? rc : FC_ERR_UNSUPPORTED;
}

// Workgroups per compute unit of the vector-ALU split pass that would run
// for this store (kernel occupancy, cached per instantiation); 0 if the
// runtime cannot report it.
template <typename TS, int KIND, bool SREG, int GM>
int valu_occupancy_of() {
  static int cached = -1;
  if (cached < 0) {
    int n = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &n, reinterpret_cast<const void*>(&attn_split_kernel<TS, KIND, SREG, 8, GM>),
        kAttnThreads, 0);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    cached = n;
  }
  return cached;
}

int valu_split_occupancy(int store_kind, int stream_dtype, int s, int gm) {
  const bool sreg = s <= 8;
  return attn_with_int<1, 2, 4, 8>(gm, [&](auto gc) -> int {
    constexpr int GM = decltype(gc)::value;
    using KI8 = std::integral_constant<int, FC_STORE_JPEG_I8>;
    using KFP = std::integral_constant<int, FC_STORE_JPEG_FP>;
    using KPNG = std::integral_constant<int, FC_STORE_PNG>;
    auto by_dtype = [&](auto kc, auto sc) -> int {
      constexpr int KIND = decltype(kc)::value;
      constexpr bool SREG = decltype(sc)::value;
      switch (stream_dtype) {
        case FC_F32: return valu_occupancy_of<float, KIND, SREG, GM>();
        case FC_F16: return valu_occupancy_of<f16_t, KIND, SREG, GM>();
        case FC_BF16: return valu_occupancy_of<bf16_t, KIND, SREG, GM>();
        default: return 0;
      }
    };
    if (store_kind == FC_STORE_JPEG_I8)
      return sreg ? valu_occupancy_of<float, FC_STORE_JPEG_I8, true, GM>()
                  : valu_occupancy_of<float, FC_STORE_JPEG_I8, false, GM>();
    if (store_kind == FC_STORE_JPEG_I8G)
      return sreg ? valu_occupancy_of<float, FC_STORE_JPEG_I8G, true, GM>()
                  : valu_occupancy_of<float, FC_STORE_JPEG_I8G, false, GM>();
    if (store_kind == FC_STORE_PNG) return by_dtype(KPNG{}, std::true_type{});
    if (store_kind == FC_STORE_JPEG_FP)
      return sreg ? by_dtype(KFP{}, std::true_type{}) : by_dtype(KFP{}, std::false_type{});
    (void)KI8{};
    return 0;
  });
}

}  // namespace fc

using namespace fc;

namespace fc {

static int64_t ws_partial_bytes(int64_t B, int64_t Hq, int64_t D, int n_splits) {
  const int64_t slots = B * Hq * (int64_t)n_splits;
  const int64_t head = (slots + 3) / 4 * 4;
  const int64_t bytes = (2 * head + slots * D) * (int64_t)sizeof(float);
  return (bytes + 255) / 256 * 256;
}

// Workspace of one call: the header line, kCounterWords 32-bit counters of
// the split passes (a fixed region, so calls of any shape find their
// counters at the same place), then pm | pl | pacc (fp32, sections 16-byte
// aligned).  The counters must be zero before a workspace's first use;
// every call leaves them zero.
WsLayout ws_layout(void* workspace, int64_t B, int64_t Hq, int n_splits) {
  WsLayout w;
  unsigned int* base = static_cast<unsigned int*>(workspace);
  w.done = base;
  w.counters = base + kWsHeadWords;
  const int64_t ws_head = (B * Hq * (int64_t)n_splits + 3) / 4 * 4;
  w.pm = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  w.pl = w.pm + ws_head;
  w.pacc = w.pl + ws_head;
  return w;
}

}  // namespace fc

extern "C" {

int64_t fc_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t D, int n_splits) {
  if (B <= 0 || Hq <= 0 || D <= 0 || n_splits <= 0) return 0;
  return fc::kCounterBytes + fc::ws_partial_bytes(B, Hq, D, n_splits);
}

int fc_attention_default_splits(int64_t nb, int64_t B, int64_t Hkv, int64_t G, int n_cu) {
  if (nb <= 0) return 0;
  if (n_cu <= 0) n_cu = 256;
  // one round of workgroups: two per compute unit, one per (split, batch,
  // kv head, group of up to 16 query heads)
  const int64_t groups = (G + 15) / 16;
  const int64_t cols = std::max<int64_t>(1, B * Hkv * groups);
  int64_t want = (2 * (int64_t)n_cu + cols - 1) / cols;
  // at least ~16 blocks per split, at most kMaxSplits splits
  want = std::min<int64_t>(want, (nb + 15) / 16);
  want = std::max<int64_t>(1, std::min<int64_t>(want, kMaxSplits));
  // splits that are actually non-empty
  const int64_t bps = (nb + want - 1) / want;
  return (int)((nb + bps - 1) / bps);
}

int fc_attention_splits(int store_kind, int stream_dtype, int q_dtype, int s, int64_t nb,
                        int64_t B, int64_t Hkv, int64_t G, int64_t D, int n_cu) {
  if (nb <= 0) return 0;
  if (n_cu <= 0) n_cu = 256;
  if (store_kind == FC_STORE_PNG_PACKED) {
    // one round of the packed png pass's workgroups (two per compute unit),
    // at least one iteration (256 / D blocks) per wavefront and at most
    // max(16, iterations / 10) splits, within the fused merge's limit
    const int64_t groups = (G + 15) / 16;
    const int64_t cols = std::max<int64_t>(1, B * Hkv * groups);
    int64_t want = (2 * (int64_t)n_cu + cols - 1) / cols;
    const int64_t per_it = D > 0 && D <= 256 ? std::max<int64_t>(1, 256 / D) : 1;
    const int64_t nit = (nb + per_it - 1) / per_it;
    want = std::min<int64_t>(want, std::max<int64_t>(1, nit / 4));
    want = std::min<int64_t>(want, std::max<int64_t>(16, nit / 10));
    want = std::max<int64_t>(1, std::min<int64_t>(want, fc::kFuseMaxSplitsPk));
    const int64_t bps = (nb + want - 1) / want;
    return (int)((nb + bps - 1) / bps);
  }
  const bool png_mfma =
      store_kind == FC_STORE_PNG && fc::png_mfma_shape_supported(q_dtype, stream_dtype, D, s);
  const bool fpj_mfma =
      store_kind == FC_STORE_JPEG_FP && fc::fpj_mfma_shape_supported(q_dtype, stream_dtype, D, s);
  const bool mfma = (png_mfma || fpj_mfma ||
                     (store_kind == FC_STORE_JPEG_I8 && fc::mfma_shape_supported(q_dtype, D, s)) ||
                     (store_kind == FC_STORE_JPEG_I8G &&
                      fc::mfma_group_shape_supported(q_dtype, D, s))) &&
                    fc::mfma_split_allowed();
  if (n_cu <= 0) n_cu = 256;
  if (mfma) {
    // one round of matrix-core workgroups (two per compute unit), but at
    // least one pass (64 rows; 32 at D = 256) per wavefront, and no more
    // than 16 splits or a tenth of the passes (each split adds a partial to
    // the final merge): measured on the MI355X, 16 splits take 14.9 us at
    // B=1, Hkv=8, G=2, k=2, S=16K where 64 take 25.9, 24 splits 20.3 us at
    // S=64K where 64 take 28.6
    const int64_t groups = (G + 15) / 16;
    const int64_t cols = std::max<int64_t>(1, B * Hkv * groups);
    // fp32 coefficient archives run on the png pass (16-row passes)
    const bool fpj32 = fpj_mfma && stream_dtype == FC_F32;
    const int64_t per_cu = png_mfma || fpj32 ? fc::kPngWgPerCu : 2;
    int64_t want = (per_cu * (int64_t)n_cu + cols - 1) / cols;
    // rows per pass
    const int64_t pr = png_mfma || fpj32 ? 16 : fpj_mfma ? (D == 64 ? 64 : 32) : D == 256 ? 32 : 64;
    const int64_t npass = (nb * s + pr - 1) / pr;
    want = std::min<int64_t>(want, std::max<int64_t>(1, npass / 4));
    want = std::min<int64_t>(want, std::max<int64_t>(16, npass / 10));
    want = std::max<int64_t>(1, std::min<int64_t>(want, fc::kMaxSplits));
    const int64_t bps = (nb + want - 1) / want;
    return (int)((nb + bps - 1) / bps);
  }
  // vector-ALU split pass: one round of its workgroups at the occupancy the
  // kernel reaches on this device (two per compute unit if it cannot be read)
  const int gm = G >= 8 ? 8 : (G >= 4 ? 4 : (G >= 2 ? 2 : 1));
  int per_cu = fc::valu_split_occupancy(store_kind, stream_dtype, s, gm);
  if (per_cu <= 0) per_cu = 2;
  const int64_t cols = std::max<int64_t>(1, B * Hkv * ((G + gm - 1) / gm));
  int64_t want = ((int64_t)per_cu * n_cu + cols - 1) / cols;
  want = std::min<int64_t>(want, (nb + 15) / 16);
  want = std::max<int64_t>(1, std::min<int64_t>(want, fc::kMaxSplits));
  const int64_t bps = (nb + want - 1) / want;
  return (int)((nb + bps - 1) / bps);
}

}  // extern "C"

namespace fc {

// Groups of the vector-ALU pass: (batch, kv head, group of <= 8 query heads).
static int64_t valu_groups(int64_t B, int64_t Hkv, int64_t G) {
  const int gm = G >= 8 ? 8 : (G >= 4 ? 4 : (G >= 2 ? 2 : 1));
  return B * Hkv * ((G + gm - 1) / gm);
}

// Whether the workspace holds a merge counter for every group.
static bool valu_fusable(int64_t B, int64_t Hkv, int64_t G) {
  return valu_groups(B, Hkv, G) * kCounterStride <= kCounterWords;
}

// Enqueues the vector-ALU split pass (VEC = 8 features per lane, LPR =
// lanes per row).  counters != NULL: the merge is fused (split 0 folds the
// n_raw tail tokens in, the last workgroup per group writes `out`).
// state != NULL (fused only): the block and tail counts come from the
// device pair (n_blocks, n_tail) before the step's token, nb sizing nothing
// but the caller's split count.
static int launch_split_valu(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                             int64_t Hkv, int64_t G, int64_t D, int store_kind, int stream_dtype,
                             int r, int s, int64_t nb, const fc_stream_view* key,
                             const fc_stream_view* value, int64_t n_raw, const float* A,
                             float scale_log2, void* out, int64_t o_sb, int64_t o_sh, float* pm,
                             float* pl, float* pacc, int n_splits, unsigned int* counters,
                             const int64_t* state, hipStream_t st) {
  if (D % 8) return FC_ERR_UNSUPPORTED;
  const int64_t chunks = D / 8;
  int lg = 0;
  while ((int64_t(1) << lg) < chunks) ++lg;
  const int gm = G >= 8 ? 8 : (G >= 4 ? 4 : (G >= 2 ? 2 : 1));
  AttnArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.krows = key->rows;
  a.kscales = key->scales;
  a.kanch = key->anchors;
  a.kcap = key->cap;
  a.vrows = value->rows;
  a.vscales = value->scales;
  a.vanch = value->anchors;
  a.vcap = value->cap;
  a.A = A;
  a.Hkv = Hkv;
  a.G = G;
  a.D = D;
  a.nb = nb;
  a.r = r;
  a.s = s;
  a.scale_log2 = scale_log2;
  a.lpr_log2 = lg;
  a.blocks_per_split = (nb + n_splits - 1) / n_splits;
  a.n_splits = n_splits;
  a.pm = pm;
  a.pl = pl;
  a.pacc = pacc;
  a.state = state;
  const int64_t zg = (G + gm - 1) / gm;
  if (counters) {
    a.arrive = counters;
    a.cstride = kCounterStride;
    a.kraw = key->raw;
    a.vraw = value->raw;
    a.raw_dtype = stream_dtype;
    a.kr_sb = key->raw_sb;
    a.kr_sh = key->raw_sh;
    a.kr_st = key->raw_st;
    a.vr_sb = value->raw_sb;
    a.vr_sh = value->raw_sh;
    a.vr_st = value->raw_st;
    a.n_raw = n_raw;
    a.out = out;
    a.o_sb = o_sb;
    a.o_sh = o_sh;
  }
  const dim3 grid((unsigned)n_splits, (unsigned)(B * Hkv), (unsigned)zg);
  const bool sreg = s <= 8;
  auto go = [&](auto ts, auto kc, auto sc) {
    using TS = decltype(ts);
    constexpr int KIND = decltype(kc)::value;
    constexpr bool SREG = decltype(sc)::value;
    return attn_with_int<1, 2, 4, 8>(gm, [&](auto gc) {
      constexpr int GM = decltype(gc)::value;
      attn_split_kernel<TS, KIND, SREG, 8, GM><<<grid, kAttnThreads, 0, st>>>(a);
      return FC_OK;
    });
  };
  using KI8 = std::integral_constant<int, FC_STORE_JPEG_I8>;
  using KFP = std::integral_constant<int, FC_STORE_JPEG_FP>;
  using KPNG = std::integral_constant<int, FC_STORE_PNG>;
  using ST = std::true_type;
  using SF = std::false_type;
  int rc = FC_ERR_ARG;
  if (store_kind == FC_STORE_JPEG_I8) {
    // int8 rows do not depend on the stream dtype (the tail's dtype is read
    // at run time)
    rc = sreg ? go(float{}, KI8{}, ST{}) : go(float{}, KI8{}, SF{});
  } else if (store_kind == FC_STORE_JPEG_I8G) {
    if (D % 32) return FC_ERR_ARG;
    using KI8G = std::integral_constant<int, FC_STORE_JPEG_I8G>;
    rc = sreg ? go(float{}, KI8G{}, ST{}) : go(float{}, KI8G{}, SF{});
  } else if (store_kind == FC_STORE_JPEG_FP || store_kind == FC_STORE_PNG) {
    const bool png = store_kind == FC_STORE_PNG;
    auto pick = [&](auto ts) {
      if (png) return go(ts, KPNG{}, ST{});
      return sreg ? go(ts, KFP{}, ST{}) : go(ts, KFP{}, SF{});
    };
    switch (stream_dtype) {
      case FC_F32: rc = pick(float{}); break;
      case FC_F16: rc = pick(f16_t{}); break;
      case FC_BF16: rc = pick(bf16_t{}); break;
      default: return FC_ERR_ARG;
    }
  }
  if (rc != FC_OK) return rc;
  return check_launch();
}

// Validates the arguments and enqueues the requested parts: the split pass
// over the archived blocks and/or the merge pass (split partials + raw tail).
int decode_attention_parts(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                                  int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int store_kind,
                                  int stream_dtype, int r, int s, int64_t nb,
                                  const fc_stream_view* key, const fc_stream_view* value,
                                  int64_t n_raw, const float* A, float scale, void* out,
                                  int64_t o_sb, int64_t o_sh, void* workspace, int n_splits,
                                  void* stream, int parts) {
  if (!q || !out || !key || !value || B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0) return FC_ERR_ARG;
  if (Hq % Hkv) return FC_ERR_ARG;
  if (nb < 0 || n_raw < 0 || (nb == 0 && n_raw == 0)) return FC_ERR_ARG;
  if (esize_of(q_dtype) == 0 || q_dtype == FC_I8) return FC_ERR_ARG;
  if (esize_of(stream_dtype) == 0 || stream_dtype == FC_I8) return FC_ERR_ARG;
  if (D > FC_MAX_HEAD_DIM || r > FC_MAX_BLOCK || n_raw > FC_MAX_BLOCK) return FC_ERR_UNSUPPORTED;
  if (r < 1 || s < 1 || s > FC_MAX_BLOCK) return FC_ERR_ARG;
  if (store_kind == FC_STORE_PNG && s != r) return FC_ERR_ARG;
  if (store_kind == FC_STORE_PNG_PACKED && (s >= r || r > 16)) return FC_ERR_ARG;
  if (nb > 0) {
    if (!A || !key->rows || !value->rows || !workspace) return FC_ERR_ARG;
    if (n_splits < 1 || n_splits > kMaxSplits) return FC_ERR_ARG;
    if ((store_kind == FC_STORE_JPEG_I8 || store_kind == FC_STORE_JPEG_I8G) &&
        (!key->scales || !value->scales))
      return FC_ERR_ARG;
    if (store_kind == FC_STORE_JPEG_I8G && D % 32) return FC_ERR_ARG;
    if ((store_kind == FC_STORE_PNG || store_kind == FC_STORE_PNG_PACKED) &&
        (!key->anchors || !value->anchors))
      return FC_ERR_ARG;
    if (store_kind == FC_STORE_PNG_PACKED && (!key->masks || !value->masks)) return FC_ERR_ARG;
    if (nb > key->cap || nb > value->cap) return FC_ERR_ARG;
  } else {
    n_splits = 0;
  }
  if (n_raw > 0 && (!key->raw || !value->raw)) return FC_ERR_ARG;
  const int64_t G = Hq / Hkv;
  const float scale_log2 = scale * kLog2e;
  hipStream_t st = (hipStream_t)stream;
  // workspace: status | counters | pm | pl | pacc
  const WsLayout ws = ws_layout(workspace, B, Hq, n_splits);
  unsigned int* counters = ws.counters;
  float* pm = ws.pm;
  float* pl = ws.pl;
  float* pacc = ws.pacc;
  // counters of the matrix-core passes: arrival and queue per head group
  const int64_t mstride = counter_stride(2 * B * Hkv * ((G + 15) / 16));

  const bool grouped = store_kind == FC_STORE_JPEG_I8G;
  if (nb > 0 && (parts & kPartSplit) && store_kind == FC_STORE_PNG_PACKED) {
    // packed png archives have one pass (no vector-ALU form)
    if (!split_pngpk_supported(q, q_dtype, q_sb, q_sh, D, r, s, stream_dtype, key, value) ||
        mstride == 0)
      return FC_ERR_UNSUPPORTED;
    if ((((nb + n_splits - 1) / n_splits) * (n_splits - 1)) >= nb) return FC_ERR_ARG;
    const bool fuse = (parts & kPartMerge) && n_splits <= kFuseMaxSplitsPk;
    MfmaFuse fz{};
    if (fuse) {
      fz.raw_dtype = stream_dtype;
      fz.n_raw = n_raw;
      fz.out = out;
      fz.o_sb = o_sb;
      fz.o_sh = o_sh;
    }
    const int rc = launch_split_pngpk(q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, r, s, stream_dtype,
                                      nb, key, value, scale_log2, pm, pl, pacc, n_splits,
                                      counters, kCounterWords, mstride, fuse ? &fz : nullptr,
                                      nullptr, st);
    if (rc != FC_OK || fuse) return rc;
  } else if (nb > 0 && (parts & kPartSplit) &&
      i8_mfma_takes(store_kind, q, q_dtype, q_sb, q_sh, D, s, key, value) && mstride > 0 &&
      mfma_split_allowed()) {
    if ((((nb + n_splits - 1) / n_splits) * (n_splits - 1)) >= nb) return FC_ERR_ARG;
    // one launch per call when the merge is requested too: the split pass's
    // last workgroup per head group merges
    const bool fuse = (parts & kPartMerge) && split_i8_mfma_fusable(n_splits);
    MfmaFuse fz{};
    if (fuse) {
      fz.raw_dtype = stream_dtype;
      fz.n_raw = n_raw;
      fz.out = out;
      fz.o_sb = o_sb;
      fz.o_sh = o_sh;
    }
    const int rc = launch_split_i8_mfma(q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, r, s, nb, key,
                                        value, A, scale_log2, pm, pl, pacc, n_splits, counters,
                                        kCounterWords, mstride,
                                        fuse ? &fz : nullptr, st, grouped);
    if (rc != FC_OK || fuse) return rc;
  } else if (nb > 0 && (parts & kPartSplit) && store_kind == FC_STORE_PNG &&
             split_png_mfma_supported(q, q_dtype, q_sb, q_sh, D, r, stream_dtype, key, value) &&
             mstride > 0 &&
             mfma_split_allowed()) {
    if ((((nb + n_splits - 1) / n_splits) * (n_splits - 1)) >= nb) return FC_ERR_ARG;
    const bool fuse = (parts & kPartMerge) && split_i8_mfma_fusable(n_splits);
    MfmaFuse fz{};
    if (fuse) {
      fz.raw_dtype = stream_dtype;
      fz.n_raw = n_raw;
      fz.out = out;
      fz.o_sb = o_sb;
      fz.o_sh = o_sh;
    }
    const int rc = launch_split_png_mfma(q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, r, nb, key, value,
                                         scale_log2, pm, pl, pacc, n_splits, counters,
                                         kCounterWords, mstride,
                                         fuse ? &fz : nullptr, nullptr, st);
    if (rc != FC_OK || fuse) return rc;
  } else if (nb > 0 && (parts & kPartSplit) && store_kind == FC_STORE_JPEG_FP &&
             split_fpj_mfma_supported(q, q_dtype, q_sb, q_sh, D, s, stream_dtype, key, value) &&
             mstride > 0 && mfma_split_allowed()) {
    if ((((nb + n_splits - 1) / n_splits) * (n_splits - 1)) >= nb) return FC_ERR_ARG;
    const bool fuse = (parts & kPartMerge) && split_i8_mfma_fusable(n_splits);
    MfmaFuse fz{};
    if (fuse) {
      fz.raw_dtype = stream_dtype;
      fz.n_raw = n_raw;
      fz.out = out;
      fz.o_sb = o_sb;
      fz.o_sh = o_sh;
    }
    const int rc = launch_split_fpj_mfma(q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, r, s, nb, key,
                                         value, A, scale_log2, pm, pl, pacc, n_splits, counters,
                                         kCounterWords, mstride, fuse ? &fz : nullptr, nullptr,
                                         st);
    if (rc != FC_OK || fuse) return rc;
  } else if (nb > 0 && (parts & kPartSplit)) {
    // the merge runs inside the split pass when every group has a counter
    if (D % 8) return FC_ERR_UNSUPPORTED;
    if ((((nb + n_splits - 1) / n_splits) * (n_splits - 1)) >= nb) return FC_ERR_ARG;  // empty split
    const bool fuse = (parts & kPartMerge) && valu_fusable(B, Hkv, G);
    const int rc = launch_split_valu(q, q_dtype, q_sb, q_sh, B, Hkv, G, D, store_kind, stream_dtype,
                                     r, s, nb, key, value, fuse ? n_raw : 0, A, scale_log2, out,
                                     o_sb, o_sh, pm, pl, pacc, n_splits,
                                     fuse ? counters : nullptr, nullptr, st);
    if (rc != FC_OK || fuse) return rc;
  } else if (nb > 0 && store_kind != FC_STORE_PNG_PACKED) {
    // merge only: the split geometry must still be consistent
    if (D % 8) return FC_ERR_UNSUPPORTED;
  }
  if (!(parts & kPartMerge)) return FC_OK;

  MergeArgs mg{};
  mg.q = q;
  mg.q_dtype = q_dtype;
  mg.q_sb = q_sb;
  mg.q_sh = q_sh;
  mg.kraw = key->raw;
  mg.vraw = value->raw;
  mg.raw_dtype = stream_dtype;
  mg.kr_sb = key->raw_sb;
  mg.kr_sh = key->raw_sh;
  mg.kr_st = key->raw_st;
  mg.vr_sb = value->raw_sb;
  mg.vr_sh = value->raw_sh;
  mg.vr_st = value->raw_st;
  mg.n_raw = n_raw;
  mg.out = out;
  mg.o_sb = o_sb;
  mg.o_sh = o_sh;
  mg.Hkv = Hkv;
  mg.G = G;
  mg.D = D;
  mg.scale_log2 = scale_log2;
  mg.n_splits = n_splits;
  mg.pm = pm;
  mg.pl = pl;
  mg.pacc = pacc;
  if (D % 4 == 0 && D / 4 <= kMerge2Threads) {
    attn_merge_head_kernel<<<dim3((unsigned)(B * Hq)), kMerge2Threads, 0, st>>>(mg);
  } else {
    attn_merge_kernel<<<dim3((unsigned)(B * Hkv)), kAttnThreads, 0, st>>>(mg);
  }
  return check_launch();
}

int decode_attention_state(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                           int64_t Hq, int64_t Hkv, int64_t D, int store_kind, int stream_dtype,
                           int r, int s, int64_t nb_hint, const fc_stream_view* key,
                           const fc_stream_view* value, const float* A, float scale, void* out,
                           int64_t o_sb, int64_t o_sh, void* workspace, int64_t workspace_bytes,
                           int n_cu, const int64_t* state, void* stream) {
  if (!state || !q || !out || !key || !value || !A || !workspace || nb_hint < 1) return FC_ERR_ARG;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || Hq % Hkv) return FC_ERR_ARG;
  if (r < 1 || r > FC_MAX_BLOCK || s < 1 || s > r) return FC_ERR_ARG;
  if (!key->rows || !value->rows || !key->raw || !value->raw) return FC_ERR_ARG;
  if ((store_kind == FC_STORE_JPEG_I8 || store_kind == FC_STORE_JPEG_I8G) &&
      (!key->scales || !value->scales))
    return FC_ERR_ARG;
  if (store_kind == FC_STORE_PNG && (!key->anchors || !value->anchors || s != r)) return FC_ERR_ARG;
  if (store_kind == FC_STORE_PNG_PACKED &&
      (!key->anchors || !value->anchors || !key->masks || !value->masks || s >= r))
    return FC_ERR_ARG;
  const int64_t G = Hq / Hkv;
  const int n_splits =
      fc_attention_splits(store_kind, stream_dtype, q_dtype, s, nb_hint, B, Hkv, G, D, n_cu);
  if (n_splits < 1) return FC_ERR_UNSUPPORTED;
  if (fc_attention_workspace_bytes(B, Hq, D, n_splits) > workspace_bytes) return FC_ERR_ARG;
  const WsLayout ws = ws_layout(workspace, B, Hq, n_splits);
  unsigned int* counters = ws.counters;
  float* pm = ws.pm;
  float* pl = ws.pl;
  float* pacc = ws.pacc;
  const int64_t mstride = counter_stride(2 * B * Hkv * ((G + 15) / 16));
  hipStream_t st = (hipStream_t)stream;
  // the same pass fc_attention_splits sized: matrix cores for int8 jpeg
  // archives they support, else the vector-ALU pass; both with the merge
  // fused (no second launch depends on the counts)
  if (i8_mfma_takes(store_kind, q, q_dtype, q_sb, q_sh, D, s, key, value) &&
      mfma_split_allowed() && mstride > 0) {
    if (!split_i8_mfma_fusable(n_splits)) return FC_ERR_UNSUPPORTED;
    MfmaFuse fz{};
    fz.raw_dtype = stream_dtype;
    fz.n_raw = 0;  // taken from the state
    fz.out = out;
    fz.o_sb = o_sb;
    fz.o_sh = o_sh;
    fz.state = state;
    return launch_split_i8_mfma(q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, r, s, nb_hint, key, value,
                                A, scale * kLog2e, pm, pl, pacc, n_splits, counters,
                                kCounterWords, mstride, &fz, st,
                                store_kind == FC_STORE_JPEG_I8G);
  }
  if (store_kind == FC_STORE_PNG_PACKED) {
    if (!split_pngpk_supported(q, q_dtype, q_sb, q_sh, D, r, s, stream_dtype, key, value) ||
        mstride == 0 || n_splits > kFuseMaxSplitsPk)
      return FC_ERR_UNSUPPORTED;
    MfmaFuse fz{};
    fz.raw_dtype = stream_dtype;
    fz.n_raw = 0;  // taken from the state
    fz.out = out;
    fz.o_sb = o_sb;
    fz.o_sh = o_sh;
    return launch_split_pngpk(q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, r, s, stream_dtype, nb_hint,
                              key, value, scale * kLog2e, pm, pl, pacc, n_splits, counters,
                              kCounterWords, mstride, &fz, state, st);
  }
  if (store_kind == FC_STORE_PNG &&
      split_png_mfma_supported(q, q_dtype, q_sb, q_sh, D, r, stream_dtype, key, value) &&
      mfma_split_allowed() && mstride > 0) {
    if (!split_i8_mfma_fusable(n_splits)) return FC_ERR_UNSUPPORTED;
    MfmaFuse fz{};
    fz.raw_dtype = stream_dtype;
    fz.n_raw = 0;  // taken from the state
    fz.out = out;
    fz.o_sb = o_sb;
    fz.o_sh = o_sh;
    return launch_split_png_mfma(q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, r, nb_hint, key, value,
                                 scale * kLog2e, pm, pl, pacc, n_splits, counters, kCounterWords,
                                 mstride, &fz, state, st);
  }
  if (store_kind == FC_STORE_JPEG_FP &&
      split_fpj_mfma_supported(q, q_dtype, q_sb, q_sh, D, s, stream_dtype, key, value) &&
      mfma_split_allowed() && mstride > 0) {
    if (!split_i8_mfma_fusable(n_splits)) return FC_ERR_UNSUPPORTED;
    MfmaFuse fz{};
    fz.raw_dtype = stream_dtype;
    fz.n_raw = 0;  // taken from the state
    fz.out = out;
    fz.o_sb = o_sb;
    fz.o_sh = o_sh;
    return launch_split_fpj_mfma(q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, r, s, nb_hint, key, value,
                                 A, scale * kLog2e, pm, pl, pacc, n_splits, counters,
                                 kCounterWords, mstride, &fz, state, st);
  }
  if (!valu_fusable(B, Hkv, G)) return FC_ERR_UNSUPPORTED;
  return launch_split_valu(q, q_dtype, q_sb, q_sh, B, Hkv, G, D, store_kind, stream_dtype, r, s,
                           nb_hint, key, value, 0, A, scale * kLog2e, out, o_sb, o_sh, pm, pl,
                           pacc, n_splits, counters, state, st);
}

}  // namespace fc

extern "C" {

#define FC_ATTN_PARAMS                                                                        \
  const void *q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B, int64_t Hq, int64_t Hkv, \
      int64_t D, int store_kind, int stream_dtype, int r, int s, int64_t nb,                  \
      const fc_stream_view *key, const fc_stream_view *value, int64_t n_raw, const float *A,  \
      float scale, void *out, int64_t o_sb, int64_t o_sh, void *workspace, int n_splits,      \
      void *stream
#define FC_ATTN_ARGS                                                                         \
  q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, store_kind, stream_dtype, r, s, nb, key, value, n_raw, \
      A, scale, out, o_sb, o_sh, workspace, n_splits, stream

int fc_decode_attention(FC_ATTN_PARAMS) {
  return decode_attention_parts(FC_ATTN_ARGS, kPartSplit | kPartMerge);
}

int fc_decode_attention_split(FC_ATTN_PARAMS) {
  return decode_attention_parts(FC_ATTN_ARGS, kPartSplit);
}

int fc_decode_attention_merge(FC_ATTN_PARAMS) {
  return decode_attention_parts(FC_ATTN_ARGS, kPartMerge);
}

int fc_set_attention_pass(int pass) {
  if (pass != FC_PASS_AUTO && pass != FC_PASS_VECTOR && pass != FC_PASS_STATIC) return FC_ERR_ARG;
  g_attention_pass = pass;
  return FC_OK;
}

int fc_get_attention_pass(void) { return g_attention_pass; }

}  // extern "C"
