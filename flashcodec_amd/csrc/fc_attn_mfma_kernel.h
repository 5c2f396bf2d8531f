// Split pass of the decode attention for int8 jpeg archives on gfx950 matrix
// cores, with the merge of the split partials fused in: the kernel template
// and its device code.  Its instantiations are compiled in one translation
// unit per stored-row count (fc_attn_mfma_s<S>.hip, through
// launch_mfma_rows<S>); the host side is fc_attn_mfma.hip.
//
// With G query heads per kv head, a block's work is a skinny GEMM: scores
// S = K_rows . Q^T (M = rows, N = heads, K-dim = features) and output
// O = W . V_rows (M = heads, N = features, K-dim = rows).  On the vector ALU
// that costs ~4 fp32 FMAs per code byte per head group — more VALU time than
// the HBM time of the bytes — so both products run on the matrix cores and
// the VALU runs the softmax and the V code conversion.
//
// Scores: v_mfma_i32_16x16x64_i8 straight on the K codes.  Each head's query
// is scaled by a power of two to integers of at most 14 bits and split as
// q' = 256 hi + lo (int8 hi, lo): 256 (K . hi) + (K . lo) is the exact
// integer score.
// Values: v_mfma_f32_16x16x32_f16.  A V code b converts to f16 exactly:
// u = b ^ 0x80 = b + 128, the f16 with bits 0x6400 | u is 1024 + u, and one
// packed f16 add of -1152 (exact) leaves b.  Output weights enter as f16
// scaled by a per-wavefront power of two; products are exact in fp32 and
// the matrix cores accumulate in fp32.
//
// Workgroup = 4 wavefronts = one (batch, kv head, split, group of <= 16 query
// heads).  The wavefronts of a group's workgroups take passes of the group's
// stored rows, three quarters in a fixed order and the rest from a queue (64
// rows of 16-row tiles, 32 at D = 256; with 3 rows per block a pass is 63 /
// 30 rows, the last tile row reading zero):
//   scores: per 16-row tile and 64-feature chunk k, lane (q, m) holds row m,
//      features 64k + 16q .. +15 (one 64-byte run of each row per load; any
//      relabelling of the feature axis shared by both operands is allowed);
//      lane (q, c < G) gets the scores of rows 4q..4q+3 for head c and parks
//      them in LDS.
//   softmax: (block, head) pairs over all 64 lanes (head = lane % GP): r
//      logits from the s scores, exponentials against a running reference
//      maximum, and s output weights w_j = sum_p 2^(logit_p - m) A[p][j] times
//      the V row scale, stored as f16 in LDS.
//   values: per 32-row slab, lane (q, c) loads rows 8q..8q+7, bytes
//      [8c, 8c+8) (16 lanes cover a 128-byte row) and transposes the 8x8
//      byte tile in registers, so matrix-core instance e of the slab sees
//      feature 8c + e in column c.
// The four wavefronts combine their (max, sum, acc) in LDS into one partial
// per (query head, split); the last workgroup of each head group to finish
// merges the partials with the raw tail (fused_merge).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "fc_attn_internal.h"
#include "fc_common.h"
#include "fc_mfma_pass.h"

namespace fc {

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
  int64_t ngroups;  // B * Hkv * zg (zg = groups of <= 16 query heads per kv head)
  int zg;
  unsigned int* arrive;  // per group: workgroups done (zero between calls)
  unsigned int* passq;   // per group: next pass to take (zero between calls)
  int64_t cstride;       // words between the counters of consecutive groups
  float* pm;
  float* pl;
  float* pacc;
  // fused merge (fused != 0): raw tail, output and arrival counters
  int fused;
  const void* kraw;
  const void* vraw;
  int raw_dtype;
  int64_t kr_sb, kr_sh, kr_st, vr_sb, vr_sh, vr_st;
  int64_t n_raw;
  void* out;
  int64_t o_sb, o_sh;
  // decode-step state on the device (or NULL): (n_blocks, n_tail) before
  // the step's token; nb and n_raw are then taken from it (graph replays)
  const int64_t* state;
  // per-32 scales (FC_STORE_JPEG_I8G): D / 32 fp32 scales per stored row
  int qgroup;
  // static pass order (no queue): wavefront w of the group's n_splits * 4
  // takes passes w, w + n_splits * 4, ...; fixed summation order, so the
  // output is bitwise reproducible
  int static_passes;
  // fused decode step (step != 0): the step's key / value tokens
  // (B, Hkv, 1, D) join the tails (kraw / vraw: (B, Hkv, r, D) contiguous
  // buffers) at row t; when they complete a block, split 0 archives it as
  // block nb (codes at kcodes_w / vcodes_w, scales at kscales_w / vscales_w,
  // DCT basis `basis`, k = SROWS) and attends it from the fresh codes, and
  // the passes cover the blocks before it.  t and nb come from `state`
  // (then the last workgroup of the launch advances it, counting workgroups
  // on `done`) or from step_t / step_nb.
  int step;
  const void* ktok;
  const void* vtok;
  int64_t kt_sb, kt_sh, vt_sb, vt_sh;
  int8_t* kcodes_w;
  int8_t* vcodes_w;
  float* kscales_w;
  float* vscales_w;
  const float* basis;
  int64_t step_t, step_nb;
  unsigned int* done;
  // png archives (fc_attn_png.hip): anchors (B, H, cap, D) in the stream
  // dtype and fp32 deltas (B, H, cap, r - 1, D)
  const void* kanch;
  const void* vanch;
  const float* kdel;
  const float* vdel;
  // packed png archives (fc_attn_pngpk.hip): kdel / vdel are the value
  // stores (B, H, cap, keep_m, D), kmask / vmask the mask words (B, H, cap, D)
  const uint32_t* kmask;
  const uint32_t* vmask;
  int keep_m;
  // jpeg archives of fp coefficients (fc_attn_fpj.hip): (B, H, cap, k, D)
  // rows in the stream dtype
  const void* kfp;
  const void* vfp;
};

constexpr int kMThreads = 256;
constexpr int kFuseMaxSplits = 64;  // split count limit of the fused merge

constexpr int kWaves = kMThreads / 64;


// Element load / store with the dtype fixed at compile time (T = f16_t,
// bf16_t) or read at run time (T = void).
template <typename T>
__device__ __forceinline__ float ld_elem(const void* ptr, int dt, int64_t i) {
  if constexpr (std::is_void_v<T>) {
    return load_q(ptr, dt, i);
  } else {
    return to_f32(static_cast<const T*>(ptr)[i]);
  }
}
template <typename T>
__device__ __forceinline__ void st_elem(void* ptr, int dt, int64_t i, float v) {
  if constexpr (std::is_void_v<T>) {
    store_any(ptr, dt, i, v);
  } else {
    static_cast<T*>(ptr)[i] = from_f32<T>(v);
  }
}

// Raw-tail partial of one (batch, kv head, head group): for each of its G
// query heads the base-2 logits of the n_raw tail tokens at full precision,
// their maximum tm[h], sum tl[h] = sum_t 2^(logit_t - tm[h]) and
// acc[h][d] = sum_t 2^(logit_t - tm[h]) v_t[d].  `etl` holds
// 16 * FC_MAX_BLOCK floats; every thread of the workgroup takes part.  QT /
// RT are the query and tail element types: with them fixed at compile time
// each thread issues all its loads before it uses any (this runs while the
// other workgroups stream the archive, where every serialized load waits
// several microseconds).
template <int D, typename QT, typename RT>
__device__ __forceinline__ void raw_tail_partial_t(const MfmaArgs& p, int64_t b, int64_t hkv, int64_t g0, int G,
                                   int nr, int tid, float* etl, float* acc, float* tm,
                                   float* tl) {
  const int lane = tid & 63, wave = tid >> 6;
  const QT* qb = static_cast<const QT*>(p.q) + b * p.q_sb;
  const RT* kb = static_cast<const RT*>(p.kraw) + b * p.kr_sb + hkv * p.kr_sh;
  const RT* vb = static_cast<const RT*>(p.vraw) + b * p.vr_sb + hkv * p.vr_sh;
  {
    // logits: 16 lanes per (head, token), features strided by 16
    const int grp = tid >> 4, gl = tid & 15;
    for (int u = grp; u < G * nr; u += kMThreads / 16) {
      const int h = u / nr, t = u - h * nr;
      const QT* qr = qb + (hkv * p.G + g0 + h) * p.q_sh + gl;
      const RT* kr = kb + t * p.kr_st + gl;
      float qv[D / 16], kv[D / 16];
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        qv[i] = to_f32(qr[16 * i]);
        kv[i] = to_f32(kr[16 * i]);
      }
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) a = __builtin_fmaf(qv[i], kv[i], a);
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) a += __shfl_xor(a, m, 16);
      if (gl == 0) etl[h * FC_MAX_BLOCK + t] = a * p.scale_log2;
    }
  }
  __syncthreads();
  for (int h = wave; h < G; h += kWaves) {
    float mx = -INFINITY;
    for (int t = lane; t < nr; t += 64) mx = fmaxf(mx, etl[h * FC_MAX_BLOCK + t]);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    float l = 0.f;
    for (int t = lane; t < nr; t += 64) {
      const float e = __builtin_amdgcn_exp2f(etl[h * FC_MAX_BLOCK + t] - mx);
      etl[h * FC_MAX_BLOCK + t] = e;
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
  constexpr int kT = 8;  // tail rows requested together
  for (int x = tid; x < G * D; x += kMThreads) {
    const int h = x / D, d = x - h * D;
    float o = 0.f;
    for (int t0 = 0; t0 < nr; t0 += kT) {
      float vv[kT];
#pragma unroll
      for (int j = 0; j < kT; ++j) vv[j] = t0 + j < nr ? to_f32(vb[(t0 + j) * p.vr_st + d]) : 0.f;
#pragma unroll
      for (int j = 0; j < kT; ++j)
        if (t0 + j < nr) o = __builtin_fmaf(etl[h * FC_MAX_BLOCK + t0 + j], vv[j], o);
    }
    acc[h * D + d] = o;
  }
}

// QF32: fp32 queries (the png pass, fp32 queries of the int8 pass); else fp16 / bf16.
template <int D, bool QF32 = false>
__device__ __forceinline__ void raw_tail_partial(const MfmaArgs& p, int64_t b, int64_t hkv, int64_t g0, int G,
                                 int nr, int tid, float* etl, float* acc, float* tm, float* tl) {
  // tails in the stream dtype
  auto with_q = [&](auto rt) {
    using RT = decltype(rt);
    if constexpr (QF32)
      raw_tail_partial_t<D, float, RT>(p, b, hkv, g0, G, nr, tid, etl, acc, tm, tl);
    else if (p.q_dtype == FC_F16)
      raw_tail_partial_t<D, f16_t, RT>(p, b, hkv, g0, G, nr, tid, etl, acc, tm, tl);
    else
      raw_tail_partial_t<D, bf16_t, RT>(p, b, hkv, g0, G, nr, tid, etl, acc, tm, tl);
  };
  switch (p.raw_dtype) {
    case FC_F16: with_q(f16_t{}); break;
    case FC_BF16: with_q(bf16_t{}); break;
    default: with_q(float{}); break;
  }
}

// Archive of one stream's completed block inside the fused decode step:
// rows x (r rows of D fp32 values of the stream dtype TT) -> DCT-II
// coefficients by the fma chain over the taps rounded to TT, per-frequency
// absmax scale rounded to TT (1 when not > 0), codes as quant_code — the
// archive kernels' arithmetic, bit for bit — stored when `write`; then x is
// replaced by the block's tokens synthesised from the dequantised codes
// through A (r x SROWS), so the block is attended exactly as an archived
// one.  NG scales per row: 1 (the row's absmax) or D / 32 (per 32 features,
// scales[row * NG + group]); NG = 0: no quantizer, the coefficients rounded
// to TT are the stored rows (`codes` then points at TT, `scales` is unused).
// kk: SROWS x D, sc: SROWS * NG floats of LDS scratch.
template <int D, int SROWS, typename TT, int NG = 1>
__device__ __forceinline__ void step_archive(float* x, int r, const float* basis, const float* A,
                                             bool write, void* codes, float* scales, float* kk,
                                             float* sc, int tid) {
  static_assert(NG <= 1 || NG * 32 == D, "one scale per row or per 32 features");
  const int lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < SROWS * D; e += kMThreads) {
    const int j = e / D, d = e - j * D;
    float a = 0.f;
    for (int i = 0; i < r; ++i) a = __builtin_fmaf(x[i * D + d], basis[j * r + i], a);
    kk[e] = to_f32(from_f32<TT>(a));
    if constexpr (NG == 0) {
      if (write) static_cast<TT*>(codes)[e] = from_f32<TT>(a);
    }
  }
  __syncthreads();
  for (int j = wave; j < SROWS && NG > 0; j += kMThreads / 64) {  // one row per wavefront
    if constexpr (NG == 1) {
      float m = 0.f;
      for (int d = lane; d < D; d += 64) m = fmaxf(m, fabsf(kk[j * D + d]));
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      float sj = to_f32(from_f32<TT>(m / 127.0f));
      if (!(sj > 0.f)) sj = 1.0f;
      if (lane == 0) {
        sc[j] = sj;
        if (write) scales[j] = sj;
      }
    } else {
      // features 64 i + lane: group 2 i + lane / 32, its max over 32 lanes
      for (int i = 0; 64 * i < D; ++i) {
        const int d = 64 * i + lane;
        float m = d < D ? fabsf(kk[j * D + d]) : 0.f;
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float sj = to_f32(from_f32<TT>(m / 127.0f));
        if (!(sj > 0.f)) sj = 1.0f;
        if ((lane & 31) == 0 && d < D) {
          sc[j * NG + d / 32] = sj;
          if (write) scales[j * NG + d / 32] = sj;
        }
      }
    }
  }
  if constexpr (NG > 0) {
    __syncthreads();
    for (int e = tid; e < SROWS * D; e += kMThreads) {
      const float sj = NG == 1 ? sc[e / D] : sc[(e / D) * NG + (e % D) / 32];
      const float q = quant_code(kk[e], sj, 1.0f / sj);
      if (write) static_cast<int8_t*>(codes)[e] = (int8_t)(int)q;
      kk[e] = q * sj;
    }
  }
  __syncthreads();
  for (int e = tid; e < r * D; e += kMThreads) {
    const int i = e / D, d = e - i * D;
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < SROWS; ++j) a = __builtin_fmaf(A[i * SROWS + j], kk[j * D + d], a);
    x[e] = a;
  }
  __syncthreads();
}

// Fused decode step, split 0: the rows this step adds to the attention, in
// LDS as fp32 (xk, xv: n rows of D), and the partial of the group's G heads
// over them (as raw_tail_partial_t: tm, tl, acc).
//   * t + 1 < r: the tail rows 0..t-1 (buffer) and the new token; the token
//     is written to tail row t.
//   * t + 1 == r: the block of tail rows 0..r-2 and the new token is
//     archived as block nb (step_archive) and attended from its codes.
// `write`: this workgroup stores the token / the block (one head group per
// (batch, kv head) does; all compute the partial).  The query rows are
// q + qb + (h0 + h) * q_sh for the G heads.
template <int D, int SROWS, typename TT, int NG = 1>
__device__ __forceinline__ void step_partial(
    int64_t t, int r, TT* ktail, TT* vtail, const TT* ktok, const TT* vtok, bool write,
    void* kcodes, float* kscales, void* vcodes, float* vscales, const float* basis,
    const float* A, const void* q, int q_dtype, int64_t qb, int64_t q_sh, int64_t h0, int G,
    float scale_log2, int tid, float* xk, float* xv, float* kk, float* sc, float* etl, float* acc,
    float* tm, float* tl) {
  const int lane = tid & 63, wave = tid >> 6;
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
  if (complete) {
    step_archive<D, SROWS, TT, NG>(xk, r, basis, A, write, kcodes, kscales, kk, sc, tid);
    step_archive<D, SROWS, TT, NG>(xv, r, basis, A, write, vcodes, vscales, kk, sc, tid);
  }
  // the partial over the n rows, at full precision
  {
    const int grp = tid >> 4, gl = tid & 15;
    for (int u = grp; u < G * n; u += kMThreads / 16) {
      const int h = u / n, i = u - h * n;
      const int64_t qr = qb + (h0 + h) * q_sh + gl;
      float a = 0.f;
      for (int c = 0; c < D / 16; ++c)
        a = __builtin_fmaf(load_q(q, q_dtype, qr + 16 * c), xk[i * D + gl + 16 * c], a);
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

// Merge of one (batch, kv head, head group) by the workgroup that arrived
// last, once every other workgroup of the group has published its partial:
// out = sum_s w_s acc_s / sum_s w_s l_s over the n_splits partials of its G
// query heads, w_s = 2^(m_s - max_s m_s).  This workgroup's own partial is
// read from LDS (own_acc [16][D], own_m, own_l), the others with
// device-scope loads; the raw tail is part of split 0's partial.  The
// statistics of all splits come in with one load per thread; then each
// thread owns an output task (head, 4 features) and requests its partials
// kPre splits at a time.  The code runs once per call, after the pass loop,
// when its instructions are not in the instruction cache: it is kept short
// and free of per-element branches (every load of a batch is issued and
// splits past n_splits are selected away; one store branch per task).
// `lds` holds >= 2 * 16 * kFuseMaxSplits floats.
template <int D, bool QF32 = false, bool COMPACT = true>
__device__ __forceinline__ void fused_merge(const MfmaArgs& p, int64_t b, int64_t hkv, int64_t g0, int G,
                            int split, int tid, float* lds, const float* own_acc,
                            const float* own_m, const float* own_l) {
  constexpr int C4 = D / 4;  // float4 chunks of a head's output
  constexpr int kPre = 8;    // partials in flight per task
  const int ns = p.n_splits;
  const int64_t bq0 = b * (p.Hkv * p.G) + hkv * p.G + g0;  // slot of head 0 of the group
  float* wsp = lds;                        // [16][kFuseMaxSplits] split maxima
  float* plv = wsp + 16 * kFuseMaxSplits;  // [16][kFuseMaxSplits] split sums

  // device-scope (L2-missing) loads of the group's partials and statistics;
  // offsets past the group's slots read as zero
  const __amdgpu_buffer_rsrc_t rp = buf_rsrc(p.pacc + bq0 * ns * D, G * ns * D * 4);
  const __amdgpu_buffer_rsrc_t rm = buf_rsrc(p.pm + bq0 * ns, G * ns * 4);
  const __amdgpu_buffer_rsrc_t rl = buf_rsrc(p.pl + bq0 * ns, G * ns * 4);
  auto load_batch = [&](int h, int sp0, int c, float4_t (&pre)[kPre]) {
#pragma unroll
    for (int j = 0; j < kPre; ++j)
      pre[j] = __builtin_bit_cast(
          float4_t, __builtin_amdgcn_raw_buffer_load_b128(rp, ((h * ns + sp0 + j) * C4 + c) * 16, 0,
                                                          kCachePolicySc1));
  };
  auto task_out = [&](int h, int c, float4_t (&pre)[kPre], bool have0) {
    const float* wh = wsp + h * kFuseMaxSplits;
    const float* lh = plv + h * kFuseMaxSplits;
    float mx = -INFINITY;
    for (int sp = 0; sp < ns; ++sp) mx = fmaxf(mx, wh[sp]);
    const float4_t own = *reinterpret_cast<const float4_t*>(own_acc + h * D + 4 * c);
    float l = 0.f;
    float4_t o = {0.f, 0.f, 0.f, 0.f};
    for (int sp0 = 0; sp0 < ns; sp0 += kPre) {
      if (sp0 > 0 || !have0) load_batch(h, sp0, c, pre);
#pragma unroll
      for (int j = 0; j < kPre; ++j) {
        const int sp = sp0 + j;
        const bool ok = sp < ns;
        const int si = ok ? sp : 0;
        const float pmv = wh[si];
        const float w = (!ok || pmv == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(pmv - mx);
        l = __builtin_fmaf(w, lh[si], l);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = sp == split ? own[i] : (ok ? pre[j][i] : 0.f);
          o[i] = __builtin_fmaf(w, v, o[i]);
        }
      }
    }
    const float iv = 1.0f / l;
    const int64_t ob = b * p.o_sb + (hkv * p.G + g0 + h) * p.o_sh + 4 * c;
    if constexpr (QF32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) static_cast<float*>(p.out)[ob + i] = o[i] * iv;
    } else if (p.q_dtype == FC_F16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) static_cast<f16_t*>(p.out)[ob + i] = from_f32<f16_t>(o[i] * iv);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) static_cast<bf16_t*>(p.out)[ob + i] = from_f32<bf16_t>(o[i] * iv);
    }
  };
  auto stats = [&]() {
    for (int u = tid; u < G * ns; u += kMThreads) {
      const int h = u / ns, sp = u - h * ns;
      const bool own = sp == split;
      const float mv = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rm, u * 4, 0, kCachePolicySc1));
      const float lv = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rl, u * 4, 0, kCachePolicySc1));
      wsp[h * kFuseMaxSplits + sp] = own ? own_m[h] : mv;
      plv[h * kFuseMaxSplits + sp] = own ? own_l[h] : lv;
    }
  };
  if (COMPACT && G * C4 <= kMThreads && ns <= kPre) {
    // one task per thread and at most kPre splits (the common case): the
    // statistics and partials of the task's head come in with one batch of
    // loads, no LDS staging and no barrier (0.33 us shorter than the general
    // form below at C3); same summation order.  Not in the fused step's
    // kernels, where its registers would spill.
    const bool act = tid < G * C4;
    const int h = act ? tid / C4 : 0, c = tid - h * C4;
    float4_t pa[kPre];
    float pmv[kPre], plv[kPre];
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      const int sp = j < ns ? j : 0;
      pa[j] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                               rp, ((h * ns + sp) * C4 + c) * 16, 0, kCachePolicySc1));
      pmv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rm, (h * ns + sp) * 4, 0,
                                                                               kCachePolicySc1));
      plv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, (h * ns + sp) * 4, 0,
                                                                               kCachePolicySc1));
    }
    const float4_t own = *reinterpret_cast<const float4_t*>(own_acc + h * D + 4 * c);
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      if (j == split) pmv[j] = own_m[h];
      if (j == split) plv[j] = own_l[h];
      if (j < ns) mx = fmaxf(mx, pmv[j]);
    }
    float l = 0.f;
    float4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      const float w = (j >= ns || pmv[j] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(pmv[j] - mx);
      l = __builtin_fmaf(w, plv[j], l);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = __builtin_fmaf(w, j == split ? own[i] : pa[j][i], o[i]);
    }
    if (!act) return;
    const float iv = 1.0f / l;
    const int64_t ob = b * p.o_sb + (hkv * p.G + g0 + h) * p.o_sh + 4 * c;
    if constexpr (QF32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) static_cast<float*>(p.out)[ob + i] = o[i] * iv;
    } else if (p.q_dtype == FC_F16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) static_cast<f16_t*>(p.out)[ob + i] = from_f32<f16_t>(o[i] * iv);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) static_cast<bf16_t*>(p.out)[ob + i] = from_f32<bf16_t>(o[i] * iv);
    }
    return;
  }
  float4_t pre[kPre];
  if (G * C4 <= kMThreads) {
    // one task per thread: its first kPre partials fly with the statistics
    const bool act = tid < G * C4;
    const int h = act ? tid / C4 : 0, c = tid - h * C4;
    load_batch(h, 0, c, pre);
    stats();
    __syncthreads();
    if (act) task_out(h, c, pre, true);
    return;
  }
  stats();
  __syncthreads();
  for (int task = tid; task < G * C4; task += kMThreads) {
    const int h = task / C4, c = task - h * C4;
    task_out(h, c, pre, false);
  }
}


// Merge of up to NMAX split partials (NMAX / 2 per thread) for one output
// task of 4 features per pair of adjacent threads (G * D / 4 * 2 <= the
// workgroup's threads): each thread requests its half of the splits'
// partials and statistics in one batch (16-byte loads: at most NMAX / 2 + NMAX
// / 4 loads in flight, within the wavefront's load counter), then the pair
// exchanges its maximum and its sums through a lane shuffle (half 0 + half
// 1, a fixed order).  For the png pass's 32 splits per group.
template <int D, int NMAX, bool QF32>
__device__ __forceinline__ void wide_merge(const MfmaArgs& p, int64_t b, int64_t hkv, int64_t g0,
                                           int G, int split, int tid, const float* own_acc,
                                           const float* own_m, const float* own_l) {
  constexpr int C4 = D / 4;
  constexpr int NH = NMAX / 2;  // splits per thread
  const int ns = p.n_splits;
  const int64_t bq0 = b * (p.Hkv * p.G) + hkv * p.G + g0;
  const int task = tid >> 1, half = tid & 1;
  const bool act = task < G * C4;
  const int h = act ? task / C4 : 0, c = task - h * C4;
  const __amdgpu_buffer_rsrc_t rp = buf_rsrc(p.pacc + bq0 * ns * D, G * ns * D * 4);
  const __amdgpu_buffer_rsrc_t rm = buf_rsrc(p.pm + bq0 * ns, G * ns * 4);
  const __amdgpu_buffer_rsrc_t rl = buf_rsrc(p.pl + bq0 * ns, G * ns * 4);
  const int s0 = half * NH;
  float4_t pa[NH];
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    const int sp = s0 + j < ns ? s0 + j : 0;
    pa[j] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                             rp, ((h * ns + sp) * C4 + c) * 16, 0, kCachePolicySc1));
  }
  // statistics of splits s0 .. s0 + NH - 1 of head h: contiguous (ns % 4 == 0)
  float pmv[NH], plv[NH];
#pragma unroll
  for (int j = 0; j < NH; j += 4) {
    const float4_t m4 = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                       rm, (h * ns + s0 + j) * 4, 0, kCachePolicySc1));
    const float4_t l4 = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                       rl, (h * ns + s0 + j) * 4, 0, kCachePolicySc1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pmv[j + i] = m4[i];
      plv[j + i] = l4[i];
    }
  }
  const float4_t own = *reinterpret_cast<const float4_t*>(own_acc + h * D + 4 * c);
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    if (s0 + j == split) pmv[j] = own_m[h];
    if (s0 + j == split) plv[j] = own_l[h];
    if (s0 + j < ns) mx = fmaxf(mx, pmv[j]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
  float l = 0.f;
  float4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    const float w = (s0 + j >= ns || pmv[j] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(pmv[j] - mx);
    l = __builtin_fmaf(w, plv[j], l);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __builtin_fmaf(w, s0 + j == split ? own[i] : pa[j][i], o[i]);
  }
  // half 0's sums plus half 1's
  const float l1 = __shfl_xor(l, 1, 64);
  float4_t o1;
#pragma unroll
  for (int i = 0; i < 4; ++i) o1[i] = __shfl_xor(o[i], 1, 64);
  if (!act || half != 0) return;
  const float iv = 1.0f / (l + l1);
  const int64_t ob = b * p.o_sb + (hkv * p.G + g0 + h) * p.o_sh + 4 * c;
  if constexpr (QF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) static_cast<float*>(p.out)[ob + i] = (o[i] + o1[i]) * iv;
  } else if (p.q_dtype == FC_F16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) static_cast<f16_t*>(p.out)[ob + i] = from_f32<f16_t>((o[i] + o1[i]) * iv);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) static_cast<bf16_t*>(p.out)[ob + i] = from_f32<bf16_t>((o[i] + o1[i]) * iv);
  }
}

// End of a split-pass workgroup of the matrix-core passes, once its
// wavefronts have parked their (max, sum, accumulator scale) per head in
// comb and their accumulators in cbuf (rows = heads):
//   * combine: thread x of the G * D outputs combines the four wavefronts
//     (and, in split 0, the raw tail's partial from part_lds / tail_ml)
//     into this workgroup's partial (part_lds, wg_ml);
//   * publication, then arrival: every workgroup publishes its partial
//     (device-scope stores), waits until the stores are complete and then
//     counts its arrival on the group's counter.  The one that counts last
//     knows every other partial is complete: it returns the group's
//     counters to zero for the next call and merges (fused_merge), using its
//     own partial from LDS, with no wait.  Ordering: each partial word is
//     written by an agent-scope store, performed at the device's coherence
//     point (not held in the writer XCD's L2), and complete (vmcnt(0))
//     before its writer counts itself; the merge reads partials with
//     agent-scope loads issued after the count has returned, so no load is
//     served by a stale line.  No cache-wide writeback / invalidate is used
//     (each costs ~0.1 us and they serialize per XCD).  Counting first and
//     publishing only from the workgroups that are not last took one more
//     round trip at the end (C3 49.65 -> 49.27 us, C4 50.41 -> 50.05 us with
//     this order).  Without the fused merge the merge runs as its own kernel.
// step_done() runs when the workgroup is finished (the fused step's state
// advance); `scratch` holds the merge's statistics (>= 2 * 16 * 64 floats).
template <int D, int CB, bool QF32, bool COMPACT, typename Done, int WIDE = 0>
__device__ __forceinline__ void split_epilogue(
    const MfmaArgs& p, int64_t g, int64_t b, int64_t hkv, int64_t g0, int G, int split, int tid,
    bool fold_tail, float (&comb)[kWaves][16][3], float (&cbuf)[kWaves][CB][D], float* part_lds,
    float (&tail_ml)[2][16], float (&wg_ml)[2][16], float* scratch, int& s_last,
    unsigned int* passq, Done&& step_done) {
  __syncthreads();
  {
    for (int x = tid; x < G * D; x += kMThreads) {
      const int h = x / D, d = x - h * D;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, comb[w][h][0]);
      float o = 0.f, l = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float mw = comb[w][h][0];
        const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        o = __builtin_fmaf(f * comb[w][h][2], cbuf[w][h][d], o);
        l = __builtin_fmaf(f, comb[w][h][1], l);
      }
      if (fold_tail) {
        // rescale both sums to the common maximum max(M, mt)
        const float mt = tail_ml[0][h];
        const float mm = fmaxf(M, mt);
        const float fw = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - mm);
        const float ft = __builtin_amdgcn_exp2f(mt - mm);
        o = __builtin_fmaf(ft, part_lds[h * D + d], o * fw);
        l = __builtin_fmaf(ft, tail_ml[1][h], l * fw);
        M = mm;
      }
      part_lds[x] = o;
      if (d == 0) {
        wg_ml[0][h] = M;
        wg_ml[1][h] = l;
      }
    }
  }
  // ---- publication, then arrival: every workgroup publishes its partial
  // (with p.fused the last to arrive keeps its own in LDS, but does not know
  // it is last yet), waits for its stores to complete and then counts
  // itself; the workgroup that counts last finds every other partial
  // complete and merges, with no wait
  unsigned int* arrive = p.arrive + g * p.cstride;
  {
    const int64_t bq0 = b * (p.Hkv * p.G) + hkv * p.G + g0;
    for (int x = tid; x < G * D; x += kMThreads) {
      const int h = x / D, d = x - h * D;
      const int64_t slot = (bq0 + h) * p.n_splits + split;
      __hip_atomic_store(p.pacc + slot * D + d, part_lds[x], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
        __hip_atomic_store(p.pm + slot, wg_ml[0][h], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p.pl + slot, wg_ml[1][h], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (!p.fused) {
    if (tid == 0) {
      const unsigned int old = atomicAdd(arrive, 1u);
      if (old + 1 == (unsigned int)p.n_splits) {
        __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(passq, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    return;
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0) {
    const unsigned int old = atomicAdd(arrive, 1u);
    s_last = old + 1 == (unsigned int)p.n_splits ? 1 : 0;
    if (s_last) {
      __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(passq, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  const bool last = s_last != 0;
  if (!last) {
    step_done();
    return;
  }
  if constexpr (WIDE > 0) {
    if (G * (D / 4) * 2 <= kMThreads && p.n_splits <= WIDE && p.n_splits % 4 == 0) {
      wide_merge<D, WIDE, QF32>(p, b, hkv, g0, G, split, tid, part_lds, wg_ml[0], wg_ml[1]);
      step_done();  // every exit counts itself for a state-advancing step
      return;
    }
  }
  fused_merge<D, QF32, COMPACT>(p, b, hkv, g0, G, split, tid, scratch, part_lds, wg_ml[0], wg_ml[1]);
  step_done();
}

// D: head size (64, 80, 96, 128, 256); the products run on DC = D rounded up
// to 64 features: the query's features past D are zero, so the score
// product's code bytes past a row's end (the next row's, or zeros past the
// pass) add nothing, and value-product outputs past D are not kept.
template <int D>
constexpr int mfma_width() {
  return (D + 63) / 64 * 64;
}

// QF: fp32 queries (else fp16 / bf16): the query is split into four int8
// digits (30 bits relative to its head's largest element: the fp32 value
// itself but for elements 2^-7 below the largest), the stored rows' logits
// and their taps are formed in fp64, and each output weight is kept in fp32
// and split into two f16 halves (w = hi + lo / 2^12, 22 bits), so fp32
// outputs keep fp32 accuracy; two more score products and one more value
// product per tile.
template <int SROWS, int D, int GP, bool STEP, bool QF = false, bool QG = false>
__global__ __launch_bounds__(kMThreads, mfma_width<D>() == 256 ? 1 : 2) void attn_split_i8_mfma(
    MfmaArgs p) {
  static_assert(!QG || D % 32 == 0, "per-32 scales: D = 64 / 96 / 128 / 256");
  constexpr int DC = mfma_width<D>();
  constexpr int DK = DC / 32;
  constexpr int DV = (DC + 127) / 128;  // 128-feature groups of the value product
  // rows per wavefront pass: its K codes (NT tiles of 16 rows) and V codes
  // (NS slabs of 32) are in flight while the previous stage computes; a pass
  // holds whole blocks (PR rows of the PRT tile rows; the rest read zero)
  constexpr int PRT = DC == 256 ? 32 : 64;
  constexpr int PR = (PRT / SROWS) * SROWS;
  constexpr int NT = PRT / 16;
  constexpr int NS = PRT / 32;
  constexpr int KDW = 2 * DK;  // K dwords per lane per tile
  static_assert(DK % 2 == 0 && PRT <= kPassRowsW, "feature width");
  __shared__ float s_lds[kWaves][16][kSPad];
  // weights of the pass: fp16 operands, or (QF) fp32 values split into two
  // fp16 operands as they are read
  union WeightLds {
    _Float16 h[kWaves][16][kWPad];
    float f[QF ? kWaves : 1][16][QF ? kSPad : 4];
  };
  __shared__ __attribute__((aligned(16))) WeightLds w_buf;
  auto& w_lds = w_buf.h;
  auto& w_lds_f = w_buf.f;
  __shared__ float sc_lds[kWaves][2][PRT];  // K and V row scales of the pass
  // QG (one scale per 32 features): the pass's K group scales and the V
  // group scales relative to their row's largest (QF: in fp32), by group
  // then row
  constexpr int NGR = QG ? D / 32 : 1;
  using vg_t = std::conditional_t<QF, float, _Float16>;
  __shared__ __attribute__((aligned(16))) float kg_lds[QG ? kWaves : 1][NGR][PRT];
  __shared__ __attribute__((aligned(16))) vg_t vg_lds[QG ? kWaves : 1][NGR][PRT];
  __shared__ float a_lds[FC_MAX_BLOCK * SROWS];
  __shared__ float comb[kWaves][16][3];
  // the wavefronts' accumulators, for the combine (and the fused step's
  // SROWS x D coefficient scratch before the passes)
  constexpr int CB = GP * kWaves >= SROWS ? GP : (SROWS + kWaves - 1) / kWaves;
  __shared__ float cbuf[kWaves][CB][D];
  __shared__ __attribute__((aligned(16))) float part_lds[16 * D];  // raw-tail partial, then this workgroup's partial
  __shared__ float tail_ml[2][16];    // raw-tail (max, sum) per head
  __shared__ float wg_ml[2][16];      // this workgroup's (max, sum) per head
  __shared__ int s_last;
  __shared__ int s_final;

  // 1-D grid, split-major: workgroup L runs split s of group g; the splits of
  // a group are spread over the dispatch order and over the XCDs
  const int64_t L = blockIdx.x;
  const int split = (int)(L / p.ngroups);
  const int64_t g = ((L % p.ngroups) - split % p.ngroups + p.ngroups) % p.ngroups;
  const int64_t bh = g / p.zg;
  const int64_t g0 = (g % p.zg) * 16;
  const int64_t b = bh / p.Hkv, hkv = bh - b * p.Hkv;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, lc = lane & 15;
  const int G = (int)min<int64_t>(16, p.G - g0);  // heads of this group (<= GP)
  const int r = p.r;

  for (int i = tid; i < r * SROWS; i += kMThreads) a_lds[i] = p.A[i];

  // The group's rows are cut into passes of PR rows.  Every wavefront of the
  // group's n_splits workgroups takes its first passes in a fixed order and
  // then the next untaken pass from the group's queue until none is left, so
  // faster wavefronts take more passes.
  int64_t nb = p.nb, n_raw = p.n_raw;
  int64_t step_t = 0, step_nb = 0;  // fused step: tail length and blocks before the token
  bool step_write = false;
  if constexpr (STEP) {
    const int64_t cap = min(p.kcap, p.vcap);
    step_t = p.state ? min<int64_t>(max<int64_t>(p.state[1], 0), p.r - 1) : p.step_t;
    step_nb = p.state ? max<int64_t>(p.state[0], 0) : p.step_nb;
    // one head group per (batch, kv head) stores the token / block; a block
    // past the capacity is not stored (the state's overflow word says so)
    step_write = split == 0 && g0 == 0 && (step_t + 1 < p.r || step_nb < cap);
    nb = min(step_nb, cap);
    n_raw = 0;
  } else if (p.state) {
    // counts of the step's view, kept inside the buffers whatever the words hold
    const int64_t t = min<int64_t>(max<int64_t>(p.state[1], 0), p.r - 1) + 1;
    nb = min<int64_t>(max<int64_t>(p.state[0], 0) + (t == p.r ? 1 : 0), min(p.kcap, p.vcap));
    n_raw = t == p.r ? 0 : t;
  }
  const int64_t rows_total = nb * SROWS;
  const int64_t npass = (rows_total + PR - 1) / PR;
  unsigned int* passq = p.passq + g * p.cstride;
  // fused step: split 0's wavefronts run the step's prologue first and then
  // take passes from the queue only; the other splits' wavefronts take the
  // fixed first passes
  const bool step_q = STEP && p.n_splits > 1 && !p.static_passes;
  const bool step0 = step_q && split == 0;
  const unsigned int wslot = step_q ? (unsigned int)(max(split - 1, 0) * kWaves + wave)
                                    : (unsigned int)(split * kWaves + wave);
  const unsigned int wstride =
      step_q ? (unsigned int)((p.n_splits - 1) * kWaves) : (unsigned int)(p.n_splits * kWaves);
  // Pass k < nfix of a wavefront is fixed, wslot + k * wstride: three
  // quarters of the group's passes need no queue round trip (each queue
  // atomic costs HBM time: one per pass measured 2.2 us slower at C3; the
  // queued quarter still levels the wavefronts' finishing times).  The queue
  // hands out the rest from qbase = nfix * wstride on; in the static order
  // every pass is fixed.  The fused step's kernels keep the queue for every
  // pass after the first (the fixed order's registers spilled there).
  const unsigned int nfix = (unsigned int)max<int64_t>(1, 3 * npass / (4 * (int64_t)wstride));
  const unsigned int qbase = STEP ? wstride : wstride * nfix;  // first queued pass
  unsigned int next_fixed = wslot + wstride;
  auto grab = [&]() -> unsigned int {  // result in lane 0, read when needed
    const unsigned int f = next_fixed;
    next_fixed += wstride;
    if (!step0 && (p.static_passes || f < qbase)) return f;
    unsigned int v = 0;
    if (lane == 0)
      v = __hip_atomic_fetch_add(passq, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + qbase;
    return v;
  };
  auto pass_of = [](unsigned int v) { return (int64_t)__builtin_amdgcn_readfirstlane((int)v); };

  const int8_t* kbase = p.kcodes + bh * p.kcap * SROWS * D;
  const int8_t* vbase = p.vcodes + bh * p.vcap * SROWS * D;
  const float* ksc = p.kscales + bh * p.kcap * SROWS * NGR;
  const float* vsc = p.vscales + bh * p.vcap * SROWS * NGR;

  // ---- queries: B operand of the score product.  Lane (q, c): head c,
  // features q*D/4 + 8*kc + i of product kc, scaled per head by a power of two
  const bool hq_ok = lc < G;
  const int64_t hq = hkv * p.G + g0 + (hq_ok ? lc : 0);
  // lane (q, c) holds features 64 k + 16 q + [0, 16) of chunk k
  const int64_t qoff = b * p.q_sb + hq * p.q_sh + 16 * lq;
  const bool q_f16 = p.q_dtype == FC_F16;
  // the query's loads go out first; it is converted after the first pass's
  // K loads have been issued behind them.  8 features per kc: one 16-byte
  // load of fp16 / bf16, two of fp32.
  constexpr int QW = QF ? 2 : 1;
  u32x4_t qraw[DK][QW];
#pragma unroll
  for (int kc = 0; kc < DK; ++kc) {
    // features past D (D = 80, 96) are not loaded and stay zero
    const int f0 = 64 * (kc / 2) + 16 * lq + 8 * (kc % 2);
    const int64_t e0 = qoff + 64 * (kc / 2) + 8 * (kc % 2);
#pragma unroll
    for (int u = 0; u < QW; ++u) {
      qraw[kc][u] = (u32x4_t){0u, 0u, 0u, 0u};
      if (D % 64 == 0 || f0 < D) {
        if constexpr (QF)
          qraw[kc][u] = *reinterpret_cast<const u32x4_t*>(static_cast<const float*>(p.q) + e0 + 4 * u);
        else
          qraw[kc][u] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p.q) + e0);
      }
    }
  }

  float4_t acc[DV][8];
#pragma unroll
  for (int dv = 0; dv < DV; ++dv)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[dv][e] = (float4_t){0.f, 0.f, 0.f, 0.f};
  // Head (lane % GP): reference max m_run (identical in all lanes of a head)
  // and this lane's share of the exponential sum, both relative to m_run.
  // The accumulators hold acc * 2^-sig_run.  Both references move only when
  // a logit exceeds m_run + kLazyMax or a V row scale reaches 2^(sig_run+1).
  const int myh = lane % GP;
  float m_run = -INFINITY, l_lane = 0.f;
  int sig_run = -1000;
  float wmul_run = INFINITY;  // 2^-sig_run

  // loop-invariant lane offsets (bytes) of the pass loads
  const int k_off = lc * D + 16 * lq;
  int v_off[DV];
#pragma unroll
  for (int dv = 0; dv < DV; ++dv) v_off[dv] = 8 * lq * D + min(128 * dv + 8 * lc, D - 8);
  const int sc_off = (lane % PRT) * 4;

  uint32_t kr[NT][KDW];
  float ks_r, vs_r;
  float kgr[NGR], vgr[NGR];  // QG: the group scales of row lane % PRT
  const int sg_off = (lane % PRT) * NGR * 4;
  // QG: the NGR group scales of row lane % PRT, in 16 / 8-byte pieces (NGR
  // = 2, 4, 8) or dwords (NGR = 3: rows 12 bytes apart)
  auto load_groups = [&](__amdgpu_buffer_rsrc_t rs, float* dst) {
    if constexpr (NGR % 4 == 0) {
#pragma unroll
      for (int u = 0; u < NGR / 4; ++u) {
        const u32x4_t a = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, sg_off + 16 * u, 0, 0));
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[4 * u + i] = __uint_as_float(a[i]);
      }
    } else if constexpr (NGR == 2) {
      const u32x2_t a = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rs, sg_off, 0, 0));
#pragma unroll
      for (int i = 0; i < 2; ++i) dst[i] = __uint_as_float(a[i]);
    } else {
#pragma unroll
      for (int i = 0; i < NGR; ++i)
        dst[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, sg_off + 4 * i, 0, 0));
    }
  };
  // Code rows are read once per call: streaming (nontemporal) loads for K and
  // V, so the archive does not displace what the end phase needs from the
  // caches (C3 over rotating archive sets: 50.6 -> 49.9 us; the row scales
  // stay on the default policy, streaming them measured slower)
  auto load_k = [&](int64_t pr0, int prow) {
    // group scales ahead of the codes: the score stage needs them first
    if constexpr (QG) load_groups(buf_rsrc(ksc + pr0 * NGR, prow * NGR * 4), kgr);
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(kbase + pr0 * D, prow * D);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < DK / 2; ++h) {
        const u32x4_t v = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, k_off + 16 * t * D + 64 * h, 0,
                                                           kCachePolicyNt));
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[t][4 * h + i] = v[i];
      }
    if constexpr (!QG) {
      ks_r = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           buf_rsrc(ksc + pr0, prow * 4), sc_off, 0, 0));
      vs_r = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           buf_rsrc(vsc + pr0, prow * 4), sc_off, 0, 0));
    }
  };
  uint32_t vr[NS][DV][16];
  auto load_v = [&](int64_t pr0, int prow) {
    // group scales ahead of the codes, with this pass's V (held one pass
    // ahead with the K loads they cost registers that spilled)
    if constexpr (QG) load_groups(buf_rsrc(vsc + pr0 * NGR, prow * NGR * 4), vgr);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vbase + pr0 * D, prow * D);
#pragma unroll
    for (int sl = 0; sl < NS; ++sl)
#pragma unroll
      for (int dv = 0; dv < DV; ++dv)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const u32x2_t v = __builtin_bit_cast(
              u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
                           rv, v_off[dv] + (32 * sl + i) * D, 0, kCachePolicyNt));
          vr[sl][dv][2 * i] = v[0];
          vr[sl][dv][2 * i + 1] = v[1];
        }
  };

  // Output weights of the pass's (block, head) pairs, exponentials relative
  // to mref, scaled by the V row scale * wm, into w_lds; returns this lane's
  // largest logit and exponential sum.
  auto weights = [&](int prow, float mref, float wm, float& pmax, float& lsum) {
    pmax = -INFINITY;
    lsum = 0.f;
    if (myh >= G) return;
    const int npair = (prow / SROWS) * GP;
    for (int u = lane; u < npair; u += 64) {
      const int row0 = (u / GP) * SROWS;
      // QF: the stored rows' logits and their taps in fp64 (the logits of
      // stored rows reach hundreds; fp32 roundings there are 1e-5 absolute)
      using sv_t = std::conditional_t<QF, double, float>;
      sv_t sv[SROWS];
      float w[SROWS];
#pragma unroll
      for (int j = 0; j < SROWS; ++j) {
        if constexpr (QF)
          sv[j] = (double)s_lds[wave][myh][row0 + j] *
                  ((double)sc_lds[wave][0][row0 + j] * (double)p.scale_log2);
        else
          sv[j] = s_lds[wave][myh][row0 + j] * sc_lds[wave][0][row0 + j];
        w[j] = 0.f;
      }
      auto tap = [&](int t) {
        float lg, d;
        if constexpr (QF) {
          double lgd = 0.0;
#pragma unroll
          for (int j = 0; j < SROWS; ++j) lgd = __builtin_fma((double)a_lds[t * SROWS + j], sv[j], lgd);
          lg = (float)lgd;
          d = (float)(lgd - (double)mref);
        } else {
          lg = 0.f;
#pragma unroll
          for (int j = 0; j < SROWS; ++j) lg = __builtin_fmaf(a_lds[t * SROWS + j], sv[j], lg);
          d = lg - mref;
        }
        pmax = fmaxf(pmax, lg);
        const float e = __builtin_amdgcn_exp2f(d);
        lsum += e;
#pragma unroll
        for (int j = 0; j < SROWS; ++j) w[j] = __builtin_fmaf(e, a_lds[t * SROWS + j], w[j]);
      };
      // taps unrolled up to 4 stored rows (with 8, or the fp64 taps of fp32
      // queries, the unrolled taps' A coefficients no longer fit the registers)
      if (!QF && SROWS <= 4 && r <= kTapsUnrolled) {
#pragma unroll
        for (int t = 0; t < kTapsUnrolled; ++t)
          if (t < r) tap(t);
      } else {
        for (int t = 0; t < r; ++t) tap(t);
      }
#pragma unroll
      for (int j = 0; j < SROWS; ++j)
      {
        const float wv = w[j] * (sc_lds[wave][1][row0 + j] * wm);
        if constexpr (QF)
          w_lds_f[wave][myh][row0 + j] = wv;
        else
          w_lds[wave][myh][row0 + j] = (_Float16)wv;
      }
    }
  };

  // The first pass's K loads go out right behind the query's: its prologue
  // waits for the query only.  (Issuing the first V loads here as well
  // measured slower: 16 KB per wavefront requested at once at the start.)
  // A fused step issues them after its step partial, whose registers they
  // would otherwise share.
  auto rows_of = [&](int64_t pass) { return (int)min<int64_t>(PR, rows_total - pass * PR); };
  int64_t cur = step0 ? npass : wslot;
  bool v_first = false;  // the first pass's V codes are in flight already
  if (!step0 && (!STEP || step_q) && cur < npass) {
    load_k(cur * PR, rows_of(cur));
    if constexpr (STEP) {
      load_v(cur * PR, rows_of(cur));
      v_first = true;
    }
  }

  // ---- the query as the B operand: per head a power of two scales it to
  // integers of at most 14 bits (QF: 30 bits)
  float qf[DK][8];
  float qmax = 0.f;
  // dtype branch outside the loops; fp16 lanes are read through a half8 view
  // (hipcc 7.2 reused dword 0's conversion for all dwords when each dword was
  // bit-cast to half2 inside an unrolled loop)
#pragma unroll
  for (int kc = 0; kc < DK; ++kc) {
    const u32x4_t raw = qraw[kc][0];
    if constexpr (QF) {
#pragma unroll
      for (int i = 0; i < 8; ++i) qf[kc][i] = __uint_as_float(qraw[kc][i / 4][i % 4]);
    } else if (q_f16) {
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
  // 14-bit integer query per head (largest magnitude in [2^13, 2^14)), split
  // q' = 256 * hi + lo into two int8 operands: scores are exact integers
  // 256 * (K . hi) + (K . lo) from the int8 matrix cores
  // (QF: 30-bit integers, q' = sum_i 256^i d_i over four int8 digits d_i)
  constexpr int ND = QF ? 4 : 2;  // digits
  const int qe = pow2_exp_for(qmax, QF ? 30 : 14);
  constexpr int NC = DC / 64;  // 64-feature chunks of the score product
  i32x4_t qdig[ND][NC];        // qdig[0]: the lowest digit
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t dw[ND];
#pragma unroll
      for (int i = 0; i < ND; ++i) dw[i] = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 16 * c + 4 * w + j;  // feature 64c + 16q + 4w + j
        int qi = (int)rintf(ldexpf(qf[e / 8][e % 8], -qe));
#pragma unroll
        for (int i = 0; i < ND - 1; ++i) {  // balanced digits: each in [-128, 127]
          const int d = (int)(int8_t)(qi & 0xff);
          dw[i] |= (uint32_t)(d & 0xff) << (8 * j);
          qi = (qi - d) >> 8;
        }
        dw[ND - 1] |= (uint32_t)(qi & 0xff) << (8 * j);
      }
#pragma unroll
      for (int i = 0; i < ND; ++i) qdig[i][c][w] = (int)dw[i];
    }
  const float head_mul = ldexpf(p.scale_log2, qe);  // integer score -> base-2 logit / K scale

  // raw tail (fused calls): split 0 computes its partial before the passes
  // and folds it into its own, so the final merge reads partials only; in a
  // fused step that partial covers the rows the step adds
  const bool fold_tail = p.fused && split == 0 && (STEP || n_raw > 0);
  if constexpr (STEP) {
    if (split == 0) {
      __shared__ float step_sc[SROWS * NGR];
      float* xk = &s_lds[0][0][0];  // the pass loop has not started: its scratch is free
      float* etl = reinterpret_cast<float*>(&w_lds[0][0][0]);
      const int64_t bh_s = b * p.Hkv + hkv;
      const int64_t kblk = (bh_s * p.kcap + step_nb) * SROWS, vblk = (bh_s * p.vcap + step_nb) * SROWS;
      auto go = [&](auto tt) {
        using TT = decltype(tt);
        step_partial<D, SROWS, TT, NGR>(
            step_t, p.r, static_cast<TT*>(const_cast<void*>(p.kraw)) + bh_s * p.r * D,
            static_cast<TT*>(const_cast<void*>(p.vraw)) + bh_s * p.r * D,
            static_cast<const TT*>(p.ktok) + b * p.kt_sb + hkv * p.kt_sh,
            static_cast<const TT*>(p.vtok) + b * p.vt_sb + hkv * p.vt_sh, step_write,
            p.kcodes_w + kblk * D, p.kscales_w + kblk * NGR, p.vcodes_w + vblk * D,
            p.vscales_w + vblk * NGR,
            p.basis, p.A, p.q, p.q_dtype, b * p.q_sb, p.q_sh, hkv * p.G + g0, G, p.scale_log2,
            tid, xk, xk + p.r * D, cbuf[0][0], step_sc, etl, part_lds, tail_ml[0], tail_ml[1]);
      };
      if (p.raw_dtype == FC_F16)
        go(f16_t{});
      else if (p.raw_dtype == FC_BF16)
        go(bf16_t{});
      else
        go(float{});
    }
  } else if (fold_tail) {
    raw_tail_partial<D, QF>(p, b, hkv, g0, G, (int)n_raw, tid,
                        reinterpret_cast<float*>(&w_lds[0][0][0]), part_lds, tail_ml[0],
                        tail_ml[1]);
  }

  __syncthreads();  // a_lds; the tail's scratch (w_lds) is free again
  if (step0) {
    // split 0's first pass: the queue's next, after its step prologue
    unsigned int v = 0;
    if (lane == 0)
      v = __hip_atomic_fetch_add(passq, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + wstride;
    cur = pass_of(v);
  }
  if (STEP && (step0 || !step_q) && cur < npass) load_k(cur * PR, rows_of(cur));
  while (cur < npass) {
    const int64_t pr0 = cur * PR;
    const int prow = rows_of(cur);  // multiple of SROWS
    if (!v_first) load_v(pr0, prow);
    v_first = false;
    // the next pass, taken now and read after the score products (a wavefront
    // holds at most one pass beyond the current one)
    const unsigned int nxt_v = grab();

    // ------------------------------------------------------------ scores
    if constexpr (QG) {
      if (lane < PRT) {
#pragma unroll
        for (int i = 0; i < NGR; ++i) kg_lds[wave][i][lane] = kgr[i];
      }
      wave_lds_sync();
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if constexpr (QG) {
        // per 32-feature group: one score product (lanes q < 2 hold group 2c
        // of chunk c, q >= 2 group 2c + 1), scaled by the rows' group scales
        // (QF: the group's exact digit sums joined in fp32, as the per-row
        // pass joins them)
        float4_t accg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const i32x4_t a = {(int)kr[t][4 * c], (int)kr[t][4 * c + 1], (int)kr[t][4 * c + 2],
                             (int)kr[t][4 * c + 3]};
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            if (2 * c + hf >= NGR) continue;  // D = 96: features 96.. are padding
            // the codes of the other group's lanes zeroed (the query stays
            // whole: a masked copy of it would be hoisted out of the loop)
            const bool mine = (lq >> 1) == hf;
            const i32x4_t am = mine ? a : (i32x4_t){0, 0, 0, 0};
            i32x4_t sd[ND];
#pragma unroll
            for (int i = 0; i < ND; ++i)
              sd[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, qdig[i][c], (i32x4_t){0, 0, 0, 0}, 0, 0, 0);
            const float4_t kgv =
                *reinterpret_cast<const float4_t*>(&kg_lds[wave][2 * c + hf][16 * t + 4 * lq]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if constexpr (QF) {
                float v = (float)sd[ND - 1][i];
#pragma unroll
                for (int k = ND - 2; k >= 0; --k) v = __builtin_fmaf(v, 256.f, (float)sd[k][i]);
                accg[i] = __builtin_fmaf(kgv[i], v, accg[i]);
              } else {
                accg[i] = __builtin_fmaf(kgv[i], (float)(sd[1][i] * 256 + sd[0][i]), accg[i]);
              }
            }
          }
        }
        if constexpr (QF) {
#pragma unroll
          for (int i = 0; i < 4; ++i) accg[i] = ldexpf(accg[i], qe);  // the scale follows in fp64
        } else {
          accg *= head_mul;
        }
        if (lc < G) *reinterpret_cast<float4_t*>(&s_lds[wave][lc][16 * t + 4 * lq]) = accg;
        continue;
      }
      i32x4_t sd[ND];
#pragma unroll
      for (int i = 0; i < ND; ++i) sd[i] = (i32x4_t){0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        // lane (q, m): row m, features 64c + 16q .. +15, straight from the load
        const i32x4_t a = {(int)kr[t][4 * c], (int)kr[t][4 * c + 1], (int)kr[t][4 * c + 2],
                           (int)kr[t][4 * c + 3]};
#pragma unroll
        for (int i = 0; i < ND; ++i)
          sd[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qdig[i][c], sd[i], 0, 0, 0);
      }
      if (lc < G) {
        float4_t sv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (QF) {  // the digits' sums are exact; their weighted sum in fp32
            float acc_s = (float)sd[ND - 1][i];
#pragma unroll
            for (int k = ND - 2; k >= 0; --k) acc_s = __builtin_fmaf(acc_s, 256.f, (float)sd[k][i]);
            sv[i] = ldexpf(acc_s, qe);  // exact; the scales follow in fp64
          } else {
            sv[i] = (float)(sd[1][i] * 256 + sd[0][i]) * head_mul;
          }
        }
        *reinterpret_cast<float4_t*>(&s_lds[wave][lc][16 * t + 4 * lq]) = sv;
      }
    }
    if constexpr (QG) {
      // V group scales relative to the row's largest (that one joins the
      // output weights as the row scale)
      float vmax = 0.f;
#pragma unroll
      for (int i = 0; i < NGR; ++i) vmax = fmaxf(vmax, vgr[i]);
      const float rv = vmax > 0.f ? __builtin_amdgcn_rcpf(vmax) : 0.f;
      if (lane < PRT) {
#pragma unroll
        for (int i = 0; i < NGR; ++i) {
          if constexpr (QF)
            vg_lds[wave][i][lane] = vmax > 0.f ? vgr[i] / vmax : 0.f;
          else
            vg_lds[wave][i][lane] = (_Float16)(vgr[i] * rv);
        }
      }
      ks_r = 1.f;
      vs_r = vmax;
    }
    if (lane < PRT) {
      sc_lds[wave][0][lane] = ks_r;
      sc_lds[wave][1][lane] = vs_r;
    }
    // a V row scale past the headroom of the current exponent forces a rescale
    const bool sig_need = vs_r * wmul_run >= 2.0f;
    const float vs_pass = vs_r;
    // next pass's K codes and scales fly during the softmax and value stages
    const int64_t nxt = pass_of(nxt_v);
    if (nxt < npass) load_k(nxt * PR, rows_of(nxt));
    wave_lds_sync();

    // ------------------------------------------------------------ softmax
    float pmax, lsum;
    weights(prow, m_run, wmul_run, pmax, lsum);
    const bool m_need = pmax > m_run + kLazyMax;
    if (__builtin_amdgcn_ballot_w64(sig_need || m_need) != 0) {
      // move the references: V exponent from the pass's largest row scale,
      // head maxima from the pass's logits; recompute the weights
      float smax = vs_pass;
#pragma unroll
      for (int m = 1; m < 64; m <<= 1) smax = fmaxf(smax, __shfl_xor(smax, m, 64));
      const int sig_new = max(sig_run, pow2_exp_for(smax, 1));
#pragma unroll
      for (int m = GP; m < 64; m <<= 1) pmax = fmaxf(pmax, __shfl_xor(pmax, m, 64));
      const float m_new = fmaxf(m_run, pmax);
      const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      const float wm = ldexpf(1.0f, -sig_new);
      float pdummy;
      weights(prow, m_new, wm, pdummy, lsum);
      l_lane = l_lane * alpha + lsum;
      // lane (q, c) register i holds head 4q + i
      const float sfix = ldexpf(1.0f, sig_run - sig_new);
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * lq + i, 64) * sfix;
#pragma unroll
      for (int dv = 0; dv < DV; ++dv)
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[dv][e][i] *= al[i];
      m_run = m_new;
      sig_run = sig_new;
      wmul_run = wm;
    } else {
      l_lane += lsum;
    }
    // rows past the pass end carry zero weight (their codes read as zero)
    if (prow < PRT)
      for (int i = prow + lane; i < PRT; i += 64)
        for (int h = 0; h < G; ++h) {
          if constexpr (QF)
            w_lds_f[wave][h][i] = 0.f;
          else
            w_lds[wave][h][i] = (_Float16)0.f;
        }
    wave_lds_sync();

    // ------------------------------------------------------------ values
    if constexpr (QF && QG) {
      // fp32 weights by fp32 values (codes times their group scale relative
      // to the row's largest, one rounding): v_mfma_f32_16x16x4_f32, row
      // 32 sl + 8 q + m of the pass as k = q of instruction m; lane (q, c)
      // holds column c (feature 128 dv + 8 c + e) of its rows 8q .. 8q+7
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
        float4_t f0 = *reinterpret_cast<const float4_t*>(&w_lds_f[wave][lc][32 * sl + 8 * lq]);
        float4_t f1 = *reinterpret_cast<const float4_t*>(&w_lds_f[wave][lc][32 * sl + 8 * lq + 4]);
        if (lc >= G) f0 = f1 = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dv = 0; dv < DV; ++dv) {
          const int gi = min(4 * dv + lc / 4, NGR - 1);
          const float4_t r0 = *reinterpret_cast<const float4_t*>(&vg_lds[wave][gi][32 * sl + 8 * lq]);
          const float4_t r1 = *reinterpret_cast<const float4_t*>(&vg_lds[wave][gi][32 * sl + 8 * lq + 4]);
#pragma unroll
          for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int m = 0; m < 8; ++m) {
              // code + 128 as an unsigned byte; (u - 128) * rat in one fma
              const uint32_t u = (vr[sl][dv][2 * m + e / 4] ^ 0x80808080u) >> (8 * (e % 4));
              const float rt = m < 4 ? r0[m] : r1[m - 4];
              const float bv = __builtin_fmaf((float)(u & 0xffu), rt, -128.0f * rt);
              acc[dv][e] = __builtin_amdgcn_mfma_f32_16x16x4f32(m < 4 ? f0[m] : f1[m - 4], bv,
                                                                acc[dv][e], 0, 0, 0);
            }
        }
      }
      wave_lds_sync();
      cur = nxt;
      continue;
    }
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
      half8_t wop, wop_lo = {};
      if constexpr (QF) {
        // w = hi + lo / 2^12: the low half scaled by 2^12 stays a normal
        // f16 down to |w| ~ 2^-14 (its value operand carries the 2^-12)
        float4_t f0 = *reinterpret_cast<const float4_t*>(&w_lds_f[wave][lc][32 * sl + 8 * lq]);
        float4_t f1 = *reinterpret_cast<const float4_t*>(&w_lds_f[wave][lc][32 * sl + 8 * lq + 4]);
        if (lc >= G) f0 = f1 = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float x = k < 4 ? f0[k] : f1[k - 4];
          const _Float16 hi = (_Float16)x;
          wop[k] = hi;
          wop_lo[k] = (_Float16)((x - (float)hi) * kLoScale);
        }
      } else {
        u32x4_t wa = *reinterpret_cast<const u32x4_t*>(&w_lds[wave][lc][32 * sl + 8 * lq]);
        if (lc >= G) wa = (u32x4_t){0u, 0u, 0u, 0u};
        wop = __builtin_bit_cast(half8_t, wa);
      }
#pragma unroll
      for (int dv = 0; dv < DV; ++dv) {
        // QG: column c holds features 128 dv + 8 c + e, group 4 dv + c / 4
        // (clamped: columns past D are dropped); the codes of rows 8q .. 8q+7
        // times their group scale relative to the row's largest
        half8_t rat = {};
        if constexpr (QG)
          rat = *reinterpret_cast<const half8_t*>(
              &vg_lds[wave][min(4 * dv + lc / 4, NGR - 1)][32 * sl + 8 * lq]);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          // row pair (a, b) = (2pp, 2pp+1): t0 = [a0 b0 a1 b1], t1 = [a2 b2 a3 b3]
          uint32_t t0[4], t1[4];
#pragma unroll
          for (int pp = 0; pp < 4; ++pp) {
            const uint32_t ra = vr[sl][dv][2 * (2 * pp) + hh] ^ 0x80808080u;
            const uint32_t rb = vr[sl][dv][2 * (2 * pp + 1) + hh] ^ 0x80808080u;
            t0[pp] = __builtin_amdgcn_perm(rb, ra, 0x05010400u);
            t1[pp] = __builtin_amdgcn_perm(rb, ra, 0x07030602u);
          }
#pragma unroll
          for (int ee = 0; ee < 4; ++ee) {
            // the operand is built in place as one 4-dword vector (no copies)
            half8_t ov;
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const uint32_t src = ee < 2 ? t0[pp] : t1[pp];
              const uint32_t sel = (ee & 1) ? 0x04030402u : 0x04010400u;
              const half2_t h2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, src, sel)) +
                                 (half2_t){(_Float16)-1152.0f, (_Float16)-1152.0f};
              ov[2 * pp] = h2[0];
              ov[2 * pp + 1] = h2[1];
            }
            const int e = 4 * hh + ee;
            if constexpr (QG) ov *= rat;
            if constexpr (QF) {  // codes times 2^-12: exact in f16
              const half8_t ovl = ov * (_Float16)(1.0f / kLoScale);
              acc[dv][e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop_lo, ovl, acc[dv][e], 0, 0, 0);
            }
            acc[dv][e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop, ov, acc[dv][e], 0, 0, 0);
          }
        }
      }
    }
    wave_lds_sync();
    cur = nxt;
  }

  // ---- combine the wavefronts.  Each wavefront parks its (max, sum,
  // 2^sig_run) per head and its accumulators in its own LDS region; after one
  // barrier thread x of the G * D outputs combines them (lane (q, c) of a
  // wavefront carries head c's statistics; its register i holds head 4q + i).
#pragma unroll
  for (int m = GP; m < 64; m <<= 1) l_lane += __shfl_xor(l_lane, m, 64);
  if (lane < GP) {
    comb[wave][lane][0] = m_run;
    comb[wave][lane][1] = l_lane;
    comb[wave][lane][2] = ldexpf(1.0f, sig_run);
  }
  // One predicate per lane, not per element (per-element conditions became a
  // branch per store): lanes whose registers hold heads < GP (rows of
  // cbuf; heads in [G, GP) carry zeros and are never read) and features < D.
  constexpr int NI = GP < 4 ? GP : 4;  // accumulator registers that can hold a head
  if (lq < (GP >= 4 ? GP / 4 : 1) && (D % 128 == 0 || lc < D / 8)) {
#pragma unroll
    for (int dv = 0; dv < DV; ++dv)
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int i = 0; i < NI; ++i) cbuf[wave][4 * lq + i][128 * dv + 8 * lc + e] = acc[dv][e][i];
  }
  // fused step with a device state: the launch's last workgroup to finish
  // (all others have read the state by then) advances it
  auto step_done = [&]() {
    if constexpr (!STEP) return;
    if (!p.state) return;
    if (tid == 0) s_final = atomicAdd(p.done, 1u) + 1 == gridDim.x ? 1 : 0;
    __syncthreads();
    if (s_final && tid < 64) {  // lane-indexed vector stores
      const int64_t cap = min(p.kcap, p.vcap);
      const bool full = step_t + 1 == p.r;
      const bool over = full && step_nb >= cap;
      const int64_t word = tid == 0   ? (full ? step_nb + 1 : step_nb)
                           : tid == 1 ? (full ? 0 : step_t + 1)
                                      : ((p.state[2] != 0 || over) ? 1 : 0);
      if (tid < 3) const_cast<int64_t*>(p.state)[tid] = word;
      if (tid == 0) __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  split_epilogue<D, CB, QF, !STEP>(p, g, b, hkv, g0, G, split, tid, fold_tail, comb, cbuf,
                                      part_lds,
                               tail_ml, wg_ml, &s_lds[0][0][0], s_last, passq, step_done);
}

template <int... Vs, typename F>
int mfma_with_int(int v, F&& f) {
  int rc = FC_ERR_UNSUPPORTED;
  bool hit = false;
  ((v == Vs ? (rc = f(std::integral_constant<int, Vs>{}), hit = true) : false), ...);
  return hit ? rc : FC_ERR_UNSUPPORTED;
}

// stored rows per block and head sizes the matrix-core pass is built for
#define FC_MFMA_ROWS_LIST 1, 2, 3, 4, 8
#define FC_MFMA_HEAD_DIMS 64, 80, 96, 128, 256

// Launch of the split pass with SR stored rows per block, dispatched on the
// head size and the head-group size: one scale per row (launch_mfma_rows)
// or per 32 features (launch_mfma_rows_g).  Each SR and scale layout is
// instantiated in a translation unit of its own (fc_attn_mfma_s<SR>.hip,
// fc_attn_mfma_g<SR>.hip).
template <int SR>
int launch_mfma_rows(const MfmaArgs& a, int d, int gp, dim3 grid, hipStream_t st) {
  return mfma_with_int<FC_MFMA_HEAD_DIMS>(d, [&](auto dc) {
    constexpr int Dv = decltype(dc)::value;
    return mfma_with_int<1, 2, 4, 8, 16>(gp, [&](auto gc) {
      constexpr int GPv = decltype(gc)::value;
      if (a.step && a.q_dtype == FC_F32) {
        attn_split_i8_mfma<SR, Dv, GPv, true, true><<<grid, kMThreads, 0, st>>>(a);
      } else if (a.step) {
        attn_split_i8_mfma<SR, Dv, GPv, true><<<grid, kMThreads, 0, st>>>(a);
      } else if (a.q_dtype == FC_F32) {
        attn_split_i8_mfma<SR, Dv, GPv, false, true><<<grid, kMThreads, 0, st>>>(a);
      } else {
        attn_split_i8_mfma<SR, Dv, GPv, false><<<grid, kMThreads, 0, st>>>(a);
      }
      return FC_OK;
    });
  });
}

template <int SR>
int launch_mfma_rows_g(const MfmaArgs& a, int d, int gp, dim3 grid, hipStream_t st) {
  return mfma_with_int<64, 96, 128, 256>(d, [&](auto dc) {
    constexpr int Dv = decltype(dc)::value;
    return mfma_with_int<1, 2, 4, 8, 16>(gp, [&](auto gc) {
      constexpr int GPv = decltype(gc)::value;
      if (a.step && a.q_dtype == FC_F32) {
        attn_split_i8_mfma<SR, Dv, GPv, true, true, true><<<grid, kMThreads, 0, st>>>(a);
      } else if (a.step) {
        attn_split_i8_mfma<SR, Dv, GPv, true, false, true><<<grid, kMThreads, 0, st>>>(a);
      } else if (a.q_dtype == FC_F32) {
        attn_split_i8_mfma<SR, Dv, GPv, false, true, true><<<grid, kMThreads, 0, st>>>(a);
      } else {
        attn_split_i8_mfma<SR, Dv, GPv, false, false, true><<<grid, kMThreads, 0, st>>>(a);
      }
      return FC_OK;
    });
  });
}

#define FC_MFMA_EXTERN(SR)                                                                 \
  extern template int launch_mfma_rows<SR>(const MfmaArgs&, int, int, dim3, hipStream_t); \
  extern template int launch_mfma_rows_g<SR>(const MfmaArgs&, int, int, dim3, hipStream_t);
FC_MFMA_EXTERN(1)
FC_MFMA_EXTERN(2)
FC_MFMA_EXTERN(3)
FC_MFMA_EXTERN(4)
FC_MFMA_EXTERN(8)
#undef FC_MFMA_EXTERN

}  // namespace fc
