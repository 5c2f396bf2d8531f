// Matrix-core split pass of the decode attention over jpeg archives of
// floating-point coefficients (FC_STORE_JPEG_FP: (B, H, cap, k, D) rows in
// the stream dtype, the reference's default codec, quant_bits = 0;
// flashcodec/attention.py:45-61, 101-140), fp16 or bf16 rows queried in the
// same dtype.
//
// The structure of the int8 pass (fc_attn_mfma_kernel.h): a group (batch, kv
// head, up to 16 query heads) cut into passes of PR rows, three quarters of
// each wavefront's passes in a fixed order and the rest from the group's
// queue, the next pass's K rows requested after the score products, the
// shared end phase (combine, publication, arrival, fused merge).  A pass is
// 8 KiB of rows per stream: 32 rows at D = 128, 64 at D = 64.
//   scores: v_mfma_f32_16x16x32_{f16,bf16} straight on the rows: lane (q, m)
//      holds features 32c + 8q .. +7 of row m of a 16-row tile (16-byte
//      loads: 64 contiguous bytes of each row per load instruction), the
//      query group the same features of head c as the B operand; products
//      are exact and summed in fp32;
//   softmax: (block, head) pairs over the lanes, r logits from the k scores
//      through A, exponentials against a running reference maximum that
//      moves only when a logit exceeds it by 2^8, the stored rows' weights
//      sum_t e_t A[t][j] (no row scales: the rows are the coefficients);
//   values: W (16 heads x 32 rows) by the rows (32 rows x 16 features): lane
//      (q, c) loads rows 8q .. 8q+7 of features 8c .. 8c+7 and forms the
//      operand of feature 8c + e from their 16-bit halves with v_perm_b32
//      (no conversion).  fp16: the weights as f16 (2^-11 relative, as the
//      int8 pass); bf16: the weights split w = hi + lo into two bf16
//      operands (16 bits), two products.
// STEP: the one-launch decode step, as the int8 pass's: split 0's
// workgroups append the step's tokens to the tails (or archive the block
// they complete: the coefficients rounded to the stream dtype, the fp
// archive kernel's arithmetic, stored in place) and attend the step's rows
// at full precision before their passes.
#include "fc_attn_mfma_kernel.h"

namespace fc {

// fp32 coefficient rows take the png pass's fp32 products (JPG variant of
// attn_split_png_mfma, launched from fc_attn_png.hip)
int launch_fpj32_t(const MfmaArgs& a, int s, int D, int gp, dim3 grid, hipStream_t st);

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

template <int SROWS, int D, int GP, bool BF, bool STEP>
__global__ __launch_bounds__(kMThreads, 2) void attn_split_fpj_mfma(MfmaArgs p) {
  static_assert(D == 64 || D == 128, "head size");
  using T = std::conditional_t<BF, bf16_t, f16_t>;
  constexpr int NC = D / 32;                      // 32-feature chunks of a score product
  constexpr int PRT = D == 64 ? 64 : 32;          // tile rows of a pass (8 KiB per stream)
  constexpr int PR = (PRT / SROWS) * SROWS;       // whole blocks
  constexpr int NT = PRT / 16;                    // score tiles
  constexpr int NS = PRT / 32;                    // value slabs
  __shared__ float s_lds[kWaves][16][kSPad];
  union WeightLds {
    _Float16 h[kWaves][16][kWPad];
    float f[BF ? kWaves : 1][16][BF ? kSPad : 4];
  };
  __shared__ __attribute__((aligned(16))) WeightLds w_buf;
  auto& w_lds = w_buf.h;
  auto& w_lds_f = w_buf.f;
  __shared__ float a_lds[FC_MAX_BLOCK * SROWS];
  __shared__ float comb[kWaves][16][3];
  // the wavefronts' accumulators, for the combine (and the step's SROWS x D
  // coefficient scratch before the passes)
  constexpr int CB = GP * kWaves >= SROWS ? GP : (SROWS + kWaves - 1) / kWaves;
  __shared__ float cbuf[kWaves][CB][D];
  __shared__ __attribute__((aligned(16))) float part_lds[16 * D];
  __shared__ float tail_ml[2][16];
  __shared__ float wg_ml[2][16];
  __shared__ int s_last;
  __shared__ int s_final;

  // 1-D grid, split-major, as the int8 pass
  const int64_t L = blockIdx.x;
  const int split = (int)(L / p.ngroups);
  const int64_t g = ((L % p.ngroups) - split % p.ngroups + p.ngroups) % p.ngroups;
  const int64_t bh = g / p.zg;
  const int64_t g0 = (g % p.zg) * 16;
  const int64_t b = bh / p.Hkv, hkv = bh - b * p.Hkv;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, lc = lane & 15;
  const int G = (int)min<int64_t>(16, p.G - g0);
  const int r = p.r;

  for (int i = tid; i < r * SROWS; i += kMThreads) a_lds[i] = p.A[i];

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
    // counts of a decode step's view on the device (graph replays)
    const int64_t t = min<int64_t>(max<int64_t>(p.state[1], 0), p.r - 1) + 1;
    nb = min<int64_t>(max<int64_t>(p.state[0], 0) + (t == p.r ? 1 : 0), min(p.kcap, p.vcap));
    n_raw = t == p.r ? 0 : t;
  }
  const int64_t rows_total = nb * SROWS;
  const int64_t npass = (rows_total + PR - 1) / PR;
  unsigned int* passq = p.passq + g * p.cstride;
  const unsigned int wslot = (unsigned int)(split * kWaves + wave);
  const unsigned int wstride = (unsigned int)(p.n_splits * kWaves);
  const unsigned int nfix = (unsigned int)max<int64_t>(1, 3 * npass / (4 * (int64_t)wstride));
  const unsigned int qbase = wstride * nfix;
  unsigned int next_fixed = wslot + wstride;
  auto grab = [&]() -> unsigned int {  // result in lane 0, read when needed
    const unsigned int f = next_fixed;
    next_fixed += wstride;
    if (p.static_passes || f < qbase) return f;
    unsigned int v = 0;
    if (lane == 0)
      v = __hip_atomic_fetch_add(passq, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + qbase;
    return v;
  };
  auto pass_of = [](unsigned int v) { return (int64_t)__builtin_amdgcn_readfirstlane((int)v); };

  const T* kbase = static_cast<const T*>(p.kfp) + bh * p.kcap * SROWS * D;
  const T* vbase = static_cast<const T*>(p.vfp) + bh * p.vcap * SROWS * D;

  // ---- queries (B operand): lane (q, c) holds head c's features 32ch + 8q ..
  const bool hq_ok = lc < G;
  const int64_t hq = hkv * p.G + g0 + (hq_ok ? lc : 0);
  const T* qrow = static_cast<const T*>(p.q) + b * p.q_sb + hq * p.q_sh + 8 * lq;
  u32x4_t qop[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    qop[c] = *reinterpret_cast<const u32x4_t*>(qrow + 32 * c);
    if (!hq_ok) qop[c] = (u32x4_t){0u, 0u, 0u, 0u};
  }

  float4_t acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = (float4_t){0.f, 0.f, 0.f, 0.f};
  const int myh = lane % GP;
  float m_run = -INFINITY, l_lane = 0.f;

  // rows past the pass end read as zero (buffer descriptors sized to the pass)
  u32x4_t kr[NT][NC];
  auto load_k = [&](int64_t pr0, int prow) {
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(kbase + pr0 * D, prow * D * 2);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int c = 0; c < NC; ++c)
        kr[t][c] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                         rk, ((16 * t + lc) * D + 32 * c + 8 * lq) * 2, 0, kCachePolicyNt));
  };
  // lane (q, c): rows 32 sl + 8q + i, features 8c .. 8c+7 (columns past D
  // read the last 8 features again; their outputs are dropped)
  const int v_col = min(8 * lc, D - 8);
  u32x4_t vr[NS][8];
  auto load_v = [&](int64_t pr0, int prow) {
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vbase + pr0 * D, prow * D * 2);
#pragma unroll
    for (int sl = 0; sl < NS; ++sl)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        vr[sl][i] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                         rv, ((32 * sl + 8 * lq + i) * D + v_col) * 2, 0, kCachePolicyNt));
  };

  // weights of the pass's (block, head) pairs against mref into w_lds (f16,
  // or fp32 for bf16 rows); this lane's largest logit and exponential sum
  auto weights = [&](int prow, float mref, float& pmax, float& lsum) {
    pmax = -INFINITY;
    lsum = 0.f;
    if (myh >= G) return;
    const int npair = (prow / SROWS) * GP;
    for (int u = lane; u < npair; u += 64) {
      const int row0 = (u / GP) * SROWS;
      float sv[SROWS], w[SROWS];
#pragma unroll
      for (int j = 0; j < SROWS; ++j) {
        sv[j] = s_lds[wave][myh][row0 + j];
        w[j] = 0.f;
      }
      auto tap = [&](int t) {
        float lg = 0.f;
#pragma unroll
        for (int j = 0; j < SROWS; ++j) lg = __builtin_fmaf(a_lds[t * SROWS + j], sv[j], lg);
        pmax = fmaxf(pmax, lg);
        const float e = __builtin_amdgcn_exp2f(lg - mref);
        lsum += e;
#pragma unroll
        for (int j = 0; j < SROWS; ++j) w[j] = __builtin_fmaf(e, a_lds[t * SROWS + j], w[j]);
      };
      if (SROWS <= 4 && r <= kTapsUnrolled) {
#pragma unroll
        for (int t = 0; t < kTapsUnrolled; ++t)
          if (t < r) tap(t);
      } else {
        for (int t = 0; t < r; ++t) tap(t);
      }
#pragma unroll
      for (int j = 0; j < SROWS; ++j) {
        if constexpr (BF)
          w_lds_f[wave][myh][row0 + j] = w[j];
        else
          w_lds[wave][myh][row0 + j] = (_Float16)w[j];
      }
    }
  };

  auto rows_of = [&](int64_t pass) { return (int)min<int64_t>(PR, rows_total - pass * PR); };
  int64_t cur = wslot;
  if (!STEP && cur < npass) load_k(cur * PR, rows_of(cur));

  // raw tail (fused calls): split 0 computes its partial before the passes;
  // in a fused step that partial covers the rows the step adds
  const bool fold_tail = p.fused && split == 0 && (STEP || n_raw > 0);
  if constexpr (STEP) {
    if (split == 0) {
      __shared__ float step_sc[1];  // no quantizer: unused
      float* xk = &s_lds[0][0][0];  // the pass loop has not started: its scratch is free
      float* etl = reinterpret_cast<float*>(&w_buf);
      const int64_t kblk = (bh * p.kcap + step_nb) * SROWS, vblk = (bh * p.vcap + step_nb) * SROWS;
      T* kw = static_cast<T*>(const_cast<void*>(p.kfp)) + kblk * D;
      T* vw = static_cast<T*>(const_cast<void*>(p.vfp)) + vblk * D;
      step_partial<D, SROWS, T, 0>(
          step_t, p.r, static_cast<T*>(const_cast<void*>(p.kraw)) + bh * p.r * D,
          static_cast<T*>(const_cast<void*>(p.vraw)) + bh * p.r * D,
          static_cast<const T*>(p.ktok) + b * p.kt_sb + hkv * p.kt_sh,
          static_cast<const T*>(p.vtok) + b * p.vt_sb + hkv * p.vt_sh, step_write, kw, nullptr, vw,
          nullptr, p.basis, p.A, p.q, p.q_dtype, b * p.q_sb, p.q_sh, hkv * p.G + g0, G,
          p.scale_log2, tid, xk, xk + p.r * D, cbuf[0][0], step_sc, etl, part_lds, tail_ml[0],
          tail_ml[1]);
    }
  } else if (fold_tail) {
    raw_tail_partial<D>(p, b, hkv, g0, G, (int)n_raw, tid, &s_lds[0][0][0], part_lds, tail_ml[0],
                        tail_ml[1]);
  }
  __syncthreads();  // a_lds; the prologue's scratch is free again
  if (STEP && cur < npass) load_k(cur * PR, rows_of(cur));

  while (cur < npass) {
    const int64_t pr0 = cur * PR;
    const int prow = rows_of(cur);  // multiple of SROWS
    load_v(pr0, prow);
    const unsigned int nxt_v = grab();

    // ------------------------------------------------------------ scores
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if constexpr (BF)
          sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[t][c]),
                                                         __builtin_bit_cast(bf16x8_t, qop[c]),
                                                         sacc, 0, 0, 0);
        else
          sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, kr[t][c]),
                                                        __builtin_bit_cast(half8_t, qop[c]), sacc,
                                                        0, 0, 0);
      }
      if (lc < G)
        *reinterpret_cast<float4_t*>(&s_lds[wave][lc][16 * t + 4 * lq]) = sacc * p.scale_log2;
    }
    const int64_t nxt = pass_of(nxt_v);
    if (nxt < npass) load_k(nxt * PR, rows_of(nxt));  // flies during softmax and values
    wave_lds_sync();

    // ------------------------------------------------------------ softmax
    float pmax, lsum;
    weights(prow, m_run, pmax, lsum);
    if (__builtin_amdgcn_ballot_w64(pmax > m_run + kLazyMax) != 0) {
#pragma unroll
      for (int m = GP; m < 64; m <<= 1) pmax = fmaxf(pmax, __shfl_xor(pmax, m, 64));
      const float m_new = fmaxf(m_run, pmax);
      const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      float pdummy;
      weights(prow, m_new, pdummy, lsum);
      l_lane = l_lane * alpha + lsum;
      // lane (q, c) register i holds head 4q + i
      float al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * lq + i, 64);
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[e][i] *= al[i];
      m_run = m_new;
    } else {
      l_lane += lsum;
    }
    // rows past the pass end carry zero weight (they read as zero)
    if (prow < PRT)
      for (int i = prow + lane; i < PRT; i += 64)
        for (int h = 0; h < G; ++h) {
          if constexpr (BF)
            w_lds_f[wave][h][i] = 0.f;
          else
            w_lds[wave][h][i] = (_Float16)0.f;
        }
    wave_lds_sync();

    // ------------------------------------------------------------ values
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) {
      u32x4_t whi, wlo = {};
      if constexpr (BF) {
        // w = hi + lo, each a bf16 (RNE), rows 8q .. 8q+7 of head c
        float4_t f0 = *reinterpret_cast<const float4_t*>(&w_lds_f[wave][lc][32 * sl + 8 * lq]);
        float4_t f1 = *reinterpret_cast<const float4_t*>(&w_lds_f[wave][lc][32 * sl + 8 * lq + 4]);
        if (lc >= G) f0 = f1 = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float x0 = k < 2 ? f0[2 * k] : f1[2 * k - 4];
          const float x1 = k < 2 ? f0[2 * k + 1] : f1[2 * k - 3];
          const bf16_t h0 = from_f32<bf16_t>(x0), h1 = from_f32<bf16_t>(x1);
          const bf16_t l0 = from_f32<bf16_t>(x0 - to_f32(h0)), l1 = from_f32<bf16_t>(x1 - to_f32(h1));
          whi[k] = (uint32_t)h0.bits | ((uint32_t)h1.bits << 16);
          wlo[k] = (uint32_t)l0.bits | ((uint32_t)l1.bits << 16);
        }
      } else {
        whi = *reinterpret_cast<const u32x4_t*>(&w_lds[wave][lc][32 * sl + 8 * lq]);
        if (lc >= G) whi = (u32x4_t){0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // rows (2pp, 2pp+1): feature e's halves of the two rows in one dword
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        u32x4_t ov;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp)
          ov[pp] = __builtin_amdgcn_perm(vr[sl][2 * pp + 1][e / 2], vr[sl][2 * pp][e / 2], sel);
        if constexpr (BF) {
          acc[e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wlo),
                                                           __builtin_bit_cast(bf16x8_t, ov),
                                                           acc[e], 0, 0, 0);
          acc[e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, whi),
                                                           __builtin_bit_cast(bf16x8_t, ov),
                                                           acc[e], 0, 0, 0);
        } else {
          acc[e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, whi),
                                                          __builtin_bit_cast(half8_t, ov), acc[e],
                                                          0, 0, 0);
        }
      }
    }
    wave_lds_sync();
    cur = nxt;
  }

  // ---- combine the wavefronts (lane (q, c) register i of acc[e]: head
  // 4q + i, feature 8c + e)
#pragma unroll
  for (int m = GP; m < 64; m <<= 1) l_lane += __shfl_xor(l_lane, m, 64);
  if (lane < GP) {
    comb[wave][lane][0] = m_run;
    comb[wave][lane][1] = l_lane;
    comb[wave][lane][2] = 1.f;
  }
  constexpr int NI = GP < 4 ? GP : 4;
  if (lq < (GP >= 4 ? GP / 4 : 1) && lc < D / 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int i = 0; i < NI; ++i) cbuf[wave][4 * lq + i][8 * lc + e] = acc[e][i];
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
  split_epilogue<D, CB, false, !STEP>(p, g, b, hkv, g0, G, split, tid, fold_tail, comb, cbuf,
                                      part_lds, tail_ml, wg_ml, &s_lds[0][0][0], s_last, passq,
                                      step_done);
}

}  // namespace

// Query / stream dtypes, head sizes and stored rows per block of the pass.
bool fpj_mfma_shape_supported(int q_dtype, int stream_dtype, int64_t D, int s) {
  if (q_dtype == FC_F32)  // fp32 coefficient rows: the png pass's fp32 products (JPG)
    return stream_dtype == FC_F32 && (D == 64 || D == 128) &&
           (s == 1 || s == 2 || s == 4 || s == 8 || s == 16);
  return (q_dtype == FC_F16 || q_dtype == FC_BF16) && stream_dtype == q_dtype &&
         (D == 64 || D == 128) && (s == 1 || s == 2 || s == 3 || s == 4 || s == 8);
}

// Whether the pass takes this call: its shapes, 16-byte aligned query rows
// and stores (16-byte row loads).
bool split_fpj_mfma_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                              int s, int stream_dtype, const fc_stream_view* key,
                              const fc_stream_view* value) {
  const auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  return fpj_mfma_shape_supported(q_dtype, stream_dtype, D, s) && al16(q) && q_sb % 8 == 0 &&
         q_sh % 8 == 0 && al16(key->rows) && al16(value->rows);
}

int launch_split_fpj_mfma(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                          int64_t Hq, int64_t Hkv, int64_t D, int r, int s, int64_t nb,
                          const fc_stream_view* key, const fc_stream_view* value, const float* A,
                          float scale_log2, float* pm, float* pl, float* pacc, int n_splits,
                          unsigned int* counters, int64_t counter_words, int64_t stride,
                          const MfmaFuse* fuse, const int64_t* state, hipStream_t st) {
  MfmaArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.kfp = key->rows;
  a.vfp = value->rows;
  a.kcap = key->cap;
  a.vcap = value->cap;
  a.A = A;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.nb = nb;
  a.r = r;
  a.scale_log2 = scale_log2;
  a.n_splits = n_splits;
  a.pm = pm;
  a.pl = pl;
  a.pacc = pacc;
  a.state = state ? state : (fuse ? fuse->state : nullptr);
  a.raw_dtype = q_dtype;
  if (fuse) {
    if (n_splits > kFuseMaxSplits) return FC_ERR_ARG;
    a.fused = 1;
    a.kraw = key->raw;
    a.vraw = value->raw;
    a.raw_dtype = fuse->raw_dtype;
    a.kr_sb = key->raw_sb;
    a.kr_sh = key->raw_sh;
    a.kr_st = key->raw_st;
    a.vr_sb = value->raw_sb;
    a.vr_sh = value->raw_sh;
    a.vr_st = value->raw_st;
    a.n_raw = fuse->n_raw;
    a.out = fuse->out;
    a.o_sb = fuse->o_sb;
    a.o_sh = fuse->o_sh;
    if (fuse->step) {
      a.step = 1;
      a.ktok = fuse->ktok;
      a.vtok = fuse->vtok;
      a.kt_sb = fuse->kt_sb;
      a.kt_sh = fuse->kt_sh;
      a.vt_sb = fuse->vt_sb;
      a.vt_sh = fuse->vt_sh;
      a.basis = fuse->basis;
      a.step_t = fuse->step_t;
      a.step_nb = fuse->step_nb;
      a.done = fuse->done;
    }
  }
  const int64_t G = Hq / Hkv;
  const int gg = (int)std::min<int64_t>(G, 16);
  const int gp = gg <= 1 ? 1 : gg <= 2 ? 2 : gg <= 4 ? 4 : gg <= 8 ? 8 : 16;
  a.zg = (int)((G + 15) / 16);
  a.ngroups = B * Hkv * a.zg;
  if (!counters || 2 * a.ngroups * stride > counter_words) return FC_ERR_ARG;
  a.arrive = counters;
  a.passq = counters + counter_words / 2;
  a.static_passes = static_pass_order() ? 1 : 0;
  a.cstride = stride;
  const dim3 grid((unsigned)(a.ngroups * n_splits));
  if (q_dtype == FC_F32) {  // fp32 coefficient rows (fc_attn_png_kernel.h, JPG)
    if (a.step && r > 16) return FC_ERR_UNSUPPORTED;  // the step's rows in LDS: r <= 16
    const int rc = launch_fpj32_t(a, s, (int)D, gp, grid, st);
    if (rc != FC_OK) return rc;
    return check_launch();
  }
  const bool bf = q_dtype == FC_BF16;
  const bool step = a.step != 0;
  const int rc = mfma_with_int<1, 2, 3, 4, 8>(s, [&](auto sc) {
    constexpr int Sv = decltype(sc)::value;
    return mfma_with_int<64, 128>((int)D, [&](auto dc) {
      constexpr int Dv = decltype(dc)::value;
      return mfma_with_int<1, 2, 4, 8, 16>(gp, [&](auto gc) {
        constexpr int GPv = decltype(gc)::value;
        if (bf && step)
          attn_split_fpj_mfma<Sv, Dv, GPv, true, true><<<grid, kMThreads, 0, st>>>(a);
        else if (bf)
          attn_split_fpj_mfma<Sv, Dv, GPv, true, false><<<grid, kMThreads, 0, st>>>(a);
        else if (step)
          attn_split_fpj_mfma<Sv, Dv, GPv, false, true><<<grid, kMThreads, 0, st>>>(a);
        else
          attn_split_fpj_mfma<Sv, Dv, GPv, false, false><<<grid, kMThreads, 0, st>>>(a);
        return FC_OK;
      });
    });
  });
  if (rc != FC_OK) return rc;
  return check_launch();
}

}  // namespace fc
