// Causal prefill over an int8 jpeg archive with the passes shared by the
// workgroup (4 stored rows per block of RC = 4 or 8 tokens, one fp32 scale
// per row, D = 64 / 128): the C5 prefill's kernel.
//
// The 4 wavefronts of a workgroup own 16 queries each on consecutive token
// runs of one (batch, kv head, head group), so they walk the same archived
// rows (their pass counts differ by at most one).  Each pass of 64 stored
// rows is brought in once per workgroup: every thread loads its share of
// the next pass's K codes, V codes and row scales into registers while the
// current pass is computed, converts its V share to f16 value operands
// (1152 + code, transposed to (feature, row) with v_perm) and stores both
// into the other half of a double-buffered LDS tile; one barrier per pass.
// Each wavefront then runs the register-resident pass of prefill_i8_mfma's
// RC variant: int8 score products with K operands read from LDS, the
// softmax on v_mfma_f32_4x4x1_16b_f32 (logits, causal mask as k-steps,
// exponentials, weights), and f16 value products with the V operands read
// from LDS.  The LDS tiles are XOR-swizzled by 16-byte chunk so that the 16
// lanes of an operand read hit distinct banks.
#pragma once

#include "fc_prefill_kernel.h"

namespace fc {

template <int DK, typename QT, typename RT, int RC>
__global__ __launch_bounds__(kPThreads, 3) void prefill_i8_wg(PrefillArgs p) {
  constexpr int SROWS = 4;
  constexpr int D = 32 * DK;
  static_assert(D == 64 || D == 128, "workgroup prefill: D = 64 or 128");
  static_assert(RC == 4 || RC == 8, "block of 4 or 8 tokens");
  constexpr int PR = 64;            // stored rows per pass
  constexpr int NT = PR / 16;       // 16-row tiles of a pass
  constexpr int NS = PR / 32;       // 32-row slices of the value product
  constexpr int NC = D / 64;        // 64-feature chunks of the score product
  constexpr int NTH = RC / 4;
  constexpr int NE = D / 16;        // value products per slice (16 features each)
  constexpr int GP = 16;
  constexpr int KCH = D / 16;       // 16-byte chunks per K row
  constexpr int KSH = D == 128 ? 1 : 2;  // rows per LDS bank period = 2^KSH
  constexpr int KPT = D / 4;        // K bytes per thread per pass
  constexpr int KCPT = KPT / 16;    // of them 16-byte chunks
  constexpr int FPT = D / 32;       // V features per thread per pass (8 rows each)
  constexpr int KBUF = PR * D;      // bytes of a K tile
  constexpr int VBUF = D * PR;      // f16 elements of a V tile
  constexpr int OSTR = D + 4;       // floats per staged output row
  constexpr int OUTB = kPWaves * 16 * OSTR * 4;
  constexpr int ZB = kPWaves * 16 * 16 * 4;
  constexpr int TILES = 2 * KBUF + 2 * VBUF * 2;
  constexpr int MAIN = TILES > OUTB + ZB ? TILES : OUTB + ZB;
  __shared__ __attribute__((aligned(16))) uint8_t lds_main[MAIN];
  __shared__ __attribute__((aligned(16))) float sc_lds[2][2][PR];  // K and V row scales
  __shared__ __attribute__((aligned(16))) float a_lds[RC * SROWS];   // A, row-major (r x 4)
  __shared__ __attribute__((aligned(16))) float at_lds[SROWS * RC];  // A transposed (4 x r)
  __shared__ float fin[kPWaves][2][16];  // per query: rescale factor and final sum
  uint8_t* const ktile = lds_main;                                        // [2][PR][D]
  _Float16* const vtile = reinterpret_cast<_Float16*>(lds_main + 2 * KBUF);  // [2][D][PR]

  // tile-major grid, longest tiles (the newest tokens) first
  const int64_t L = blockIdx.x;
  const int64_t cols = p.hgroups * p.Hkv;
  const int64_t ncol = cols * (gridDim.x / (p.ntiles * cols));
  const int64_t tile = p.ntiles - 1 - L / ncol;
  const int64_t rest = L % ncol;
  const int64_t b = rest / cols;
  const int64_t hkv = (rest % cols) / p.hgroups, hg = rest % p.hgroups;
  const int64_t bh = b * p.Hkv + hkv;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, lc = lane & 15;
  const int tq = p.tq;
  const int64_t tq0 = tile * 4 * tq + (int64_t)wave * tq;  // first token of this wavefront
  // a wavefront past the last query token takes part in the loads and
  // barriers only
  const bool active = tq0 < p.Sq;

  if (p.nb > 0)
    for (int i = tid; i < RC * SROWS; i += kPThreads) {
      const float v = p.A[i];
      a_lds[i] = v;
      at_lds[(i % SROWS) * RC + i / SROWS] = v;
    }

  auto head_of = [&](int c) { return hkv * p.G + hg * p.gq + c / tq; };
  auto tok_of = [&](int c) { return min<int64_t>(tq0 + c % tq, p.Sq - 1); };
  const int64_t last_tok = min<int64_t>(tq0 + tq - 1, p.Sq - 1);
  const int64_t qpos_max = p.P0 + last_tok;
  const int64_t qpos_lane = p.P0 + tok_of(lane % GP);
  const int64_t qpos_min = p.P0 + tq0;
  // archived rows of this wavefront (up to its newest query) and of the
  // workgroup (up to its last wavefront's)
  const int64_t rows_w = active ? min<int64_t>(p.nb, qpos_max / RC + 1) * SROWS : 0;
  const int npass_w = (int)((rows_w + PR - 1) / PR);
  const int64_t wg_last = min<int64_t>(tile * 4 * tq + 4 * tq - 1, p.Sq - 1);
  const int64_t rows_wg = min<int64_t>(p.nb, (p.P0 + wg_last) / RC + 1) * SROWS;
  const int npass_wg = (int)((rows_wg + PR - 1) / PR);
  // passes without the causal mask, a prefix of the wavefront's passes
  const int n_open = (int)min<int64_t>(rows_w / PR, (qpos_min + 1) / ((PR / 4) * RC));

  const int8_t* kbase = p.kcodes + bh * p.kcap * SROWS * D;
  const int8_t* vbase = p.vcodes + bh * p.vcap * SROWS * D;
  const float* ksc = p.kscales + bh * p.kcap * SROWS;
  const float* vsc = p.vscales + bh * p.vcap * SROWS;

  // ---- queries: B operand of the score product.  Lane (q, c): query c,
  // features 64 k + 16 q + [0, 16) of chunk k
  const QT* qrow = static_cast<const QT*>(p.q) + b * p.q_sb + head_of(lc) * p.q_sh +
                   tok_of(lc) * p.q_st + 16 * lq;
  float qf[DK][8];
  float qmax = 0.f;
#pragma unroll
  for (int kc = 0; kc < DK; ++kc) {
    const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(qrow + 64 * (kc / 2) + 8 * (kc % 2));
    if constexpr (std::is_same_v<QT, f16_t>) {
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
    for (int i = 0; i < 8; ++i) qmax = fmaxf(qmax, fabsf(qf[kc][i]));
  }
  qmax = fmaxf(qmax, __shfl_xor(qmax, 16, 64));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
  const int qe = pow2_exp_for(qmax, 14);
  i32x4_t qhi[NC], qlo[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t hw = 0, lw = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 16 * c + 4 * w + j;
        const int qi = (int)rintf(ldexpf(qf[e / 8][e % 8], -qe));
        const int lo = (int)(int8_t)(qi & 0xff);
        const int hi = (qi - lo) >> 8;
        lw |= (uint32_t)(lo & 0xff) << (8 * j);
        hw |= (uint32_t)(hi & 0xff) << (8 * j);
      }
      qhi[c][w] = (int)hw;
      qlo[c][w] = (int)lw;
    }
  const float head_mul = ldexpf(p.scale_log2, qe);  // integer score -> base-2 logit / K scale

  // value accumulators: lane (q, c) register i holds query 4q + i, feature
  // 16 e + c; acc = sum w (1152 + code), accs = sum w
  constexpr float kVBias = 1152.f;
  float4_t acc[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) acc[e] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float4_t accs = {0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_lane = 0.f, nmo = 0.f;
  int sig_run = -1000;
  float wmul_run = INFINITY;

  // ---- the workgroup's loads of a pass.  K: row tid / 4, 16-byte chunks
  // KCPT (tid % 4) .. +KCPT-1.  V: the 8 rows of k-slice q = (tid / 32) % 4
  // of slice tid / 128 (rows 4q .. 4q+3 and 16+4q .. 16+4q+3 of the slice:
  // the weights' register order), features FPT (tid % 32) .. +FPT-1.  Row
  // scales: K by wavefront 0, V by wavefront 1.
  const int krow = tid >> 2;
  const int vsl = tid >> 7, vq = (tid >> 5) & 3, vm = tid & 31;
  u32x4_t kst[KCPT];
  uint32_t vst[8];
  float sst = 0.f;
  auto issue = [&](int pass) {
    const int64_t pr0 = (int64_t)pass * PR;
    const int prow = (int)min<int64_t>(PR, rows_wg - pr0);
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(kbase + pr0 * D, prow * D);
#pragma unroll
    for (int j = 0; j < KCPT; ++j)
      kst[j] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                       rk, krow * D + ((tid & 3) * KCPT + j) * 16, 0, 0));
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vbase + pr0 * D, prow * D);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = 32 * vsl + (j < 4 ? 4 * vq + j : 12 + 4 * vq + j);
      if constexpr (FPT == 4)
        vst[j] = __builtin_amdgcn_raw_buffer_load_b32(rv, row * D + 4 * vm, 0, 0);
      else
        vst[j] = __builtin_amdgcn_raw_buffer_load_b16(rv, row * D + 2 * vm, 0, 0);
    }
    // (wave-uniform descriptors: wave 0 the K scales, wave 1 the V scales)
    if (wave < 2)
      sst = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                          buf_rsrc((wave == 0 ? ksc : vsc) + pr0, prow * 4),
                                          lane * 4, 0, 0));
  };
  // K chunk L of row `row` sits at chunk L ^ ((row >> KSH) & (KCH - 1)); V
  // (feature f, 8-row chunk L) at chunk L ^ ((f >> 1) & 7)
  auto store = [&](int buf) {
    uint8_t* kb = ktile + buf * KBUF;
#pragma unroll
    for (int j = 0; j < KCPT; ++j) {
      const int lch = (tid & 3) * KCPT + j;
      const int pch = lch ^ ((krow >> KSH) & (KCH - 1));
      *reinterpret_cast<u32x4_t*>(kb + krow * D + pch * 16) = kst[j];
    }
    _Float16* vb = vtile + buf * VBUF;
    uint32_t x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = vst[j] ^ 0x80808080u;  // offset binary: code + 128
    const int lch = 4 * vsl + vq;
#pragma unroll
    for (int h = 0; h < (FPT + 1) / 2; ++h) {
      // bytes of features 2h, 2h+1 of rows (2k, 2k+1), interleaved
      uint32_t t[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        t[k] = __builtin_amdgcn_perm(x[2 * k + 1], x[2 * k], h ? 0x07030602u : 0x05010400u);
#pragma unroll
      for (int o = 0; o < 2; ++o) {
        const int f = FPT * vm + 2 * h + o;
        const uint32_t sel = o ? 0x04030402u : 0x04010400u;
        u32x4_t w;  // f16 1024 + (code + 128) of the feature's 8 rows
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = __builtin_amdgcn_perm(0x64646464u, t[k], sel);
        const int pch = lch ^ ((f >> 1) & 7);
        *reinterpret_cast<u32x4_t*>(vb + f * PR + pch * 8) = w;
      }
    }
    if (wave < 2) sc_lds[buf][wave][lane] = sst;
  };

  if (npass_wg > 0) {
    issue(0);
    store(0);
  }
  __syncthreads();  // a_lds and the first pass
  float dc_inv = 0.f;
  if (p.nb > 0) {
    const float a0 = a_lds[0];
    bool same = a0 != 0.f;
    for (int t = 1; t < RC; ++t) same = same && a_lds[t * SROWS] == a0;
    dc_inv = same ? 1.0f / a0 : 0.f;
  }
  const bool dc = __builtin_amdgcn_readfirstlane(__float_as_uint(dc_inv)) != 0;
  // A operands (row ai = lane % 4 of each 4x4 product) are read from LDS in
  // each pass rather than held in registers
  const int ai = lane & 3;

  for (int cur = 0; cur < npass_wg; ++cur) {
    const int buf = cur & 1;
    if (cur + 1 < npass_wg) issue(cur + 1);
    if (cur < npass_w) {
      const uint8_t* kb = ktile + buf * KBUF;
      const _Float16* vb = vtile + buf * VBUF;
      const int64_t pr0 = (int64_t)cur * PR;
      const int prow = (int)min<int64_t>(PR, rows_w - pr0);  // this wavefront's rows
      // ---------------------------------------------------------- scores
      // sv[t][i]: base-2 logit contribution of row 16 t + 4 lq + i for
      // query lc (score times head scale times K row scale)
      float4_t sv[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int row = 16 * t + lc;
        i32x4_t shi = {0, 0, 0, 0}, slo = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int pch = (4 * c + lq) ^ ((row >> KSH) & (KCH - 1));
          const i32x4_t a = __builtin_bit_cast(
              i32x4_t, *reinterpret_cast<const u32x4_t*>(kb + row * D + pch * 16));
          shi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qhi[c], shi, 0, 0, 0);
          slo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qlo[c], slo, 0, 0, 0);
        }
        const float4_t kh =
            *reinterpret_cast<const float4_t*>(&sc_lds[buf][0][16 * t + 4 * lq]) * head_mul;
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[t][i] = (float)(shi[i] * 256 + slo[i]) * kh[i];
      }
      // ---------------------------------------------------------- softmax
      // a V row scale at or above 2^(sig_run + 1): accumulators and weights
      // to the new exponent first
      const float vs_pass = sc_lds[buf][1][lane];
      if (__builtin_amdgcn_ballot_w64(vs_pass * wmul_run >= 2.0f) != 0) {
        float smax = vs_pass;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) smax = fmaxf(smax, __shfl_xor(smax, m, 64));
        const int sig_new = max(sig_run, pow2_exp_for(smax, 1));
        const float sfix = ldexpf(1.0f, sig_run - sig_new);
#pragma unroll
        for (int e = 0; e < NE; ++e) acc[e] *= sfix;
        accs *= sfix;
        sig_run = sig_new;
        wmul_run = ldexpf(1.0f, -sig_new);
      }
      const int64_t blk0 = pr0 / SROWS;
      float4_t a_log[NTH];  // A[4 th + ai][0..3]
#pragma unroll
      for (int th = 0; th < NTH; ++th)
        a_log[th] = *reinterpret_cast<const float4_t*>(&a_lds[(4 * th + ai) * 4]);
      float4_t Lg[NT][NTH];
      const float4_t c0 = {nmo, nmo, nmo, nmo};
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int th = 0; th < NTH; ++th) {
          Lg[t][th] = c0;
#pragma unroll
          for (int k = 0; k < 4; ++k)
            Lg[t][th] = __builtin_amdgcn_mfma_f32_4x4x1f32(a_log[th][k], sv[t][k], Lg[t][th], 0, 0, 0);
        }
      if (cur >= n_open) {
        // taps after the query's position (and every tap of blocks past the
        // wavefront's rows) get -2^100: A = -2^100 where k == i, B = [tap
        // 4 th + k of the lane's block is masked for its query]
        const int nblk = prow / 4;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int bl = 4 * t + lq;
          const int64_t rel = min<int64_t>(qpos_lane - (blk0 + bl) * RC, RC);
          const float limf = (float)(bl < nblk ? (int)rel : -1);
#pragma unroll
          for (int th = 0; th < NTH; ++th)
#pragma unroll
            for (int k = 0; k < 4; ++k)
              Lg[t][th] = __builtin_amdgcn_mfma_f32_4x4x1f32(
                  ai == k ? -0x1p100f : 0.f,
                  __builtin_amdgcn_fmed3f((float)(4 * th + k) - limf, 0.f, 1.f), Lg[t][th], 0,
                  0, 0);
        }
      }
      float pm = -INFINITY;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int th = 0; th < NTH; ++th)
#pragma unroll
          for (int i = 0; i < 4; ++i) pm = fmaxf(pm, Lg[t][th][i]);
      if (cur == 0 || __builtin_amdgcn_ballot_w64(pm > kLazyMax) != 0) {
        // query lc's maximum over the pass (its 4 lanes)
#pragma unroll
        for (int m = GP; m < 64; m <<= 1) pm = fmaxf(pm, __shfl_xor(pm, m, 64));
        const float m_new = fmaxf(m_run, pm - nmo);
        const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
        const float nmo_new = m_new == -INFINITY ? 0.f : -m_new;
        const float dm = nmo_new - nmo;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int th = 0; th < NTH; ++th) Lg[t][th] += dm;
        l_lane *= alpha;
        // accumulator lane (q, c) register i holds query 4q + i
        float al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * lq + i, 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int e = 0; e < NE; ++e) acc[e][i] *= al[i];
          accs[i] *= al[i];
        }
        m_run = m_new;
        nmo = nmo_new;
      }
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int th = 0; th < NTH; ++th)
#pragma unroll
          for (int i = 0; i < 4; ++i) Lg[t][th][i] = __builtin_amdgcn_exp2f(Lg[t][th][i]);
      float4_t a_w[NTH];  // A[4 j .. 4 j + 3][ai]
#pragma unroll
      for (int j = 0; j < NTH; ++j) a_w[j] = *reinterpret_cast<const float4_t*>(&at_lds[ai * RC + 4 * j]);
      float4_t W[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        W[t] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < RC; ++u)
          W[t] = __builtin_amdgcn_mfma_f32_4x4x1f32(a_w[u / 4][u % 4], Lg[t][u / 4][u % 4], W[t], 0,
                                                    0, 0);
      }
      if (dc) {
#pragma unroll
        for (int t = 0; t < NT; ++t) l_lane = __builtin_fmaf(W[t][0], dc_inv, l_lane);
      } else {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int th = 0; th < NTH; ++th)
#pragma unroll
            for (int i = 0; i < 4; ++i) l_lane += Lg[t][th][i];
      }
      half8_t wop[NS];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float4_t vw =
            *reinterpret_cast<const float4_t*>(&sc_lds[buf][1][16 * t + 4 * lq]) * wmul_run;
#pragma unroll
        for (int i = 0; i < 4; ++i) wop[t / 2][4 * (t % 2) + i] = (_Float16)(W[t][i] * vw[i]);
      }
      // ---------------------------------------------------------- values
      const half8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
        accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop[sl], ones, accs, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < NE; ++e) {
          const int f = 16 * e + lc;
          const int pch = (4 * sl + lq) ^ ((f >> 1) & 7);
          const half8_t ov = *reinterpret_cast<const half8_t*>(vb + f * PR + pch * 8);
          acc[e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop[sl], ov, acc[e], 0, 0, 0);
        }
      }
    }
    if (cur + 1 < npass_wg) store(buf ^ 1);
    __syncthreads();
  }
  if (!active) return;

  // ---- raw tail and output.  The accumulators (less the weight-sum bias)
  // go through LDS to the (query, 8 consecutive features) layout of the
  // output lanes; the tiles' space is free after the last barrier.
  float* ob = reinterpret_cast<float*>(lds_main) + wave * 16 * OSTR;
  float* z = reinterpret_cast<float*>(lds_main + OUTB) + wave * 16 * 16;  // tail logits
#pragma unroll
  for (int e = 0; e < NE; ++e)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ob[(4 * lq + i) * OSTR + 16 * e + lc] = __builtin_fmaf(-kVBias, accs[i], acc[e][i]);
#pragma unroll
  for (int m = GP; m < 64; m <<= 1) l_lane += __shfl_xor(l_lane, m, 64);
  const float sigmul = sig_run == -1000 ? 0.f : ldexpf(1.0f, sig_run);
  const int64_t tail0 = p.nb * RC;  // position of the first raw-tail token
  const int nt = (int)max<int64_t>(0, min<int64_t>(p.n_raw, qpos_max - tail0 + 1));
  if (nt > 0) {
    // logits of the 16 queries against the tail tokens at full precision
    for (int u = lane; u < 16 * nt; u += 64) {
      const int c = u % 16, t = u / 16;
      const QT* qv = static_cast<const QT*>(p.q) + b * p.q_sb + head_of(c) * p.q_sh +
                     tok_of(c) * p.q_st;
      const RT* kv = static_cast<const RT*>(p.kraw) + b * p.kr_sb + hkv * p.kr_sh + t * p.kr_st;
      float a = 0.f;
      for (int d = 0; d < D; ++d) a = __builtin_fmaf(to_f32(qv[d]), to_f32(kv[d]), a);
      const bool vis = tail0 + t <= p.P0 + tok_of(c);
      z[c * 16 + t] = vis ? a * p.scale_log2 : -INFINITY;
    }
    wave_lds_sync();
    if (lane < 16) {
      float mt = -INFINITY;
      for (int t = 0; t < nt; ++t) mt = fmaxf(mt, z[lane * 16 + t]);
      const float m_new = fmaxf(m_run, mt);
      const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
      float l = l_lane * alpha;
      for (int t = 0; t < nt; ++t) {
        const float zt = z[lane * 16 + t];
        const float e = zt == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(zt - m_new);
        z[lane * 16 + t] = e;
        l += e;
      }
      fin[wave][0][lane] = alpha;
      fin[wave][1][lane] = l;
    }
  } else if (lane < 16) {
    fin[wave][0][lane] = 1.f;
    fin[wave][1][lane] = l_lane;
  }
  wave_lds_sync();
  // lane (q, c) register i: query 4q + i, features 8 c + e
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = 4 * lq + i;
    const int64_t tok = tq0 + c % tq;
    const int d0 = 8 * lc;
    if (d0 >= D) continue;
    const float alpha = fin[wave][0][c], inv = 1.0f / fin[wave][1][c];
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = ob[c * OSTR + d0 + e] * sigmul * alpha;
    for (int t = 0; t < nt; ++t) {
      const float et = z[c * 16 + t];
      const RT* vv = static_cast<const RT*>(p.vraw) + b * p.vr_sb + hkv * p.vr_sh + t * p.vr_st + d0;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(et, to_f32(vv[e]), o[e]);
    }
    if (tok < p.Sq) {
      QT* dst = static_cast<QT*>(p.out) + b * p.o_sb + head_of(c) * p.o_sh + tok * p.o_st + d0;
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[e] = from_f32<QT>(o[e] * inv);
    }
  }
}

// Launches prefill_i8_wg<DK, QT, RT, RC> for the runtime head size (D / 32),
// query and stream dtypes; instantiated per RC in fc_prefill_wg.hip.
template <int RC>
int launch_prefill_wg(const PrefillArgs& a, int dk, int q_dtype, int stream_dtype,
                      unsigned blocks, hipStream_t st) {
  return prefill_with_int<2, 4>(dk, [&](auto dc) {
    constexpr int DKv = decltype(dc)::value;
    auto go = [&](auto qt, auto rt) {
      using QT = decltype(qt);
      using RT = decltype(rt);
      prefill_i8_wg<DKv, QT, RT, RC><<<dim3(blocks), kPThreads, 0, st>>>(a);
      return FC_OK;
    };
    auto with_rt = [&](auto qt) {
      switch (stream_dtype) {
        case FC_F16: return go(qt, f16_t{});
        case FC_BF16: return go(qt, bf16_t{});
        default: return go(qt, float{});
      }
    };
    return q_dtype == FC_F16 ? with_rt(f16_t{}) : with_rt(bf16_t{});
  });
}

extern template int launch_prefill_wg<4>(const PrefillArgs&, int, int, int, unsigned, hipStream_t);
extern template int launch_prefill_wg<8>(const PrefillArgs&, int, int, int, unsigned, hipStream_t);

}  // namespace fc
