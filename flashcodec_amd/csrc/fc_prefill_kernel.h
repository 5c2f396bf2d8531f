// Causal prefill attention over an int8 jpeg archive without the
// reconstructed view (gfx950 matrix cores): the kernel template, shared by
// the translation units that instantiate its variants (fc_prefill.hip: the
// entry point and the vector-ALU softmax; fc_prefill_m4/m8/m16.hip: the
// matrix-core softmax of 4 stored rows per block, by block size).
//
// A prefill attends Sq query tokens (positions P0 .. P0+Sq-1, the newest
// tokens of the cache) to every cached token at or before their own
// position.  Archived tokens are A S: r tokens per block synthesised by
// A (r x s) from the block's s stored rows (int8 codes x per-row fp32
// scale), so for a query q
//   logit[t] = scale * sum_j A[t][j] (q . S_j)        (t in the block)
//   out     += sum_j (sum_t p[t] A[t][j]) S_j
// and neither the (S, D) K nor V reconstruction is formed
// (flashcodec/attention.py:1-27 for the decode identity; the reference's
// prefill attends on the materialised view, flashcodec/attention.py:24-26,
// flashcodec/patch_attention.py:52-61).  Raw-tail tokens (fewer than r,
// after the archive) are attended at full precision at the end.
//
// Work split: a wavefront owns 16 queries — GQ query heads of one kv head x
// TQ consecutive tokens (GQ * TQ = 16) — and walks every archived block up
// to its newest query's position by itself, in passes of 64 stored rows
// (32 at D = 256), so no partials are merged.  A workgroup is 4 such
// wavefronts on consecutive token runs.  Per pass:
//   scores: v_mfma_i32_16x16x64_i8 on the K codes with each query split as
//      256 hi + lo int8 operands after scaling it by a power of two to at
//      most 14-bit integers (exact integer scores);
//   softmax (RC == 0): (block, query) pairs over the 64 lanes (query =
//      lane % 16), r logits from the s scores through A, causal mask per token,
//      exponentials against a running reference maximum that moves only
//      when a logit exceeds it by 2^8, output weights sum_t e_t A[t][j]
//      times the V row scale stored as f16;
//   values: v_mfma_f32_16x16x32_f16 with the V codes converted to f16
//      exactly in registers (8x8 byte tiles transposed with v_perm).
#pragma once
#include <hip/hip_runtime.h>

#include <type_traits>

#include "fc_attn_internal.h"
#include "fc_common.h"
#include "fc_mfma_pass.h"

namespace fc {

struct PrefillArgs {
  const void* q;  // (B, Hq, Sq, D) element strides q_sb, q_sh, q_st
  int q_dtype;
  int64_t q_sb, q_sh, q_st;
  int64_t Sq, P0;  // query tokens, position of the first
  const int8_t* kcodes;
  const float* kscales;
  const int8_t* vcodes;
  const float* vscales;
  int64_t kcap, vcap;
  const float* A;  // r x s
  int64_t Hkv, G, nb;
  int r;
  float scale_log2;
  const void* kraw;  // (B, Hkv, n_raw, D) tails in the stream dtype
  const void* vraw;
  int64_t kr_sb, kr_sh, kr_st, vr_sb, vr_sh, vr_st;
  int64_t n_raw;
  void* out;  // (B, Hq, Sq, D) in the query dtype
  int64_t o_sb, o_sh, o_st;
  int gq, tq;        // heads and tokens of a wavefront's 16 queries
  int64_t ntiles;    // token tiles of 4 * tq tokens
  int64_t hgroups;   // G / gq
};

constexpr int kPThreads = 256;
constexpr int kPWaves = kPThreads / 64;

// QG: per-32 scales (D / 32 per stored row), as the decode pass takes them:
// one score product per 32-feature group (the query's other group zeroed)
// scaled by the rows' group scales, V codes times their group scale
// relative to the row's largest as the value operand.
//
// RC != 0 (SROWS == 4, block size r == RC): the softmax runs on
// v_mfma_f32_4x4x1_16b_f32 and the pass stays in registers (the loop of
// that variant describes the lane layout); RC == 0: the softmax above on
// the vector ALU, scores and weights through LDS.
template <int SROWS, int DK, typename QT, typename RT, bool QG = false, int RC = 0>
__global__ __launch_bounds__(kPThreads, DK == 8 ? 1 : 2) void prefill_i8_mfma(PrefillArgs p) {
  static_assert(RC == 0 || (SROWS == 4 && RC % 4 == 0 && RC <= 16), "4x4 softmax: 4 rows");
  constexpr int D = 32 * DK;
  constexpr int DV = (D + 127) / 128;
  constexpr int PR = D == 256 ? 32 : 64;
  constexpr int NT = PR / 16;
  constexpr int NS = PR / 32;
  constexpr int KDW = 2 * DK;
  constexpr int NC = D / 64;
  constexpr int GP = 16;
  __shared__ float s_lds[kPWaves][16][kSPad];
  __shared__ _Float16 w_lds[kPWaves][16][kWPad];
  __shared__ float sc_lds[kPWaves][2][PR];
  constexpr int NGR = QG ? D / 32 : 1;
  __shared__ __attribute__((aligned(16))) float kg_lds[QG ? kPWaves : 1][NGR][PR];
  __shared__ __attribute__((aligned(16))) _Float16 vg_lds[QG ? kPWaves : 1][NGR][PR];
  __shared__ float a_lds[FC_MAX_BLOCK * 4];
  __shared__ float fin[kPWaves][2][16];  // per query: rescale factor and final sum

  // tile-major grid, longest tiles (the newest tokens) first
  const int64_t L = blockIdx.x;
  const int64_t cols = p.hgroups * p.Hkv;              // (kv head, head group) pairs per batch
  const int64_t ncol = cols * (gridDim.x / (p.ntiles * cols));  // B * cols
  const int64_t tile = p.ntiles - 1 - L / ncol;
  const int64_t rest = L % ncol;                       // b * cols + (hkv * hgroups + hg)
  const int64_t b = rest / cols;
  const int64_t hkv = (rest % cols) / p.hgroups, hg = rest % p.hgroups;
  const int64_t bh = b * p.Hkv + hkv;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane >> 4, lc = lane & 15;
  const int r = p.r;
  const int tq = p.tq;
  const int64_t tq0 = tile * 4 * tq + (int64_t)wave * tq;  // first token of this wavefront

  // A is read only when blocks are archived (an empty archive may come with
  // A == NULL)
  if (p.nb > 0)
    for (int i = tid; i < r * SROWS; i += kPThreads) a_lds[i] = p.A[i];

  // query c (c = lane % 16, or lc): head hq_of(c), token tok_of(c); padding
  // queries past Sq repeat the last token and are not stored
  auto head_of = [&](int c) { return hkv * p.G + hg * p.gq + c / tq; };
  auto tok_of = [&](int c) { return min<int64_t>(tq0 + c % tq, p.Sq - 1); };
  const int64_t last_tok = min<int64_t>(tq0 + tq - 1, p.Sq - 1);
  const int64_t qpos_max = p.P0 + last_tok;
  const int myq = lane % GP;
  const int64_t qpos_lane = p.P0 + tok_of(myq);
  const int64_t qpos_min = p.P0 + tq0;  // the wave's first query token

  // archived blocks this wavefront needs: up to its newest query's position
  const int64_t nbw = min<int64_t>(p.nb, qpos_max / r + 1);
  const int64_t rows_total = nbw * SROWS;
  const int64_t npass = (rows_total + PR - 1) / PR;

  const int8_t* kbase = p.kcodes + bh * p.kcap * SROWS * D;
  const int8_t* vbase = p.vcodes + bh * p.vcap * SROWS * D;
  const float* ksc = p.kscales + bh * p.kcap * SROWS * NGR;
  const float* vsc = p.vscales + bh * p.vcap * SROWS * NGR;

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

  float4_t acc[DV][8];
#pragma unroll
  for (int dv = 0; dv < DV; ++dv)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[dv][e] = (float4_t){0.f, 0.f, 0.f, 0.f};
  // !QG: the value operand is 1152 + code (f16 0x6400 | (code ^ 0x80)), so
  // acc holds sum w (1152 + code); accs = sum w per query (a product with
  // ones), taken off at the end.  Lane (q, c) register i: query 4q + i.
  constexpr float kVBias = 1152.f;
  float4_t accs = {0.f, 0.f, 0.f, 0.f};
  // query (lane % 16): reference max m_run (equal in its 4 lanes) and this
  // lane's share of the exponential sum; accumulators hold acc * 2^-sig_run
  float m_run = -INFINITY, l_lane = 0.f;
  int sig_run = -1000;
  float wmul_run = INFINITY;

  const int k_off = lc * D + 16 * lq;
  int v_off[DV];
#pragma unroll
  // V rows of the lane's k-slice lq of a 32-row slice: 8 lq .. 8 lq + 7, or
  // (RC != 0, the weights' register order) 4 lq .. + 3 and 16 + 4 lq .. + 3
  for (int dv = 0; dv < DV; ++dv) v_off[dv] = (RC ? 4 : 8) * lq * D + min(128 * dv + 8 * lc, D - 8);
  const int sc_off = (lane % PR) * 4;

  uint32_t kr[NT][KDW];
  float ks_r, vs_r;
  float kgr[NGR], vgr[NGR];  // QG: the group scales of row lane % PR
  const int sg_off = (lane % PR) * NGR * 4;
  // QG: a row's NGR group scales (8 or 16-byte pieces) into x
  auto load_groups = [&](const float* base, int64_t pr0, int prow, float (&x)[NGR]) {
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(base + pr0 * NGR, prow * NGR * 4);
    if constexpr (NGR == 2) {
      const u32x2_t v = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rs, sg_off, 0, 0));
      x[0] = __uint_as_float(v[0]);
      x[1] = __uint_as_float(v[1]);
    } else {
#pragma unroll
      for (int u = 0; u < NGR / 4; ++u) {
        const u32x4_t v = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, sg_off + 16 * u, 0, 0));
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * u + i] = __uint_as_float(v[i]);
      }
    }
  };
  auto load_k = [&](int64_t pr0, int prow) {
    if constexpr (QG) load_groups(ksc, pr0, prow, kgr);  // ahead of the codes
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(kbase + pr0 * D, prow * D);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < DK / 2; ++h) {
        const u32x4_t v = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, k_off + 16 * t * D + 64 * h, 0, 0));
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
    if constexpr (QG) load_groups(vsc, pr0, prow, vgr);  // ahead of the codes
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vbase + pr0 * D, prow * D);
#pragma unroll
    for (int sl = 0; sl < NS; ++sl)
#pragma unroll
      for (int dv = 0; dv < DV; ++dv)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const u32x2_t v = __builtin_bit_cast(
              u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
                           rv, v_off[dv] + (32 * sl + (RC && i >= 4 ? 12 + i : i)) * D, 0, 0));
          vr[sl][dv][2 * i] = v[0];
          vr[sl][dv][2 * i + 1] = v[1];
        }
  };

  // Output weights of the pass's (block, query) pairs (exponentials against
  // mref, times the V row scale * wm) into w_lds; causal: token t of block
  // `blk` takes part only when blk * r + t <= the query's position.
  // 1 / A[t][0] when column 0 of A is one nonzero constant (jpeg: the DC
  // row of the DCT basis, sqrt(1/r) at every tap), else 0; set once a_lds
  // is filled
  float dc_inv = 0.f;
  auto weights = [&](int64_t blk0, int prow, float mref, float wm, float& pmax, float& lsum) {
    lsum = 0.f;
    const int npair = (prow / SROWS) * GP;
    // Logits are formed relative to mref by the fma chain (finite stand-in
    // 0 in a lane whose mref is -inf: that lane's weights are formed again
    // against its new maximum).
    const float mo = mref == -INFINITY ? 0.f : mref;
    float pm = -INFINITY;
    // TAPS: compile-time tap count for the common block sizes (no branches
    // between taps), else a loop (0).  MASK: causal mask per (block, query) (the
    // diagonal passes; a pass whose last token is at or before the wave's
    // first query needs none).  MX: the wave's first pass (mref = -inf in
    // every lane) yields only the maximum, its weights follow against it.
    // DC (with TAPS): a constant column 0 of A (the DCT's DC row) gives the
    // pair's exponential sum as w[0] / A[t][0], one product for r additions.
    auto pairs = [&](auto rc, auto mask, auto mx) {
      constexpr int TAPS = decltype(rc)::value;
      constexpr bool MASK = decltype(mask)::value, MX = decltype(mx)::value;
      constexpr bool DC = TAPS != 0;
      for (int u = lane; u < npair; u += 64) {
        const int row0 = (u / GP) * SROWS;
        // causal taps of the pair (<= 0: the block starts after the query)
        int tlim = r;
        if constexpr (MASK) tlim = (int)min<int64_t>(r, qpos_lane - (blk0 + u / GP) * r + 1);
        float sv[SROWS], w[SROWS];
#pragma unroll
        for (int j = 0; j < SROWS; ++j) {
          sv[j] = s_lds[wave][myq][row0 + j] * sc_lds[wave][0][row0 + j];
          w[j] = 0.f;
        }
        auto tap = [&](int t, bool on) {
          float d = -mo;
#pragma unroll
          for (int j = 0; j < SROWS; ++j) d = __builtin_fmaf(a_lds[t * SROWS + j], sv[j], d);
          if constexpr (MASK) d = on ? d : -INFINITY;
          pm = fmaxf(pm, d);
          if constexpr (!MX) {
            const float e = __builtin_amdgcn_exp2f(d);
            if constexpr (!DC) lsum += e;
#pragma unroll
            for (int j = 0; j < SROWS; ++j) w[j] = __builtin_fmaf(e, a_lds[t * SROWS + j], w[j]);
          }
        };
        if constexpr (TAPS != 0) {
#pragma unroll
          for (int t = 0; t < TAPS; ++t) tap(t, t < tlim);
        } else {
          for (int t = 0; t < tlim; ++t) tap(t, true);
        }
        if constexpr (!MX) {
          if constexpr (DC) lsum = __builtin_fmaf(w[0], dc_inv, lsum);
#pragma unroll
          for (int j = 0; j < SROWS; ++j)
            w_lds[wave][myq][row0 + j] = (_Float16)(w[j] * (sc_lds[wave][1][row0 + j] * wm));
        }
      }
    };
    auto with_rc = [&](auto mask, auto mx) {
      if (dc_inv != 0.f && r == 8)
        pairs(std::integral_constant<int, 8>{}, mask, mx);
      else if (dc_inv != 0.f && r == 4)
        pairs(std::integral_constant<int, 4>{}, mask, mx);
      else if (dc_inv != 0.f && r == 16)
        pairs(std::integral_constant<int, 16>{}, mask, mx);
      else
        pairs(std::integral_constant<int, 0>{}, mask, mx);
    };
    const bool open = (blk0 + prow / SROWS) * r - 1 <= qpos_min;
    const bool first = __builtin_amdgcn_ballot_w64(mref != -INFINITY) == 0;
    using T_ = std::true_type;
    using F_ = std::false_type;
    if (first)
      open ? with_rc(F_{}, T_{}) : with_rc(T_{}, T_{});
    else
      open ? with_rc(F_{}, F_{}) : with_rc(T_{}, F_{});
    pmax = pm + mo;
  };

  // Value product of slice sl, column block dv: the lane's V codes (8 rows
  // x 8 features, as loaded) to f16 operands by 8x8 byte transposes with
  // v_perm: 1024 + (code + 128) (the weight sums take the 1152 off at the
  // end), QG: the code times its group ratio
  auto values_dv = [&](int sl, int dv, half8_t wop, half8_t rat) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
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
        half8_t ov;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const uint32_t src = ee < 2 ? t0[pp] : t1[pp];
          const uint32_t sel = (ee & 1) ? 0x04030402u : 0x04010400u;
          half2_t h2 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, src, sel));
          if constexpr (QG) h2 += (half2_t){(_Float16)-kVBias, (_Float16)-kVBias};
          ov[2 * pp] = h2[0];
          ov[2 * pp + 1] = h2[1];
        }
        const int e = 4 * hh + ee;
        if constexpr (QG) ov *= rat;
        acc[dv][e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop, ov, acc[dv][e], 0, 0, 0);
      }
    }
  };

  __syncthreads();  // a_lds (the only workgroup barrier)
  if (tq0 >= p.Sq) return;  // a wavefront past the last query token
  if (p.nb > 0) {
    const float a0 = a_lds[0];
    bool same = a0 != 0.f;
    for (int t = 1; t < r; ++t) same = same && a_lds[t * SROWS] == a0;
    dc_inv = same ? 1.0f / a0 : 0.f;
  }
  auto rows_of = [&](int64_t pass) { return (int)min<int64_t>(PR, rows_total - pass * PR); };
  if constexpr (RC == 0) {
    if (npass > 0) load_k(0, rows_of(0));
    for (int64_t cur = 0; cur < npass; ++cur) {
      const int64_t pr0 = cur * PR;
      const int prow = rows_of(cur);  // multiple of SROWS
      load_v(pr0, prow);

      // ------------------------------------------------------------ scores
      if constexpr (QG) {
        if (lane < PR) {
#pragma unroll
          for (int i = 0; i < NGR; ++i) kg_lds[wave][i][lane] = kgr[i];
        }
        wave_lds_sync();
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if constexpr (QG) {
          // lanes q < 2 hold group 2c of chunk c, q >= 2 group 2c + 1
          float4_t accg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const i32x4_t a = {(int)kr[t][4 * c], (int)kr[t][4 * c + 1], (int)kr[t][4 * c + 2],
                               (int)kr[t][4 * c + 3]};
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
              // the codes of the other group's lanes zeroed (the query stays
              // whole: a masked copy of it would be hoisted out of the loop)
              const bool mine = (lq >> 1) == hf;
              const i32x4_t zero = {0, 0, 0, 0};
              const i32x4_t am = mine ? a : zero;
              const i32x4_t ghi = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, qhi[c], zero, 0, 0, 0);
              const i32x4_t glo = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, qlo[c], zero, 0, 0, 0);
              const float4_t kgv =
                  *reinterpret_cast<const float4_t*>(&kg_lds[wave][2 * c + hf][16 * t + 4 * lq]);
#pragma unroll
              for (int i = 0; i < 4; ++i)
                accg[i] = __builtin_fmaf(kgv[i], (float)(ghi[i] * 256 + glo[i]), accg[i]);
            }
          }
          *reinterpret_cast<float4_t*>(&s_lds[wave][lc][16 * t + 4 * lq]) = accg * head_mul;
          continue;
        }
        i32x4_t shi = {0, 0, 0, 0}, slo = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const i32x4_t a = {(int)kr[t][4 * c], (int)kr[t][4 * c + 1], (int)kr[t][4 * c + 2],
                             (int)kr[t][4 * c + 3]};
          shi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qhi[c], shi, 0, 0, 0);
          slo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qlo[c], slo, 0, 0, 0);
        }
        float4_t sv;
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = (float)(shi[i] * 256 + slo[i]) * head_mul;
        *reinterpret_cast<float4_t*>(&s_lds[wave][lc][16 * t + 4 * lq]) = sv;
      }
      if constexpr (QG) {
        // V group scales relative to the row's largest (that one joins the
        // output weights as the row scale)
        float vmax = 0.f;
#pragma unroll
        for (int i = 0; i < NGR; ++i) vmax = fmaxf(vmax, vgr[i]);
        const float rv = vmax > 0.f ? __builtin_amdgcn_rcpf(vmax) : 0.f;
        if (lane < PR) {
#pragma unroll
          for (int i = 0; i < NGR; ++i) vg_lds[wave][i][lane] = (_Float16)(vgr[i] * rv);
        }
        ks_r = 1.f;
        vs_r = vmax;
      }
      if (lane < PR) {
        sc_lds[wave][0][lane] = ks_r;
        sc_lds[wave][1][lane] = vs_r;
      }
      const bool sig_need = vs_r * wmul_run >= 2.0f;
      const float vs_pass = vs_r;
      if (cur + 1 < npass) load_k(pr0 + PR, rows_of(cur + 1));
      wave_lds_sync();

      // ------------------------------------------------------------ softmax
      const int64_t blk0 = pr0 / SROWS;
      float pmax, lsum;
      weights(blk0, prow, m_run, wmul_run, pmax, lsum);
      const bool m_need = pmax > m_run + kLazyMax;
      if (__builtin_amdgcn_ballot_w64(sig_need || m_need) != 0) {
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
        weights(blk0, prow, m_new, wm, pdummy, lsum);
        l_lane = l_lane * alpha + lsum;
        // lane (q, c) register i holds query 4q + i
        const float sfix = ldexpf(1.0f, sig_run - sig_new);
        float al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * lq + i, 64) * sfix;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int dv = 0; dv < DV; ++dv)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[dv][e][i] *= al[i];
          accs[i] *= al[i];
        }
        m_run = m_new;
        sig_run = sig_new;
        wmul_run = wm;
      } else {
        l_lane += lsum;
      }
      if (prow < PR)
        for (int i = prow + lane; i < PR; i += 64)
          for (int h = 0; h < 16; ++h) w_lds[wave][h][i] = (_Float16)0.f;
      wave_lds_sync();

      // ------------------------------------------------------------ values
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
        const u32x4_t wa = *reinterpret_cast<const u32x4_t*>(&w_lds[wave][lc][32 * sl + 8 * lq]);
        const half8_t wop = __builtin_bit_cast(half8_t, wa);
        if constexpr (!QG) {
          const half8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
          accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop, ones, accs, 0, 0, 0);
        }
#pragma unroll
        for (int dv = 0; dv < DV; ++dv) {
          // QG: column c holds features 128 dv + 8 c + e, group 4 dv + c / 4
          // (clamped: columns past D are dropped), rows 8q .. 8q+7
          half8_t rat = {};
          if constexpr (QG)
            rat = *reinterpret_cast<const half8_t*>(
                &vg_lds[wave][min(4 * dv + lc / 4, NGR - 1)][32 * sl + 8 * lq]);
          values_dv(sl, dv, wop, rat);
        }
      }
      wave_lds_sync();
    }
  } else {
    // ---- RC != 0: the pass stays in registers.  Lane (lq, lc) holds query
    // lc and, of each 16-row tile t of the pass, rows 16 t + 4 lq .. + 3 =
    // block 4 t + lq: the score product's output layout, which is also an
    // operand layout of v_mfma_f32_4x4x1_16b_f32 (its 16 independent 4x4
    // products are the (lq, lc / 4) pairs, column lc % 4 the query).  Per
    // tile: logits = A (r x 4) times the 4 scores (r / 4 products of 4
    // k-steps, A operand A[4 th + i][k] for row i = lane % 4), causal mask
    // as 4 more k-steps, exponentials in place, weights = A^T times them (r
    // k-steps, A operand A[t][i]); the weights are the value product's A
    // operand as they stand, with the value rows taken in the same order
    // (k-slice q of a 32-row slice: rows 4q .. 4q+3 and 16+4q .. 16+4q+3).
    constexpr int NTH = RC ? RC / 4 : 1;
    const int ai = lane & 3;
    float a_log[NTH][4], a_w[RC ? RC : 1];
#pragma unroll
    for (int th = 0; th < NTH; ++th)
#pragma unroll
      for (int k = 0; k < 4; ++k) a_log[th][k] = a_lds[(4 * th + ai) * 4 + k];
#pragma unroll
    for (int t = 0; t < RC; ++t) a_w[t] = a_lds[4 * t + ai];
    const bool dc = __builtin_amdgcn_readfirstlane(__float_as_uint(dc_inv)) != 0;
    float nmo = 0.f;  // minus the finite stand-in of m_run (0 while it is -inf)
    // passes without the causal mask, a prefix of the wave's passes: whole
    // and their last token at or before the wave's first query
    const int n_open = (int)min<int64_t>(rows_total / PR, (qpos_min + 1) / ((PR / 4) * RC));
    if (npass > 0) load_k(0, rows_of(0));
    for (int64_t cur = 0; cur < npass; ++cur) {
      const int64_t pr0 = cur * PR;
      const int prow = rows_of(cur);  // multiple of SROWS
      load_v(pr0, prow);
      // K row scales (QG: the K group scales) of the pass's rows to LDS
      if (lane < PR) {
        if constexpr (QG) {
#pragma unroll
          for (int i = 0; i < NGR; ++i) kg_lds[wave][i][lane] = kgr[i];
        } else {
          sc_lds[wave][0][lane] = ks_r;
        }
      }
      wave_lds_sync();

      // ---------------------------------------------------------- scores
      // sv[t][i]: base-2 logit contribution of row 16 t + 4 lq + i for
      // query lc (the score times the head scale and the K row scale)
      float4_t sv[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if constexpr (QG) {
          float4_t accg = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const i32x4_t a = {(int)kr[t][4 * c], (int)kr[t][4 * c + 1], (int)kr[t][4 * c + 2],
                               (int)kr[t][4 * c + 3]};
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
              const bool mine = (lq >> 1) == hf;
              const i32x4_t zero = {0, 0, 0, 0};
              const i32x4_t am = mine ? a : zero;
              const i32x4_t ghi = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, qhi[c], zero, 0, 0, 0);
              const i32x4_t glo = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, qlo[c], zero, 0, 0, 0);
              const float4_t kgv =
                  *reinterpret_cast<const float4_t*>(&kg_lds[wave][2 * c + hf][16 * t + 4 * lq]);
#pragma unroll
              for (int i = 0; i < 4; ++i)
                accg[i] = __builtin_fmaf(kgv[i], (float)(ghi[i] * 256 + glo[i]), accg[i]);
            }
          }
          *reinterpret_cast<float4_t*>(&s_lds[wave][lc][16 * t + 4 * lq]) = accg * head_mul;
        } else {
          i32x4_t shi = {0, 0, 0, 0}, slo = {0, 0, 0, 0};
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const i32x4_t a = {(int)kr[t][4 * c], (int)kr[t][4 * c + 1], (int)kr[t][4 * c + 2],
                               (int)kr[t][4 * c + 3]};
            shi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qhi[c], shi, 0, 0, 0);
            slo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, qlo[c], slo, 0, 0, 0);
          }
          const float4_t kh =
              *reinterpret_cast<const float4_t*>(&sc_lds[wave][0][16 * t + 4 * lq]) * head_mul;
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[t][i] = (float)(shi[i] * 256 + slo[i]) * kh[i];
        }
      }
      if constexpr (QG) {
        // V group scales relative to the row's largest (that one joins the
        // weights as the row scale)
        float vmax = 0.f;
#pragma unroll
        for (int i = 0; i < NGR; ++i) vmax = fmaxf(vmax, vgr[i]);
        const float rv = vmax > 0.f ? __builtin_amdgcn_rcpf(vmax) : 0.f;
        if (lane < PR) {
#pragma unroll
          for (int i = 0; i < NGR; ++i) vg_lds[wave][i][lane] = (_Float16)(vgr[i] * rv);
        }
        vs_r = vmax;
      }
      if (lane < PR) sc_lds[wave][1][lane] = vs_r;
      const bool sig_need = vs_r * wmul_run >= 2.0f;
      const float vs_pass = vs_r;
      if (cur + 1 < npass) load_k(pr0 + PR, rows_of(cur + 1));
      wave_lds_sync();

      // ---------------------------------------------------------- softmax
      // a V row scale at or above 2^(sig_run + 1): accumulators and weights
      // to the new exponent first
      if (__builtin_amdgcn_ballot_w64(sig_need) != 0) {
        float smax = vs_pass;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) smax = fmaxf(smax, __shfl_xor(smax, m, 64));
        const int sig_new = max(sig_run, pow2_exp_for(smax, 1));
        const float sfix = ldexpf(1.0f, sig_run - sig_new);
#pragma unroll
        for (int dv = 0; dv < DV; ++dv)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[dv][e] *= sfix;
        accs *= sfix;
        sig_run = sig_new;
        wmul_run = ldexpf(1.0f, -sig_new);
      }
      // QG: the scores went through LDS (the lane's own slots; kept in
      // registers, the 32 group products of the score stage are all
      // scheduled ahead and spill)
      if constexpr (QG) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
          sv[t] = *reinterpret_cast<const float4_t*>(&s_lds[wave][lc][16 * t + 4 * lq]);
      }
      const int64_t blk0 = pr0 / SROWS;
      float4_t L[NT][NTH];
      const float4_t c0 = {nmo, nmo, nmo, nmo};
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int th = 0; th < NTH; ++th) {
          L[t][th] = c0;
#pragma unroll
          for (int k = 0; k < 4; ++k)
            L[t][th] = __builtin_amdgcn_mfma_f32_4x4x1f32(a_log[th][k], sv[t][k], L[t][th], 0, 0, 0);
        }
      if ((int)cur >= n_open) {
        // taps after the query's position (and every tap of blocks past the
        // pass's rows) get -2^100: A = -2^100 where k == i, B = [tap 4 th + k
        // of the lane's block is masked for its query]
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
              L[t][th] = __builtin_amdgcn_mfma_f32_4x4x1f32(
                  ai == k ? -0x1p100f : 0.f,
                  __builtin_amdgcn_fmed3f((float)(4 * th + k) - limf, 0.f, 1.f), L[t][th], 0, 0,
                  0);
        }
      }
      float pm = -INFINITY;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int th = 0; th < NTH; ++th)
#pragma unroll
          for (int i = 0; i < 4; ++i) pm = fmaxf(pm, L[t][th][i]);
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
          for (int th = 0; th < NTH; ++th) L[t][th] += dm;
        l_lane *= alpha;
        // accumulator lane (q, c) register i holds query 4q + i
        float al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * lq + i, 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int dv = 0; dv < DV; ++dv)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[dv][e][i] *= al[i];
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
          for (int i = 0; i < 4; ++i) L[t][th][i] = __builtin_amdgcn_exp2f(L[t][th][i]);
      // weights of the block's 4 rows for the lane's query (the tiles'
      // chains independent), then the exponential sums
      float4_t W[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        W[t] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < RC; ++u)
          W[t] = __builtin_amdgcn_mfma_f32_4x4x1f32(a_w[u], L[t][u / 4][u % 4], W[t], 0, 0, 0);
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
            for (int i = 0; i < 4; ++i) l_lane += L[t][th][i];
      }
      half8_t wop[NS];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float4_t vw =
            *reinterpret_cast<const float4_t*>(&sc_lds[wave][1][16 * t + 4 * lq]) * wmul_run;
#pragma unroll
        for (int i = 0; i < 4; ++i) wop[t / 2][4 * (t % 2) + i] = (_Float16)(W[t][i] * vw[i]);
      }

      // ---------------------------------------------------------- values
#pragma unroll
      for (int sl = 0; sl < NS; ++sl) {
        if constexpr (!QG) {
          const half8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
          accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop[sl], ones, accs, 0, 0, 0);
        }
#pragma unroll
        for (int dv = 0; dv < DV; ++dv) {
          // QG: group 4 dv + c / 4 of column c, the slice's rows in k order
          half8_t rat = {};
          if constexpr (QG) {
            const int grp = min(4 * dv + lc / 4, NGR - 1);
            const u32x2_t r0 =
                *reinterpret_cast<const u32x2_t*>(&vg_lds[wave][grp][32 * sl + 4 * lq]);
            const u32x2_t r1 =
                *reinterpret_cast<const u32x2_t*>(&vg_lds[wave][grp][32 * sl + 16 + 4 * lq]);
            rat = __builtin_bit_cast(half8_t, (u32x4_t){r0[0], r0[1], r1[0], r1[1]});
          }
          values_dv(sl, dv, wop[sl], rat);
        }
      }
    }
  }

  // ---- raw tail and output.  Sum of each query's exponentials over its 4
  // lanes; accumulators back to true scale.
#pragma unroll
  for (int m = GP; m < 64; m <<= 1) l_lane += __shfl_xor(l_lane, m, 64);
  const float sigmul = sig_run == -1000 ? 0.f : ldexpf(1.0f, sig_run);
  const int64_t tail0 = p.nb * r;  // position of the first raw-tail token
  const int nt = (int)max<int64_t>(0, min<int64_t>(p.n_raw, qpos_max - tail0 + 1));
  float* z = &s_lds[wave][0][0];  // [16][kSPad] tail logits, then exponentials
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
      z[c * kSPad + t] = vis ? a * p.scale_log2 : -INFINITY;
    }
    wave_lds_sync();
    if (lane < 16) {
      float mt = -INFINITY;
      for (int t = 0; t < nt; ++t) mt = fmaxf(mt, z[lane * kSPad + t]);
      const float m_new = fmaxf(m_run, mt);
      const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
      float l = l_lane * alpha;
      for (int t = 0; t < nt; ++t) {
        const float zt = z[lane * kSPad + t];
        const float e = zt == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(zt - m_new);
        z[lane * kSPad + t] = e;
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
  // lane (q, c) register i: query 4q + i, features 128 dv + 8 c + e
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = 4 * lq + i;
    const int64_t tok = tq0 + c % tq;
    const float alpha = fin[wave][0][c], inv = 1.0f / fin[wave][1][c];
#pragma unroll
    for (int dv = 0; dv < DV; ++dv) {
      const int d0 = 128 * dv + 8 * lc;
      if (d0 >= D) continue;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        o[e] = (QG ? acc[dv][e][i] : __builtin_fmaf(-kVBias, accs[i], acc[dv][e][i])) * sigmul *
               alpha;
      for (int t = 0; t < nt; ++t) {
        const float et = z[c * kSPad + t];
        const RT* vv =
            static_cast<const RT*>(p.vraw) + b * p.vr_sb + hkv * p.vr_sh + t * p.vr_st + d0;
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
}

template <int... Vs, typename F>
int prefill_with_int(int v, F&& f) {
  int rc = FC_ERR_UNSUPPORTED;
  bool hit = false;
  ((v == Vs ? (rc = f(std::integral_constant<int, Vs>{}), hit = true) : false), ...);
  return hit ? rc : FC_ERR_UNSUPPORTED;
}

// Launches prefill_i8_mfma<SR, DK, QT, RT, grouped, RC> for the runtime
// head size (D / 32), query and stream dtypes; instantiated per (SR, RC) in
// its own translation unit.
template <int SR, int RC>
int launch_prefill(const PrefillArgs& a, int dk, int q_dtype, int stream_dtype, bool grouped,
                   unsigned blocks, hipStream_t st) {
  return prefill_with_int<2, 4, 8>(dk, [&](auto dc) {
    constexpr int DKv = decltype(dc)::value;
    auto go = [&](auto qt, auto rt) {
      using QT = decltype(qt);
      using RT = decltype(rt);
      if (grouped)
        prefill_i8_mfma<SR, DKv, QT, RT, true, RC><<<dim3(blocks), kPThreads, 0, st>>>(a);
      else
        prefill_i8_mfma<SR, DKv, QT, RT, false, RC><<<dim3(blocks), kPThreads, 0, st>>>(a);
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

#define FC_PREFILL_EXTERN(SR, RC)                                                              \
  extern template int launch_prefill<SR, RC>(const PrefillArgs&, int, int, int, bool, unsigned, \
                                             hipStream_t);
FC_PREFILL_EXTERN(1, 0)
FC_PREFILL_EXTERN(2, 0)
FC_PREFILL_EXTERN(4, 0)
FC_PREFILL_EXTERN(4, 4)
FC_PREFILL_EXTERN(4, 8)
FC_PREFILL_EXTERN(4, 16)
#undef FC_PREFILL_EXTERN

}  // namespace fc
