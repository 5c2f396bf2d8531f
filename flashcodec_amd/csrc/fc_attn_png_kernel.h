// Split pass of the decode attention for png archives on gfx950 matrix
// cores, with the merge of the split partials fused in: the pass queue,
// combine and merge of the int8 pass (fc_attn_mfma_kernel.h) over fp32 rows.
//
// A png block of r tokens is stored as its anchor (the first token, in the
// stream dtype) and r - 1 fp32 first-order deltas, token t = sum_{j <= t}
// row_j (flashcodec/codecs/png.py:36-74), so for a query q
// (flashcodec/attention.py:45-61: A is lower-triangular ones for png)
//   logit_t = scale * sum_{j <= t} (q . row_j)     prefix sums of the scores
//   out    += sum_j (sum_{t >= j} p_t) row_j        suffix sums of the weights
// and the token rows are never formed.
//
// Scores: v_mfma_f32_16x16x4_f32, 16 rows x 4 features by 4 features x 16
// heads per instruction.  Lane (q, m) holds features 16 j + 4 q + i (j < D/16,
// i < 4) of row m and lane (q, c) the same features of head c's query;
// instruction 4 j + i takes feature 16 j + 4 q + i from every lane, so the
// D/4 instructions cover all features, and each 16-byte load instruction
// reads 64 contiguous bytes of every row.  Output: lane (q, c) gets the
// scores of rows 4q .. 4q+3 for head c.
// Values: the same instruction with the weights (16 heads x 4 rows) by the
// rows (4 rows x 16 features): lane (q, c) holds rows q, q+4, q+8, q+12 of the
// pass, features 64 k + 4 c + i (k < D/64, i < 4; instruction f = 4 k + i of a
// row group takes feature 64 k + 4 c + i in column c), so a load instruction
// reads 256 contiguous bytes of a row.  (With D/4 consecutive features per
// lane, a load instruction touched 16-byte pieces 128 bytes apart in every
// row: C4 59.7 us per call over rotating sets, 52.5 us with this mapping.)
// A pass is one 16-row tile (16 / r whole blocks); a wavefront requests the
// next pass's rows after its score products and the pass's value rows at its
// start, and takes passes from its group's queue as the int8 pass does.
// Products and sums are fp32 throughout (the query and the weights are not
// rounded), so fp32 outputs meet the 1e-5 tolerance.  fp16 / bf16 streams
// (16-bit anchors, tails and queries; deltas are fp32 in every png archive)
// take the same kernel: their 16-bit elements are widened as they are loaded.
//
// The kernel template lives in this header; fc_attn_png.hip (host side,
// fp32) and fc_attn_png_f16.hip / fc_attn_png_bf16.hip instantiate
// launch_png_t for their stream dtype, so the three build in parallel.
#pragma once

#include "fc_attn_mfma_kernel.h"
#include "fc_png_step.h"

namespace fc {

namespace pngk {

// four 16-bit elements (two dwords, element 0 in the low half) as fp32
template <typename T>
__device__ __forceinline__ float4_t half4_to_f32(u32x2_t w) {
  float4_t o;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    o[2 * i] = to_f32(__builtin_bit_cast(T, (uint16_t)(w[i] & 0xffffu)));
    o[2 * i + 1] = to_f32(__builtin_bit_cast(T, (uint16_t)(w[i] >> 16)));
  }
  return o;
}

constexpr int kPngTile = 16;  // rows per pass

// kPngWgPerCu (2) workgroups per compute unit: measured at C4, 2 per CU
// (32 splits) take 59.2 us per call over rotating archive sets where 3 per
// CU (48 splits, the query operands read from LDS to fit 168 VGPRs) take
// 64.6 (more partials to merge, more contention on the pass queues).
// STEP: the fused decode step (fc_decode_step; MfmaArgs.step): split 0
// appends the token or archives the block it completes (png_step_rows)
// and the passes cover the blocks before it.  T: the stream dtype (anchors,
// tails, tokens) and the queries' (float, f16_t, bf16_t); deltas are fp32
// and products fp32 for all.
// JPG: the same pass over jpeg archives of fp32 coefficients (the reference's
// default codec, quant_bits=0, in an fp32 model): R stored coefficient rows
// per block (MfmaArgs.kfp / vfp), the p.r token logits of a (block, query)
// pair taps of A over its R scaled scores and the row weights
// w_j = sum_t p_t A[t][j] (flashcodec/attention.py:101-140), both in fp64 as
// the int8 pass forms them for fp32 queries.
template <int R, int D, int GP, bool STEP, typename T, bool JPG = false>
__global__ __launch_bounds__(kMThreads, kPngWgPerCu) void attn_split_png_mfma(MfmaArgs p) {
  constexpr bool F32 = std::is_same_v<T, float>;
  static_assert(!JPG || F32, "coefficient archives here: fp32");
  // JPG STEP: blocks of at most kJpgStepMaxR tokens (the host checks)
  constexpr int kJpgStepMaxR = 16;
  constexpr int FPL = D / 4;   // score-operand features per lane
  constexpr int FPC = D / 16;  // value-product features per lane column
  static_assert(kPngTile % R == 0 && FPC % 4 == 0, "block size / head size");
  __shared__ float s_lds[kWaves][16][kPngTile + 1];  // scaled scores [head][row]
  __shared__ float w_lds[kWaves][16][kPngTile + 4];  // weights [head][row]
  __shared__ float comb[kWaves][16][3];
  // the end phase's per-wavefront accumulators; STEP: before the passes,
  // the step's rows (2 R D floats)
  constexpr int kCb = kWaves * GP * D;
  // (JPG: the block's 2 r rows and its R coefficient rows)
  constexpr int kStepN = JPG ? (2 * kJpgStepMaxR + R) * D : 2 * R * D;
  constexpr int kCbN = STEP && kStepN > kCb ? kStepN : kCb;
  __shared__ __attribute__((aligned(16))) float cbuf_raw[kCbN];
  auto& cbuf = *reinterpret_cast<float (*)[kWaves][GP][D]>(cbuf_raw);
  __shared__ __attribute__((aligned(16))) float part_lds[16 * D];
  __shared__ float tail_ml[2][16];
  __shared__ float wg_ml[2][16];
  __shared__ float scratch[2 * 16 * kFuseMaxSplits];  // raw-tail logits, then merge statistics
  __shared__ int s_last;
  __shared__ int s_final;
  __shared__ float a_lds[JPG ? FC_MAX_BLOCK * R : 1];  // JPG: A (p.r x R)

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
  const int rblk = JPG ? p.r : R;  // tokens per block
  if constexpr (JPG)
    for (int i = tid; i < p.r * R; i += kMThreads) a_lds[i] = p.A[i];

  int64_t nb = p.nb, n_raw = p.n_raw;
  int64_t step_t = 0, step_nb = 0;  // fused step: tail length and blocks before the token
  bool step_write = false;
  if constexpr (STEP) {
    const int64_t cap = min(p.kcap, p.vcap);
    step_t = p.state ? min<int64_t>(max<int64_t>(p.state[1], 0), rblk - 1) : p.step_t;
    step_nb = p.state ? max<int64_t>(p.state[0], 0) : p.step_nb;
    // one head group per (batch, kv head) stores the token / block; a block
    // past the capacity is not stored (the state's overflow word says so)
    step_write = split == 0 && g0 == 0 && (step_t + 1 < rblk || step_nb < cap);
    nb = min(step_nb, cap);
    n_raw = 0;
  } else if (p.state) {
    // counts of a decode step's view on the device (graph replays)
    const int64_t t = min<int64_t>(max<int64_t>(p.state[1], 0), rblk - 1) + 1;
    nb = min<int64_t>(max<int64_t>(p.state[0], 0) + (t == rblk ? 1 : 0), min(p.kcap, p.vcap));
    n_raw = t == rblk ? 0 : t;
  }
  const int64_t rows_total = nb * R;
  const int64_t npass = (rows_total + kPngTile - 1) / kPngTile;
  unsigned int* passq = p.passq + g * p.cstride;
  const unsigned int wslot = (unsigned int)(split * kWaves + wave);
  const unsigned int wstride = (unsigned int)(p.n_splits * kWaves);
  // fixed order for three quarters of the passes, the rest from the queue,
  // as the int8 pass (C4: 0.5 us shorter than a queue for every pass)
  const unsigned int nfix = (unsigned int)max<int64_t>(1, 3 * npass / (4 * (int64_t)wstride));
  const unsigned int qbase = wstride * nfix;
  unsigned int next_fixed = wslot + wstride;
  auto grab = [&]() -> unsigned int {
    const unsigned int f = next_fixed;
    next_fixed += wstride;
    if (p.static_passes || f < qbase) return f;
    unsigned int v = 0;
    if (lane == 0)
      v = __hip_atomic_fetch_add(passq, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + qbase;
    return v;
  };
  auto pass_of = [](unsigned int v) { return (int64_t)__builtin_amdgcn_readfirstlane((int)v); };

  const T* kanch = JPG ? nullptr : static_cast<const T*>(p.kanch) + bh * p.kcap * D;
  const T* vanch = JPG ? nullptr : static_cast<const T*>(p.vanch) + bh * p.vcap * D;
  const float* kdel = JPG ? nullptr : p.kdel + bh * p.kcap * (R - 1) * D;
  const float* vdel = JPG ? nullptr : p.vdel + bh * p.vcap * (R - 1) * D;
  // JPG: coefficient row gr of the (batch, kv head) at + gr * D
  const float* kcoef = JPG ? static_cast<const float*>(p.kfp) + bh * p.kcap * R * D : nullptr;
  const float* vcoef = JPG ? static_cast<const float*>(p.vfp) + bh * p.vcap * R * D : nullptr;
  // row gr of a stream: the anchor of its block or one of its deltas; rows
  // past the archive read row 0 and are zeroed by the caller (fp32 anchors)
  auto row_ptr = [&](const float* anch, const float* del, int64_t gr) {
    const int64_t blk = gr / R;
    const int j = (int)(gr - blk * R);
    return j == 0 ? anch + blk * D : del + (blk * (R - 1) + (j - 1)) * D;
  };
  // 16-bit anchors: a lane's row is its block's anchor (2-byte elements) or
  // a delta (fp32).  Every lane loads a 16-byte piece of a delta row (an
  // anchor lane: its block's first delta row, which a neighbour lane loads
  // too) and an 8-byte piece of its block's anchor row (the lanes of a
  // block share those lines), then keeps the one its row is: no branch
  // holds a load, and the delta rows keep full-width loads
  struct RowRef {
    const float* del;
    const T* anch;
    bool anc;
  };
  auto row_ref = [&](const T* anch, const float* del, int64_t gr) {
    const int64_t blk = gr / R;
    const int j = (int)(gr - blk * R);
    const bool anc = j == 0;
    return RowRef{del + (blk * (R - 1) + (anc ? 0 : j - 1)) * D, anch + blk * D, anc};
  };
  // features e .. e+3 of row rr; NT: nontemporal
  auto row4_16 = [&](const RowRef& rr, int e, auto nt) -> float4_t {
    constexpr bool NT = decltype(nt)::value;
    const float4_t* dp = reinterpret_cast<const float4_t*>(rr.del + e);
    const u32x2_t* ap = reinterpret_cast<const u32x2_t*>(rr.anch + e);
    float4_t dv;
    u32x2_t av;
    if constexpr (NT) {
      dv = __builtin_nontemporal_load(dp);
      av = __builtin_nontemporal_load(ap);
    } else {
      dv = *dp;
      av = *ap;
    }
    const float4_t wide = half4_to_f32<T>(av);
    return rr.anc ? wide : dv;
  };
  // features e .. e+7 of row rr as two float4: two 16-byte delta pieces and
  // one 16-byte anchor piece (the score operand's 16-bit layout, which
  // gives each lane runs of 8 features so one anchor load serves both)
  auto row8_16 = [&](const RowRef& rr, int e, auto& lo, auto& hi) {
    const float4_t* dp = reinterpret_cast<const float4_t*>(rr.del + e);
    const float4_t d0 = dp[0], d1 = dp[1];
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(rr.anch + e);
    const float4_t w0 = half4_to_f32<T>((u32x2_t){a[0], a[1]});
    const float4_t w1 = half4_to_f32<T>((u32x2_t){a[2], a[3]});
    lo = rr.anc ? w0 : d0;
    hi = rr.anc ? w1 : d1;
  };
  // score-operand feature of lane quarter lq's piece j (4 features): fp32
  // rows 16 j + 4 lq; 16-bit rows 32 (j / 2) + 8 lq + 4 (j % 2), runs of 8
  // per lane (the product sums over features, so K and Q only have to agree)
  auto sfeat = [&](int j) { return F32 ? 16 * j + 4 * lq : 32 * (j >> 1) + 8 * lq + 4 * (j & 1); };
  // value-product feature of lane column lc's register f (runs of 8 per
  // lane here, as the score operand's, measured 1 us slower at C4's shape)
  auto vfeat = [&](int f) { return 64 * (f / 4) + 4 * lc + (f % 4); };

  // ---- queries: lane (q, c) holds head c's features sfeat(j) + i (q = lq)
  const bool hq_ok = lc < G;
  const int64_t hq = hkv * p.G + g0 + (hq_ok ? lc : 0);
  const T* qrow = static_cast<const T*>(p.q) + b * p.q_sb + hq * p.q_sh;
  using qraw_t = std::conditional_t<F32, float4_t, u32x2_t>;  // converted when read
  qraw_t qraw[FPL / 4];
#pragma unroll
  for (int j = 0; j < FPL / 4; ++j) qraw[j] = *reinterpret_cast<const qraw_t*>(qrow + sfeat(j));

  float4_t acc[FPC];
#pragma unroll
  for (int f = 0; f < FPC; ++f) acc[f] = (float4_t){0.f, 0.f, 0.f, 0.f};
  const int myh = lane % GP;  // the head of this lane's softmax pairs
  float m_run = -INFINITY, l_lane = 0.f;

  float kr[FPL];
  float qv[FPL];
  auto load_k = [&](int64_t pass) {
    const int64_t gr = pass * kPngTile + lc;
    const bool ok = gr < rows_total;
    const float* src = nullptr;
    RowRef rr{};
    if constexpr (JPG)
      src = kcoef + (ok ? gr : 0) * D;
    else if constexpr (F32)
      src = row_ptr(kanch, kdel, ok ? gr : 0);
    else
      rr = row_ref(kanch, kdel, ok ? gr : 0);
    if constexpr (F32) {
#pragma unroll
      for (int j = 0; j < FPL / 4; ++j) {
        const float4_t v = *reinterpret_cast<const float4_t*>(src + sfeat(j));
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[4 * j + i] = ok ? v[i] : 0.f;
      }
    } else {
#pragma unroll
      for (int j = 0; j < FPL / 4; j += 2) {
        float4_t lo, hi;
        row8_16(rr, sfeat(j), lo, hi);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kr[4 * j + i] = ok ? lo[i] : 0.f;
          kr[4 * j + 4 + i] = ok ? hi[i] : 0.f;
        }
      }
    }
  };
  float vr[4][FPC];
  auto load_v = [&](int64_t pass) {
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int64_t gr = pass * kPngTile + 4 * rg + lq;
      const bool ok = gr < rows_total;
      const float* src = nullptr;
      RowRef rr{};
      if constexpr (JPG)
        src = vcoef + (ok ? gr : 0) * D;
      else if constexpr (F32)
        src = row_ptr(vanch, vdel, ok ? gr : 0);
      else
        rr = row_ref(vanch, vdel, ok ? gr : 0);
#pragma unroll
      for (int k = 0; k < FPC / 4; ++k) {
        float4_t v;
        if constexpr (F32)
          v = __builtin_nontemporal_load(reinterpret_cast<const float4_t*>(src + vfeat(4 * k)));
        else
          v = row4_16(rr, vfeat(4 * k), std::true_type{});
#pragma unroll
        for (int i = 0; i < 4; ++i) vr[rg][4 * k + i] = ok ? v[i] : 0.f;
      }
    }
  };

  // weights of the pass's (block, head) pairs: prefix sums of the scaled
  // scores are the logits, exponentials against mref, suffix sums are the
  // row weights (into w_lds); this lane's largest logit and exponential sum
  auto weights = [&](int prow, float mref, float& pmax, float& lsum) {
    pmax = -INFINITY;
    lsum = 0.f;
    if (myh >= G) return;
    const int npair = (prow / R) * GP;
    if constexpr (JPG) {
      // the block's p.r logits as taps of A over its R scaled scores
      const int r = p.r;
      for (int u = lane; u < npair; u += 64) {
        const int row0 = (u / GP) * R;
        double sv[R];
        float w[R];
#pragma unroll
        for (int j = 0; j < R; ++j) {
          sv[j] = (double)s_lds[wave][myh][row0 + j];
          w[j] = 0.f;
        }
        for (int t = 0; t < r; ++t) {
          double lg = 0.0;
#pragma unroll
          for (int j = 0; j < R; ++j) lg = __builtin_fma((double)a_lds[t * R + j], sv[j], lg);
          pmax = fmaxf(pmax, (float)lg);
          const float e = __builtin_amdgcn_exp2f((float)(lg - (double)mref));
          lsum += e;
#pragma unroll
          for (int j = 0; j < R; ++j) w[j] = __builtin_fmaf(e, a_lds[t * R + j], w[j]);
        }
#pragma unroll
        for (int j = 0; j < R; ++j) w_lds[wave][myh][row0 + j] = w[j];
      }
      return;
    }
    for (int u = lane; u < npair; u += 64) {
      const int row0 = (u / GP) * R;
      float e[R];
      float run = 0.f;
#pragma unroll
      for (int t = 0; t < R; ++t) {
        run += s_lds[wave][myh][row0 + t];
        pmax = fmaxf(pmax, run);
        e[t] = __builtin_amdgcn_exp2f(run - mref);
        lsum += e[t];
      }
      float suf = 0.f;
#pragma unroll
      for (int t = R - 1; t >= 0; --t) {
        suf += e[t];
        w_lds[wave][myh][row0 + t] = suf;
      }
    }
  };

  // the first pass's rows go out right behind the query, before the query
  // is read
  int64_t cur = wslot;
  if (cur < npass) load_k(cur);
#pragma unroll
  for (int j = 0; j < FPL / 4; ++j) {
    float4_t qf;
    if constexpr (F32)
      qf = qraw[j];
    else
      qf = half4_to_f32<T>(qraw[j]);
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[4 * j + i] = hq_ok ? qf[i] : 0.f;
  }
  // raw tail (fused calls): split 0 computes its partial before the passes;
  // in a fused step that partial covers the rows the step adds
  const bool fold_tail = p.fused && split == 0 && (STEP || n_raw > 0);
  if constexpr (STEP && JPG) {
    if (split == 0) {
      // the fp archive kernel's arithmetic on a completed block (the
      // coefficients stored as fp32 rows), the step's rows at full precision
      const int64_t bh_s = b * p.Hkv + hkv;
      float* xk = cbuf_raw;  // the passes have not started: the end-phase buffer is free
      const int64_t kblk = (bh_s * p.kcap + step_nb) * R, vblk = (bh_s * p.vcap + step_nb) * R;
      float* kw = static_cast<float*>(const_cast<void*>(p.kfp)) + kblk * D;
      float* vw = static_cast<float*>(const_cast<void*>(p.vfp)) + vblk * D;
      step_partial<D, R, float, 0>(
          step_t, rblk, static_cast<float*>(const_cast<void*>(p.kraw)) + bh_s * rblk * D,
          static_cast<float*>(const_cast<void*>(p.vraw)) + bh_s * rblk * D,
          static_cast<const float*>(p.ktok) + b * p.kt_sb + hkv * p.kt_sh,
          static_cast<const float*>(p.vtok) + b * p.vt_sb + hkv * p.vt_sh, step_write, kw,
          nullptr, vw, nullptr, p.basis, p.A, p.q, FC_F32, b * p.q_sb, p.q_sh, hkv * p.G + g0, G,
          p.scale_log2, tid, xk, xk + rblk * D, xk + 2 * rblk * D, nullptr, scratch, part_lds,
          tail_ml[0], tail_ml[1]);
    }
  } else if constexpr (STEP) {
    if (split == 0) {
      const int64_t bh_s = b * p.Hkv + hkv;
      float* xk = cbuf_raw;  // the passes have not started: the end-phase buffer is free
      const int64_t kslot = bh_s * p.kcap + step_nb, vslot = bh_s * p.vcap + step_nb;
      const PngStepDst kd{static_cast<T*>(const_cast<void*>(p.kanch)) + kslot * D,
                          const_cast<float*>(p.kdel) + kslot * (R - 1) * D, nullptr};
      const PngStepDst vd{static_cast<T*>(const_cast<void*>(p.vanch)) + vslot * D,
                          const_cast<float*>(p.vdel) + vslot * (R - 1) * D, nullptr};
      const int n = png_step_rows<D, R, T, false>(
          step_t, R, static_cast<T*>(const_cast<void*>(p.kraw)) + bh_s * R * D,
          static_cast<T*>(const_cast<void*>(p.vraw)) + bh_s * R * D,
          static_cast<const T*>(p.ktok) + b * p.kt_sb + hkv * p.kt_sh,
          static_cast<const T*>(p.vtok) + b * p.vt_sb + hkv * p.vt_sh, step_write, kd, vd,
          p.keep_m, tid, xk, xk + R * D);
      png_step_attend<D, T>(n, static_cast<const T*>(p.q), b * p.q_sb, p.q_sh, hkv * p.G + g0, G,
                            p.scale_log2, tid, xk, xk + R * D, scratch, part_lds, tail_ml[0],
                            tail_ml[1]);
    }
  } else if (fold_tail) {
    raw_tail_partial<D, F32>(p, b, hkv, g0, G, (int)n_raw, tid, scratch, part_lds, tail_ml[0],
                             tail_ml[1]);
  }
  __syncthreads();

  while (cur < npass) {
    const int prow = (int)min<int64_t>(kPngTile, rows_total - cur * kPngTile);  // whole blocks
    load_v(cur);
    const unsigned int nxt_v = grab();

    // ------------------------------------------------------------ scores
    float4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < FPL; ++c) sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[c], qv[c], sacc, 0, 0, 0);
    if (lc < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s_lds[wave][lc][4 * lq + i] = sacc[i] * p.scale_log2;
    }
    const int64_t nxt = pass_of(nxt_v);
    if (nxt < npass) load_k(nxt);  // the next pass's rows fly during softmax and values
    wave_lds_sync();

    // ------------------------------------------------------------ softmax
    float pmax, lsum;
    weights(prow, m_run, pmax, lsum);
    if (__builtin_amdgcn_ballot_w64(pmax > m_run + kLazyMax) != 0) {
      // move the reference maxima to the pass's logits, recompute the weights
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
      for (int f = 0; f < FPC; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[f][i] *= al[i];
      m_run = m_new;
    } else {
      l_lane += lsum;
    }
    // rows past the pass end carry zero weight (their rows read as zero)
    if (prow < kPngTile)
      for (int i = prow + lane; i < kPngTile; i += 64)
        for (int h = 0; h < G; ++h) w_lds[wave][h][i] = 0.f;
    wave_lds_sync();

    // ------------------------------------------------------------ values
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const float a = lc < G ? w_lds[wave][lc][4 * rg + lq] : 0.f;
#pragma unroll
      for (int f = 0; f < FPC; ++f)
        acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vr[rg][f], acc[f], 0, 0, 0);
    }
    wave_lds_sync();
    cur = nxt;
  }

  // ---- combine the wavefronts: (max, sum, 1) per head and the accumulators
  // (lane (q, c) register i of acc[f]: head 4q + i, feature vfeat(f))
#pragma unroll
  for (int m = GP; m < 64; m <<= 1) l_lane += __shfl_xor(l_lane, m, 64);
  if (lane < GP) {
    comb[wave][lane][0] = m_run;
    comb[wave][lane][1] = l_lane;
    comb[wave][lane][2] = 1.f;
  }
  constexpr int NI = GP < 4 ? GP : 4;
  if (lq < (GP >= 4 ? GP / 4 : 1)) {
#pragma unroll
    for (int f = 0; f < FPC; ++f)
#pragma unroll
      for (int i = 0; i < NI; ++i) cbuf[wave][4 * lq + i][vfeat(f)] = acc[f][i];
  }
  // the merge of up to 32 splits reads every partial in one batch, two
  // threads per output task (C4: 32 splits per group; 2.1 us shorter than
  // batches of 8 with the statistics staged in LDS)
  // fused step with a device state: the launch's last workgroup to finish
  // (all others have read the state by then) advances it
  auto step_done = [&]() {
    if constexpr (!STEP) return;
    if (!p.state) return;
    if (tid == 0) s_final = atomicAdd(p.done, 1u) + 1 == gridDim.x ? 1 : 0;
    __syncthreads();
    if (s_final && tid < 64) {  // lane-indexed vector stores
      const int64_t cap = min(p.kcap, p.vcap);
      const bool full = step_t + 1 == rblk;
      const bool over = full && step_nb >= cap;
      const int64_t word = tid == 0   ? (full ? step_nb + 1 : step_nb)
                           : tid == 1 ? (full ? 0 : step_t + 1)
                                      : ((p.state[2] != 0 || over) ? 1 : 0);
      if (tid < 3) const_cast<int64_t*>(p.state)[tid] = word;
      if (tid == 0) __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  split_epilogue<D, GP, F32, false, decltype(step_done)&, 32>(
      p, g, b, hkv, g0, G, split, tid, fold_tail, comb, cbuf, part_lds, tail_ml, wg_ml, scratch,
      s_last, passq, step_done);
}


}  // namespace pngk

// Launch of the png pass for stream / query dtype T on `grid`: block size r
// (4, 8, 16), head size D (64, 128), gp (1, 2, 4, 8, 16) heads per group;
// the STEP variant when a.step.
template <typename T>
int launch_png_t(const MfmaArgs& a, int r, int D, int gp, dim3 grid, hipStream_t st) {
  return mfma_with_int<4, 8, 16>(r, [&](auto rc_) {
    constexpr int Rv = decltype(rc_)::value;
    return mfma_with_int<64, 128>(D, [&](auto dc) {
      constexpr int Dv = decltype(dc)::value;
      return mfma_with_int<1, 2, 4, 8, 16>(gp, [&](auto gc) {
        constexpr int GPv = decltype(gc)::value;
        if (a.step)
          pngk::attn_split_png_mfma<Rv, Dv, GPv, true, T><<<grid, kMThreads, 0, st>>>(a);
        else
          pngk::attn_split_png_mfma<Rv, Dv, GPv, false, T><<<grid, kMThreads, 0, st>>>(a);
        return FC_OK;
      });
    });
  });
}

// Launch of the pass over jpeg archives of fp32 coefficients (JPG): s
// stored rows per block (1, 2, 4, 8, 16), head size D (64, 128).
int launch_fpj32_t(const MfmaArgs& a, int s, int D, int gp, dim3 grid, hipStream_t st);

extern template int launch_png_t<float>(const MfmaArgs&, int, int, int, dim3, hipStream_t);
extern template int launch_png_t<f16_t>(const MfmaArgs&, int, int, int, dim3, hipStream_t);
extern template int launch_png_t<bf16_t>(const MfmaArgs&, int, int, int, dim3, hipStream_t);

}  // namespace fc
