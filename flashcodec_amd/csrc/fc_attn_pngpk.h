// Split pass of the decode attention for packed png archives: the kernel
// template (instantiated in fc_attn_pngpk_<r>_<m>.hip, one translation unit
// per block-size / kept-delta bucket; the host side is fc_attn_pngpk.hip)
// (fc_png_encode_packed: per (block, feature) the keep_m Top-M deltas in
// step order plus one mask word) on gfx950, with the merge of the split
// partials fused in (the epilogue of the matrix-core passes).
//
// A png block of r tokens is its anchor (row 0, stream dtype) and r - 1
// fp32 deltas (rows 1 .. r-1); token t = sum_{j <= t} row_j
// (flashcodec/codecs/png.py:36-74), so for a query q
// (flashcodec/attention.py:45-61, A lower-triangular ones):
//   logit_t = scale * sum_{j <= t} (q . row_j)    prefix sums of the scores
//   out    += sum_j (sum_{t >= j} p_t) row_j      suffix sums of the weights
// In the packed layout only keep_m of a feature's r - 1 deltas are stored;
// the others are zero.
//
// Work layout: lane (segment, l) owns features 4l .. 4l+3 of one block; a
// block is D / 4 lanes, so a wavefront takes 256 / D blocks per iteration
// and every load instruction reads 4 D contiguous bytes of a block (its
// anchor, its mask words, one value slot).
//   scores: each lane walks its features' steps (a kept step takes the
//     feature's next slot value, others are zero) and accumulates the
//     partial scores of 64 / R heads x R steps; a reduce-scatter over the
//     block's lanes leaves each lane 256 / D totals, parked in LDS;
//   softmax: one (block, head) pair per lane: logits as prefix sums,
//     exponentials against a running reference maximum that moves only
//     when a logit exceeds it by 2^8 (accumulators rescaled then), row
//     weights as suffix sums, into LDS as [step][head];
//   values: for each stored slot the lane reads its step's weights for all
//     heads (16-byte LDS reads) and accumulates weight x value; pruned
//     steps cost nothing.
// Products and sums are fp32 (fp32 queries meet the 1e-5 tolerance).  A
// wavefront takes iterations of its workgroup's block range round robin and
// requests the next iteration's K and V data at the start of each.
#pragma once

#include "fc_attn_mfma_kernel.h"
#include "fc_png_step.h"

namespace fc {

namespace pngpk {

constexpr int kPkF = 4;  // features per lane

// Reduce-scatter of 64 per-lane values over aligned groups of LB lanes:
// afterwards lane l of a group holds, in v[0 .. 64/LB), the group totals of
// values l * (64/LB) .. l * (64/LB) + 64/LB - 1.  Stage S (from LB/2 down to
// 1) adds the value halves of lanes l and a partner that differs in bit S
// and agrees on the higher bits; lanes with bit S set keep the upper half.
// Across rows the gfx950 permlane swaps exchange both halves in one
// instruction; inside a row the partners are DPP mirrors and quad
// permutations (which also flip lower bits: those stages come later).
template <int S>
__device__ __forceinline__ float dpp_partner(float x) {
  constexpr int ctrl = S == 8 ? 0x140 : S == 4 ? 0x141 : S == 2 ? 0x4E : 0xB1;
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xf, 0xf, false));
}

template <int S, int HALF>
__device__ __forceinline__ void reduce_scatter_stage(float (&v)[64], int l) {
  if constexpr (S >= 16) {
#pragma unroll
    for (int e = 0; e < HALF; ++e) {
      // lanes without bit S: (own lower half, partner's lower half); with
      // it: (partner's upper half, own upper half)
      const auto sw = S == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v[e]),
                                                                 __float_as_uint(v[e + HALF]),
                                                                 false, false)
                              : __builtin_amdgcn_permlane16_swap(__float_as_uint(v[e]),
                                                                 __float_as_uint(v[e + HALF]),
                                                                 false, false);
      v[e] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    reduce_scatter_stage<S / 2, HALF / 2>(v, l);
  } else if constexpr (S >= 1) {
    const bool up = (l & S) != 0;
#pragma unroll
    for (int e = 0; e < HALF; ++e) {
      const float keep = up ? v[e + HALF] : v[e];
      const float send = up ? v[e] : v[e + HALF];
      v[e] = keep + dpp_partner<S>(send);
    }
    reduce_scatter_stage<S / 2, HALF / 2>(v, l);
  }
}

template <int LB>
__device__ __forceinline__ void reduce_scatter64(float (&v)[64], int l) {
  reduce_scatter_stage<LB / 2, 32>(v, l);
}

// Scans and maxima over aligned groups of GL lanes (GL <= 16, inside a
// 16-lane row): inclusive prefix (lanes <= l of the group), inclusive suffix
// (lanes >= l) and the group maximum in every lane.  l = lane index.
template <int S>
__device__ __forceinline__ float dpp_shr(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + S, 0xf, 0xf, true));
}
template <int S>
__device__ __forceinline__ float dpp_shl(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + S, 0xf, 0xf, true));
}

template <int GL, int S = 1>
__device__ __forceinline__ float group_prefix(float x, int l) {
  if constexpr (S < GL) {
    const float y = dpp_shr<S>(x);
    x += (l % GL) >= S ? y : 0.f;
    return group_prefix<GL, 2 * S>(x, l);
  } else {
    return x;
  }
}

template <int GL, int S = 1>
__device__ __forceinline__ float group_suffix(float x, int l) {
  if constexpr (S < GL) {
    const float y = dpp_shl<S>(x);
    x += (l % GL) + S < GL ? y : 0.f;
    return group_suffix<GL, 2 * S>(x, l);
  } else {
    return x;
  }
}

template <int GL>
__device__ __forceinline__ float group_max_lanes(float x) {
  if constexpr (GL >= 2) x = fmaxf(x, dpp_partner<1>(x));
  if constexpr (GL >= 4) x = fmaxf(x, dpp_partner<2>(x));
  if constexpr (GL >= 8) x = fmaxf(x, dpp_partner<4>(x));
  if constexpr (GL >= 16) x = fmaxf(x, dpp_partner<8>(x));
  return x;
}

// four elements of an anchor row (fp32, or 16-bit bf16 / f16 chosen at run
// time) from their raw load
struct AnchorRaw {
  u32x4_t w;
};

__device__ __forceinline__ AnchorRaw load_anchor4(const void* base, int64_t elem, bool f32) {
  AnchorRaw a;
  if (f32) {
    a.w = *reinterpret_cast<const u32x4_t*>(static_cast<const float*>(base) + elem);
  } else {
    const u32x2_t h = *reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(base) + elem);
    a.w = (u32x4_t){h[0], h[1], 0u, 0u};
  }
  return a;
}

__device__ __forceinline__ void anchor_values(const AnchorRaw& a, int dt, float (&x)[kPkF]) {
  if (dt == FC_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(a.w[i]);
  } else if (dt == FC_BF16) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      x[2 * i] = __uint_as_float(a.w[i] << 16);
      x[2 * i + 1] = __uint_as_float(a.w[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      x[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(a.w[i] & 0xffffu));
      x[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(a.w[i] >> 16));
    }
  }
}

// One block's packed data for this lane's four features.
template <int MB>
struct PkData {
  AnchorRaw a;
  u32x4_t mask;
  float4_t v[MB];
};

// RB: block size bucket (r <= RB), D: head size, GP: heads per workgroup
// (>= G), MB: value slots bucket (keep_m <= MB), QF32: fp32 queries (else
// fp16 / bf16, outputs in the query dtype).  STEP: the fused decode step
// (fc_decode_step; MfmaArgs.step): split 0 appends the token or archives
// the block it completes in the packed layout (png_step_rows) and attends
// the step's rows, the iterations cover the blocks before it.
template <int RB, int D, int GP, int MB, bool QF32, bool STEP = false>
__global__ __launch_bounds__(kMThreads, GP <= 4 ? 2 : 1) void attn_split_pngpk(MfmaArgs p) {
  constexpr int F = kPkF;
  constexpr int LB = D / F;            // lanes per block
  constexpr int NB = 64 / LB;          // blocks per wavefront iteration
  constexpr int HS = 64 / RB;          // heads per score subset (HS x RB partials)
  constexpr int NSUB = (GP + HS - 1) / HS;
  constexpr int GS = NSUB * HS;        // heads with a score row in LDS
  static_assert(LB >= 16 && LB <= 64 && NB * GP <= 64 && GP % 4 == 0, "lane layout");
  constexpr int GL = RB / NB;          // lanes of one head's steps after the reduce-scatter
  constexpr int kW = kWaves * NB * RB * GP;  // weights [wave][blk][step][head]
  constexpr int kC = kWaves * GP * D;        // end phase: cbuf [wave][head][feature]
  constexpr int kBig0 = kW > kC ? kW : kC;
  constexpr int kBig = STEP && 2 * RB * D > kBig0 ? 2 * RB * D : kBig0;  // STEP: the step's rows
  __shared__ __attribute__((aligned(16))) float big[kBig];
  __shared__ float comb[kWaves][16][3];
  __shared__ __attribute__((aligned(16))) float part_lds[16 * D];
  __shared__ float tail_ml[2][16];
  __shared__ float wg_ml[2][16];
  __shared__ float scratch[2 * 16 * kFuseMaxSplits];  // raw-tail logits, then merge statistics
  __shared__ int s_last;
  __shared__ int s_final;

  // 1-D grid, split-major with a per-split rotation, as the other passes
  const int64_t L = blockIdx.x;
  const int split = (int)(L / p.ngroups);
  const int64_t g = ((L % p.ngroups) - split % p.ngroups + p.ngroups) % p.ngroups;
  const int64_t bh = g / p.zg;
  const int64_t g0 = (g % p.zg) * 16;
  const int64_t b = bh / p.Hkv, hkv = bh - b * p.Hkv;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = (int)min<int64_t>(16, p.G - g0);
  const int r = p.r, km = p.keep_m;
  const int adt = p.raw_dtype;  // anchor (stream) dtype
  const bool a32 = adt == FC_F32;

  int64_t nb = p.nb, n_raw = p.n_raw;
  int64_t step_t = 0, step_nb = 0;  // fused step: tail length and blocks before the token
  bool step_write = false;
  if constexpr (STEP) {
    const int64_t cap = min(p.kcap, p.vcap);
    step_t = p.state ? min<int64_t>(max<int64_t>(p.state[1], 0), r - 1) : p.step_t;
    step_nb = p.state ? max<int64_t>(p.state[0], 0) : p.step_nb;
    // one head group per (batch, kv head) stores the token / block; a block
    // past the capacity is not stored (the state's overflow word says so)
    step_write = split == 0 && g0 == 0 && (step_t + 1 < r || step_nb < cap);
    nb = min(step_nb, cap);
    n_raw = 0;
  } else if (p.state) {
    // counts of a decode step's view on the device (graph replays)
    const int64_t t = min<int64_t>(max<int64_t>(p.state[1], 0), r - 1) + 1;
    nb = min<int64_t>(max<int64_t>(p.state[0], 0) + (t == r ? 1 : 0), min(p.kcap, p.vcap));
    n_raw = t == r ? 0 : t;
  }
  const int64_t bps = (nb + p.n_splits - 1) / p.n_splits;
  const int64_t blo = min<int64_t>(nb, (int64_t)split * bps);
  const int64_t bhi = min<int64_t>(nb, blo + bps);
  const int64_t nit = (bhi - blo + NB - 1) / NB;
  unsigned int* passq = p.passq + g * p.cstride;

  const int seg = lane / LB, sl = lane % LB;
  const int f0 = F * sl;
  const int64_t kblk0 = bh * p.kcap, vblk0 = bh * p.vcap;
  const uint32_t* kmask = p.kmask;
  const uint32_t* vmask = p.vmask;

  auto load_blk = [&](const void* anch, const float* vals, const uint32_t* masks, int64_t blk0,
                      int64_t it, PkData<MB>& x) {
    int64_t bi = blo + it * NB + seg;
    bi = bi < bhi ? bi : blo;  // rows past the range: a valid block, weighted zero
    const int64_t slot = blk0 + bi;
    x.a = load_anchor4(anch, slot * D + f0, a32);
    x.mask = *reinterpret_cast<const u32x4_t*>(masks + slot * D + f0);
#pragma unroll
    for (int j = 0; j < MB; ++j)
      if (j < km)
        x.v[j] = *reinterpret_cast<const float4_t*>(vals + (slot * km + j) * D + f0);
  };

  // ---- queries: heads of this workgroup, this lane's four features (fp32)
  float qv[GP][F];
#pragma unroll
  for (int h = 0; h < GP; ++h) {
    const int64_t hq = hkv * p.G + g0 + (h < G ? h : 0);
    const int64_t qo = b * p.q_sb + hq * p.q_sh + f0;
    if constexpr (QF32) {
      const float4_t x = *reinterpret_cast<const float4_t*>(static_cast<const float*>(p.q) + qo);
#pragma unroll
      for (int f = 0; f < F; ++f) qv[h][f] = h < G ? x[f] : 0.f;
    } else {
      AnchorRaw x;
      const u32x2_t hw = *reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(p.q) + qo);
      x.w = (u32x4_t){hw[0], hw[1], 0u, 0u};
      float t[F];
      anchor_values(x, p.q_dtype, t);
#pragma unroll
      for (int f = 0; f < F; ++f) qv[h][f] = h < G ? t[f] : 0.f;
    }
  }

  float acc[GP][F];
#pragma unroll
  for (int h = 0; h < GP; ++h)
#pragma unroll
    for (int f = 0; f < F; ++f) acc[h][f] = 0.f;
  // after a subset's reduce-scatter lane (segment, l) holds steps i0 ..
  // i0 + NB - 1 of head hl of the subset (GL lanes per head): its running
  // reference maximum and share of the exponential sum, per subset
  const int k0 = sl * NB;
  const int hl = k0 / RB, i0 = k0 - hl * RB;
  float m_run[NSUB], l_lane[NSUB];
#pragma unroll
  for (int u = 0; u < NSUB; ++u) {
    m_run[u] = -INFINITY;
    l_lane[u] = 0.f;
  }

  float* const w_w = big + (wave * NB) * RB * GP;  // this wavefront's weights

  // K and V data of the iteration (kd, vd) and of the wavefront's next one
  // (kn, vn), requested one iteration ahead
  PkData<MB> kd, vd, kn, vn;
  int64_t it = wave;
  if (it < nit) {
    load_blk(p.kanch, p.kdel, kmask, kblk0, it, kd);
    load_blk(p.vanch, p.vdel, vmask, vblk0, it, vd);
  }

  // raw tail (fused calls): split 0 computes its partial before the passes;
  // in a fused step that partial covers the rows the step adds
  const bool fold_tail = p.fused && split == 0 && (STEP || n_raw > 0);
  if constexpr (STEP) {
    if (split == 0) {
      const int64_t bh_s = b * p.Hkv + hkv;
      const int64_t kslot = bh_s * p.kcap + step_nb, vslot = bh_s * p.vcap + step_nb;
      float* xk = big;  // the iterations have not started: their weight buffer is free
      float* xv = big + RB * D;
      const int64_t qb = b * p.q_sb, h0 = hkv * p.G + g0;
      auto go = [&](auto tt) {
        using T = decltype(tt);
        const PngStepDst kdst{static_cast<T*>(const_cast<void*>(p.kanch)) + kslot * D,
                            const_cast<float*>(p.kdel) + kslot * km * D,
                            const_cast<uint32_t*>(kmask) + kslot * D};
        const PngStepDst vdst{static_cast<T*>(const_cast<void*>(p.vanch)) + vslot * D,
                            const_cast<float*>(p.vdel) + vslot * km * D,
                            const_cast<uint32_t*>(vmask) + vslot * D};
        const int n = png_step_rows<D, RB, T, true>(
            step_t, r, static_cast<T*>(const_cast<void*>(p.kraw)) + bh_s * r * D,
            static_cast<T*>(const_cast<void*>(p.vraw)) + bh_s * r * D,
            static_cast<const T*>(p.ktok) + b * p.kt_sb + hkv * p.kt_sh,
            static_cast<const T*>(p.vtok) + b * p.vt_sb + hkv * p.vt_sh, step_write, kdst, vdst,
            km, tid, xk, xv);
        if constexpr (QF32)
          png_step_attend<D, float>(n, static_cast<const float*>(p.q), qb, p.q_sh, h0, G,
                                    p.scale_log2, tid, xk, xv, scratch, part_lds, tail_ml[0],
                                    tail_ml[1]);
        else if (p.q_dtype == FC_F16)
          png_step_attend<D, f16_t>(n, static_cast<const f16_t*>(p.q), qb, p.q_sh, h0, G,
                                    p.scale_log2, tid, xk, xv, scratch, part_lds, tail_ml[0],
                                    tail_ml[1]);
        else
          png_step_attend<D, bf16_t>(n, static_cast<const bf16_t*>(p.q), qb, p.q_sh, h0, G,
                                     p.scale_log2, tid, xk, xv, scratch, part_lds, tail_ml[0],
                                     tail_ml[1]);
      };
      if (adt == FC_F16)
        go(f16_t{});
      else if (adt == FC_BF16)
        go(bf16_t{});
      else
        go(float{});
    }
  } else if (fold_tail) {
    raw_tail_partial<D, QF32>(p, b, hkv, g0, G, (int)n_raw, tid, scratch, part_lds, tail_ml[0],
                              tail_ml[1]);
  }
  __syncthreads();

  const float sl2 = p.scale_log2;
  while (it < nit) {
    const int64_t nxt = it + kWaves;
    if (nxt < nit) {
      load_blk(p.kanch, p.kdel, kmask, kblk0, nxt, kn);
      load_blk(p.vanch, p.vdel, vmask, vblk0, nxt, vn);
    }
    const int64_t bi0 = blo + it * NB;  // first block of the iteration

    // ------------------------------------------------------------ scores
    {
      float ka[F];
      anchor_values(kd.a, adt, ka);
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        float P[64];
#pragma unroll
        for (int e = 0; e < 64; ++e) P[e] = 0.f;
#pragma unroll
        for (int hh = 0; hh < HS; ++hh) {
          const int h = sub * HS + hh;
          if (h < GP) {
            float s0 = 0.f;
#pragma unroll
            for (int f = 0; f < F; ++f) s0 = __builtin_fmaf(qv[h][f], ka[f], s0);
            P[hh * RB] = s0;
          }
        }
        // shift registers of the features' slot values: a kept step takes
        // slot 0 and the rest move down
        float cur[F][MB];
#pragma unroll
        for (int f = 0; f < F; ++f)
#pragma unroll
          for (int j = 0; j < MB; ++j) cur[f][j] = kd.v[j][f];
#pragma unroll
        // steps past r - 1 have no mask bit: they add zeros, no branch
        for (int i = 1; i < RB; ++i) {
          float d[F];
#pragma unroll
          for (int f = 0; f < F; ++f) {
            const bool kept = (kd.mask[f] >> (i - 1)) & 1u;
            d[f] = kept ? cur[f][0] : 0.f;
#pragma unroll
            for (int j = 0; j + 1 < MB; ++j) cur[f][j] = kept ? cur[f][j + 1] : cur[f][j];
          }
#pragma unroll
          for (int hh = 0; hh < HS; ++hh) {
            const int h = sub * HS + hh;
            if (h < GP) {
              float s = P[hh * RB + i];
#pragma unroll
              for (int f = 0; f < F; ++f) s = __builtin_fmaf(qv[h][f], d[f], s);
              P[hh * RB + i] = s;
            }
          }
        }
        reduce_scatter64<LB>(P, sl);

        // -------------------------------------------------- softmax (in
        // registers): logits are prefix sums of the scaled scores over the
        // head's steps (local, then across its GL lanes), exponentials
        // against the running reference maximum, weights suffix sums
        const int hg = sub * HS + hl;  // this lane's head in the workgroup
        const bool head_ok = hg < G && bi0 + seg < bhi;
        float run[NB];
        float tot = 0.f;
#pragma unroll
        for (int e = 0; e < NB; ++e) {
          tot += P[e] * sl2;
          run[e] = tot;
        }
        const float ex = group_prefix<GL>(tot, sl) - tot;
        float pmax = -INFINITY;
#pragma unroll
        for (int e = 0; e < NB; ++e) {
          run[e] += ex;
          const bool live = head_ok && i0 + e < r;
          pmax = live ? fmaxf(pmax, run[e]) : pmax;
        }
        if (__builtin_amdgcn_ballot_w64(pmax > m_run[sub] + kLazyMax) != 0) {
          // move the head's reference maximum to its largest logit so far
          float hm = group_max_lanes<GL>(pmax);
#pragma unroll
          for (int s2 = LB; s2 < 64; s2 <<= 1) hm = fmaxf(hm, __shfl_xor(hm, s2, 64));
          const float m_new = fmaxf(m_run[sub], hm);
          const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run[sub] - m_new);
          l_lane[sub] *= alpha;
#pragma unroll
          for (int hh = 0; hh < HS; ++hh) {
            const int h = sub * HS + hh;
            if (h < GP) {
              const float al = __shfl(alpha, hh * GL, 64);  // segment 0, head hh's first lane
#pragma unroll
              for (int f = 0; f < F; ++f) acc[h][f] *= al;
            }
          }
          m_run[sub] = m_new;
        }
        float ev[NB];
        float esum = 0.f;
#pragma unroll
        for (int e = 0; e < NB; ++e) {
          const bool live = head_ok && i0 + e < r;
          ev[e] = live ? __builtin_amdgcn_exp2f(run[e] - m_run[sub]) : 0.f;
          esum += ev[e];
        }
        l_lane[sub] += esum;
        const float sx = group_suffix<GL>(esum, sl) - esum;
        if (hg < GP) {
          float z = sx;
#pragma unroll
          for (int e = NB - 1; e >= 0; --e) {
            z += ev[e];
            w_w[(seg * RB + i0 + e) * GP + hg] = z;
          }
        }
      }
    }
    wave_lds_sync();

    // ------------------------------------------------------------ values
    {
      const bool ok = bi0 + seg < bhi;
      float va[F];
      anchor_values(vd.a, adt, va);
      const float* wb = w_w + seg * RB * GP;
#pragma unroll
      for (int h4 = 0; h4 < GP / 4; ++h4) {
        const float4_t w = *reinterpret_cast<const float4_t*>(wb + 4 * h4);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int f = 0; f < F; ++f)
            acc[4 * h4 + c][f] = __builtin_fmaf(w[c], ok ? va[f] : 0.f, acc[4 * h4 + c][f]);
      }
#pragma unroll
      for (int f = 0; f < F; ++f) {
        uint32_t rem = vd.mask[f] & 0x7fffu;
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          // slots past keep_m (a smaller count than the bucket's) weigh zero
          const int step = (rem ? __builtin_ctz(rem) : 0) + 1;
          rem &= rem - 1u;
          const float x = (ok && j < km) ? vd.v[j][f] : 0.f;
          const float* wr = wb + min(step, r - 1) * GP;
#pragma unroll
          for (int h4 = 0; h4 < GP / 4; ++h4) {
            const float4_t w = *reinterpret_cast<const float4_t*>(wr + 4 * h4);
#pragma unroll
            for (int c = 0; c < 4; ++c)
              acc[4 * h4 + c][f] = __builtin_fmaf(w[c], x, acc[4 * h4 + c][f]);
          }
        }
      }
    }
    wave_lds_sync();
    kd = kn;
    vd = vn;
    it = nxt;
  }

  // ---- combine: the iteration's blocks (segments) hold partial sums of the
  // same features, the GL lanes of a head (in every segment) partial
  // exponential sums
#pragma unroll
  for (int s2 = LB; s2 < 64; s2 <<= 1)
#pragma unroll
    for (int h = 0; h < GP; ++h)
#pragma unroll
      for (int f = 0; f < F; ++f) acc[h][f] += __shfl_xor(acc[h][f], s2, 64);
#pragma unroll
  for (int u = 0; u < NSUB; ++u) {
    float l = l_lane[u];
#pragma unroll
    for (int s2 = 1; s2 < GL; s2 <<= 1) l += __shfl_xor(l, s2, 64);
#pragma unroll
    for (int s2 = LB; s2 < 64; s2 <<= 1) l += __shfl_xor(l, s2, 64);
    l_lane[u] = l;
  }
  __syncthreads();  // cbuf takes the LDS of every wavefront's weights
  auto& cbuf = *reinterpret_cast<float (*)[kWaves][GP][D]>(big);
  if (seg == 0 && sl % GL == 0) {
#pragma unroll
    for (int u = 0; u < NSUB; ++u) {
      const int h = u * HS + hl;
      if (h < GP) {
        comb[wave][h][0] = m_run[u];
        comb[wave][h][1] = l_lane[u];
        comb[wave][h][2] = 1.f;
      }
    }
  }
  if (seg == 0) {
#pragma unroll
    for (int h = 0; h < GP; ++h)
      *reinterpret_cast<float4_t*>(&cbuf[wave][h][f0]) =
          (float4_t){acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
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
      const bool full = step_t + 1 == r;
      const bool over = full && step_nb >= cap;
      const int64_t word = tid == 0   ? (full ? step_nb + 1 : step_nb)
                           : tid == 1 ? (full ? 0 : step_t + 1)
                                      : ((p.state[2] != 0 || over) ? 1 : 0);
      if (tid < 3) const_cast<int64_t*>(p.state)[tid] = word;
      if (tid == 0) __hip_atomic_store(p.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  split_epilogue<D, GP, QF32, false, decltype(step_done)&, 32>(
      p, g, b, hkv, g0, G, split, tid, fold_tail, comb, cbuf, part_lds, tail_ml, wg_ml, scratch,
      s_last, passq, step_done);
}

}  // namespace pngpk

// Launch of the packed png pass for the (block size, kept deltas) bucket
// (RB, MB), dispatched on the head size, the head-group size and the query
// dtype.
template <int RB, int MB>
int launch_pngpk_rows(const MfmaArgs& a, int D, int gp, bool qf32, dim3 grid, hipStream_t st) {
  return mfma_with_int<64, 128, 256>(D, [&](auto dc) {
    constexpr int Dv = decltype(dc)::value;
    return mfma_with_int<4, 16>(gp, [&](auto gc) {
      constexpr int GPv = decltype(gc)::value;
      if (a.step && qf32)
        pngpk::attn_split_pngpk<RB, Dv, GPv, MB, true, true><<<grid, kMThreads, 0, st>>>(a);
      else if (a.step)
        pngpk::attn_split_pngpk<RB, Dv, GPv, MB, false, true><<<grid, kMThreads, 0, st>>>(a);
      else if (qf32)
        pngpk::attn_split_pngpk<RB, Dv, GPv, MB, true><<<grid, kMThreads, 0, st>>>(a);
      else
        pngpk::attn_split_pngpk<RB, Dv, GPv, MB, false><<<grid, kMThreads, 0, st>>>(a);
      return FC_OK;
    });
  });
}

extern template int launch_pngpk_rows<4, 4>(const MfmaArgs&, int, int, bool, dim3, hipStream_t);
extern template int launch_pngpk_rows<8, 4>(const MfmaArgs&, int, int, bool, dim3, hipStream_t);
extern template int launch_pngpk_rows<8, 8>(const MfmaArgs&, int, int, bool, dim3, hipStream_t);
extern template int launch_pngpk_rows<16, 4>(const MfmaArgs&, int, int, bool, dim3, hipStream_t);
extern template int launch_pngpk_rows<16, 8>(const MfmaArgs&, int, int, bool, dim3, hipStream_t);

}  // namespace fc
