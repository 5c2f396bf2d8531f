// Host side of the png matrix-core pass (kernel: fc_attn_png_kernel.h), and
// its fp32 instantiation.
#include "fc_attn_png_kernel.h"

namespace fc {

template int launch_png_t<float>(const MfmaArgs&, int, int, int, dim3, hipStream_t);

int launch_fpj32_t(const MfmaArgs& a, int s, int D, int gp, dim3 grid, hipStream_t st) {
  return mfma_with_int<1, 2, 4, 8, 16>(s, [&](auto sc) {
    constexpr int Sv = decltype(sc)::value;
    return mfma_with_int<64, 128>(D, [&](auto dc) {
      constexpr int Dv = decltype(dc)::value;
      return mfma_with_int<1, 2, 4, 8, 16>(gp, [&](auto gc) {
        constexpr int GPv = decltype(gc)::value;
        if (a.step)
          pngk::attn_split_png_mfma<Sv, Dv, GPv, true, float, true><<<grid, kMThreads, 0, st>>>(a);
        else
          pngk::attn_split_png_mfma<Sv, Dv, GPv, false, float, true><<<grid, kMThreads, 0, st>>>(a);
        return FC_OK;
      });
    });
  });
}

// Query / stream dtypes, head size and block size of the png matrix-core
// pass: queries in the stream's dtype (fp32, fp16 or bf16).
bool png_mfma_shape_supported(int q_dtype, int stream_dtype, int64_t D, int r) {
  return q_dtype == stream_dtype &&
         (stream_dtype == FC_F32 || stream_dtype == FC_F16 || stream_dtype == FC_BF16) &&
         (D == 64 || D == 128) && (r == 4 || r == 8 || r == 16);
}

// Whether the png matrix-core pass handles this call: its shapes, and 16-byte
// aligned query rows and stores (16-byte row loads).
bool split_png_mfma_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                              int r, int stream_dtype, const fc_stream_view* key,
                              const fc_stream_view* value) {
  const auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  return png_mfma_shape_supported(q_dtype, stream_dtype, D, r) && al16(q) && q_sb % 4 == 0 &&
         q_sh % 4 == 0 && al16(key->rows) && al16(value->rows) && al16(key->anchors) &&
         al16(value->anchors);
}

int launch_split_png_mfma(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                          int64_t Hq, int64_t Hkv, int64_t D, int r, int64_t nb,
                          const fc_stream_view* key,
                          const fc_stream_view* value, float scale_log2, float* pm, float* pl,
                          float* pacc, int n_splits, unsigned int* counters,
                          int64_t counter_words, int64_t stride, const MfmaFuse* fuse,
                          const int64_t* state, hipStream_t st) {
  MfmaArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.raw_dtype = q_dtype;  // the stream's dtype (anchors, tails, tokens): the queries'
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.kanch = key->anchors;
  a.vanch = value->anchors;
  a.kdel = static_cast<const float*>(key->rows);
  a.vdel = static_cast<const float*>(value->rows);
  a.kcap = key->cap;
  a.vcap = value->cap;
  a.Hkv = Hkv;
  a.G = Hq / Hkv;
  a.nb = nb;
  a.r = r;
  a.scale_log2 = scale_log2;
  a.n_splits = n_splits;
  a.pm = pm;
  a.pl = pl;
  a.pacc = pacc;
  a.state = state;
  if (fuse) {
    if (n_splits > kFuseMaxSplits) return FC_ERR_ARG;
    a.fused = 1;
    a.kraw = key->raw;
    a.vraw = value->raw;
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
      a.step_t = fuse->step_t;
      a.step_nb = fuse->step_nb;
      a.done = fuse->done;
      a.keep_m = fuse->keep_m;
      if (!fuse->done) return FC_ERR_ARG;
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
  const int rc = q_dtype == FC_F16    ? launch_png_t<f16_t>(a, r, (int)D, gp, grid, st)
                 : q_dtype == FC_BF16 ? launch_png_t<bf16_t>(a, r, (int)D, gp, grid, st)
                                      : launch_png_t<float>(a, r, (int)D, gp, grid, st);
  if (rc != FC_OK) return rc;
  return check_launch();
}

}  // namespace fc
