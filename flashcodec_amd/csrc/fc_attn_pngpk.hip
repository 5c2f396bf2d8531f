// Host side of the packed png split pass (kernel: fc_attn_pngpk.h).
#include "fc_attn_pngpk.h"

namespace fc {

// Head sizes, block sizes and kept-delta counts of the packed png pass.
bool pngpk_shape_supported(int q_dtype, int stream_dtype, int64_t D, int r, int keep_m) {
  return (q_dtype == FC_F32 || q_dtype == FC_F16 || q_dtype == FC_BF16) &&
         (stream_dtype == FC_F32 || stream_dtype == FC_F16 || stream_dtype == FC_BF16) &&
         (D == 64 || D == 128 || D == 256) && r >= 2 && r <= 16 && keep_m >= 1 &&
         keep_m <= 8 && keep_m <= r - 1;
}

// The pass's loads: 16-byte query rows (8-byte for 16-bit queries) and
// 16-byte rows of values and masks; anchors 16 / 8-byte.
bool split_pngpk_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                           int r, int keep_m, int stream_dtype, const fc_stream_view* key,
                           const fc_stream_view* value) {
  const auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  return pngpk_shape_supported(q_dtype, stream_dtype, D, r, keep_m) && al16(q) &&
         q_sb % 4 == 0 && q_sh % 4 == 0 && al16(key->rows) && al16(value->rows) &&
         al16(key->masks) && al16(value->masks) && al16(key->anchors) && al16(value->anchors);
}

int launch_split_pngpk(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                       int64_t Hq, int64_t Hkv, int64_t D, int r, int keep_m, int stream_dtype,
                       int64_t nb, const fc_stream_view* key, const fc_stream_view* value,
                       float scale_log2, float* pm, float* pl, float* pacc, int n_splits,
                       unsigned int* counters, int64_t counter_words, int64_t stride,
                       const MfmaFuse* fuse, const int64_t* state, hipStream_t st) {
  MfmaArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.kanch = key->anchors;
  a.vanch = value->anchors;
  a.kdel = static_cast<const float*>(key->rows);
  a.vdel = static_cast<const float*>(value->rows);
  a.kmask = key->masks;
  a.vmask = value->masks;
  a.keep_m = keep_m;
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
  a.raw_dtype = stream_dtype;  // the anchors' dtype (and the tails')
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
      if (!fuse->done) return FC_ERR_ARG;
    }
  }
  const int64_t G = Hq / Hkv;
  a.zg = (int)((G + 15) / 16);
  a.ngroups = B * Hkv * a.zg;
  if (!counters || 2 * a.ngroups * stride > counter_words) return FC_ERR_ARG;
  a.arrive = counters;
  a.passq = counters + counter_words / 2;
  a.static_passes = 1;
  a.cstride = stride;
  const int gp = G <= 4 ? 4 : 16;
  const int rb = r <= 4 ? 4 : r <= 8 ? 8 : 16;
  const int mb = keep_m <= 4 ? 4 : 8;
  const dim3 grid((unsigned)(a.ngroups * n_splits));
  const bool qf32 = q_dtype == FC_F32;
  int rc;
  if (rb == 4)
    rc = launch_pngpk_rows<4, 4>(a, (int)D, gp, qf32, grid, st);
  else if (rb == 8)
    rc = mb == 4 ? launch_pngpk_rows<8, 4>(a, (int)D, gp, qf32, grid, st)
                 : launch_pngpk_rows<8, 8>(a, (int)D, gp, qf32, grid, st);
  else
    rc = mb == 4 ? launch_pngpk_rows<16, 4>(a, (int)D, gp, qf32, grid, st)
                 : launch_pngpk_rows<16, 8>(a, (int)D, gp, qf32, grid, st);
  if (rc != FC_OK) return rc;
  return check_launch();
}

}  // namespace fc
