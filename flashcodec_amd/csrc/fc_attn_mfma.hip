// Host side of the matrix-core split pass of the decode attention (int8
// jpeg archives): which configurations it takes, and its launch.  The kernel
// is fc_attn_mfma_kernel.h.
#include "fc_attn_mfma_kernel.h"

namespace fc {

// Query dtypes, head sizes and stored rows per block the matrix-core split
// pass is built for (fp32 queries: not in the fused step's kernels).
bool mfma_shape_supported(int q_dtype, int64_t D, int s) {
  return (q_dtype == FC_F16 || q_dtype == FC_BF16 || q_dtype == FC_F32) &&
         (D == 64 || D == 80 || D == 96 || D == 128 || D == 256) &&
         (s == 1 || s == 2 || s == 3 || s == 4 || s == 8);
}

// Whether the matrix-core split pass handles this configuration.
// The pass reads 16 query bytes and 16 code bytes per load: the query rows
// and both code stores must be 16-byte aligned (query strides: multiples of
// 8 elements).
bool split_i8_mfma_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                             int s, const fc_stream_view* key, const fc_stream_view* value) {
  const auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  return mfma_shape_supported(q_dtype, D, s) && al16(q) && q_sb % 8 == 0 && q_sh % 8 == 0 &&
         al16(key->rows) && al16(value->rows);
}

bool split_i8_mfma_fusable(int n_splits) { return n_splits <= kFuseMaxSplits; }

// Per-32 scales (FC_STORE_JPEG_I8G) on the matrix-core pass: head sizes 64
// / 96 / 128 / 256 (whole groups of 32 features).
bool mfma_group_shape_supported(int q_dtype, int64_t D, int s) {
  return D % 32 == 0 && mfma_shape_supported(q_dtype, D, s);
}

// Whether the int8 matrix-core split pass takes this call's stores: int8
// jpeg archives with one scale per row, or per-32 scales (16-byte aligned:
// a row's scales are read in 8- / 16-byte pieces).
bool i8_mfma_takes(int store_kind, const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                   int64_t D, int s, const fc_stream_view* key, const fc_stream_view* value) {
  const auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  if (store_kind == FC_STORE_JPEG_I8G) {
    if (!mfma_group_shape_supported(q_dtype, D, s) || !al16(key->scales) ||
        !al16(value->scales))
      return false;
  } else if (store_kind != FC_STORE_JPEG_I8) {
    return false;
  }
  return split_i8_mfma_supported(q, q_dtype, q_sb, q_sh, D, s, key, value);
}

bool step_i8_mfma_supported(int stream_dtype, int r, int64_t D, int n_splits) {
  // the step's rows (2 r D floats) live in the score scratch before the passes
  return (stream_dtype == FC_F16 || stream_dtype == FC_BF16 || stream_dtype == FC_F32) &&
         split_i8_mfma_fusable(n_splits) &&
         2 * (int64_t)r * D <= (int64_t)kWaves * 16 * kSPad;
}

int launch_split_i8_mfma(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t D, int r, int s, int64_t nb,
                         const fc_stream_view* key, const fc_stream_view* value, const float* A,
                         float scale_log2, float* pm, float* pl, float* pacc, int n_splits,
                         unsigned int* counters, int64_t counter_words, int64_t stride,
                         const MfmaFuse* fuse, hipStream_t st, bool grouped) {
  MfmaArgs a{};
  a.qgroup = grouped ? 1 : 0;
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
    a.state = fuse->state;
    if (fuse->step) {
      a.step = 1;
      a.ktok = fuse->ktok;
      a.vtok = fuse->vtok;
      a.kt_sb = fuse->kt_sb;
      a.kt_sh = fuse->kt_sh;
      a.vt_sb = fuse->vt_sb;
      a.vt_sh = fuse->vt_sh;
      a.kcodes_w = const_cast<int8_t*>(a.kcodes);
      a.vcodes_w = const_cast<int8_t*>(a.vcodes);
      a.kscales_w = const_cast<float*>(a.kscales);
      a.vscales_w = const_cast<float*>(a.vscales);
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
  const int rc = mfma_with_int<FC_MFMA_ROWS_LIST>(s, [&](auto sc) {
    constexpr int SR = decltype(sc)::value;
    return grouped ? launch_mfma_rows_g<SR>(a, (int)D, gp, grid, st)
                   : launch_mfma_rows<SR>(a, (int)D, gp, grid, st);
  });
  if (rc != FC_OK) return rc;
  return check_launch();
}

}  // namespace fc
