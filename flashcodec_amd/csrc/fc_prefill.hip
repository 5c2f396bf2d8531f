// Causal prefill attention over an int8 jpeg archive without the
// reconstructed view: the entry point, and the kernel variants with the
// vector-ALU softmax (the kernel and its description: fc_prefill_kernel.h).
#include "fc_prefill_kernel.h"
#include "fc_prefill_wg.h"

namespace fc {

template int launch_prefill<1, 0>(const PrefillArgs&, int, int, int, bool, unsigned, hipStream_t);
template int launch_prefill<2, 0>(const PrefillArgs&, int, int, int, bool, unsigned, hipStream_t);
template int launch_prefill<4, 0>(const PrefillArgs&, int, int, int, bool, unsigned, hipStream_t);

}  // namespace fc

using namespace fc;

extern "C" {

int fc_prefill_attention(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t q_st,
                         int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D, int64_t P0,
                         int stream_dtype, int store_kind, int r, int s, int64_t nb,
                         const fc_stream_view* key, const fc_stream_view* value, int64_t n_raw,
                         const float* A, float scale, void* out, int64_t o_sb, int64_t o_sh,
                         int64_t o_st, void* stream) {
  if (!q || !out || !key || !value || B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || Hq % Hkv)
    return FC_ERR_ARG;
  if (nb < 0 || n_raw < 0 || P0 < 0 || r < 1 || r > FC_MAX_BLOCK || s < 1 || s > r)
    return FC_ERR_ARG;
  if (P0 + Sq > nb * r + n_raw) return FC_ERR_ARG;  // every query is a cached token
  if (q_dtype != FC_F16 && q_dtype != FC_BF16) return FC_ERR_UNSUPPORTED;
  if (!(D == 64 || D == 128 || D == 256) || !(s == 1 || s == 2 || s == 4))
    return FC_ERR_UNSUPPORTED;
  if (stream_dtype != FC_F16 && stream_dtype != FC_BF16 && stream_dtype != FC_F32)
    return FC_ERR_ARG;
  if (store_kind != FC_STORE_JPEG_I8 && store_kind != FC_STORE_JPEG_I8G) return FC_ERR_ARG;
  const bool grouped = store_kind == FC_STORE_JPEG_I8G;
  if (nb > 0 && (!A || !key->rows || !value->rows || !key->scales || !value->scales ||
                 nb > key->cap || nb > value->cap))
    return FC_ERR_ARG;
  if (n_raw > 0 && (!key->raw || !value->raw)) return FC_ERR_ARG;
  const auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  if (!al16(q) || q_sb % 8 || q_sh % 8 || q_st % 8 || !al16(key->rows) || !al16(value->rows))
    return FC_ERR_UNSUPPORTED;
  // per-32 scales are read in 8 / 16-byte pieces per row
  if (grouped && nb > 0 && (!al16(key->scales) || !al16(value->scales))) return FC_ERR_UNSUPPORTED;
  const int64_t G = Hq / Hkv;
  PrefillArgs a{};
  a.q = q;
  a.q_dtype = q_dtype;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.q_st = q_st;
  a.Sq = Sq;
  a.P0 = P0;
  a.kcodes = static_cast<const int8_t*>(key->rows);
  a.kscales = key->scales;
  a.vcodes = static_cast<const int8_t*>(value->rows);
  a.vscales = value->scales;
  a.kcap = key->cap;
  a.vcap = value->cap;
  a.A = A;
  a.Hkv = Hkv;
  a.G = G;
  a.nb = nb;
  a.r = r;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.kraw = key->raw;
  a.vraw = value->raw;
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
  a.o_st = o_st;
  // a wavefront's 16 queries: the largest power-of-two head count <= 16
  // that divides G, times 16 / that many consecutive tokens
  int gq = 1;
  while (gq < 16 && G % (2 * gq) == 0) gq *= 2;
  a.gq = gq;
  a.tq = 16 / gq;
  a.hgroups = G / gq;
  a.ntiles = (Sq + 4 * a.tq - 1) / (4 * a.tq);
  const int64_t blocks = a.ntiles * a.hgroups * Hkv * B;
  if (blocks > 0x7fffffff) return FC_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const int dk = (int)(D / 32);
  const unsigned nblocks = (unsigned)blocks;
  int rc;
  // 4 stored rows per block of 4, 8 or 16 tokens: the softmax on the
  // matrix cores (one 4x4 product per block); with one scale per row, D =
  // 64 / 128 and blocks of 4 or 8 tokens the workgroup shares each pass
  // through LDS (at 16 tokens its 3-wavefront register budget spills and
  // the register-resident pass is faster: 1326 vs 1542 us at C5's shape)
  const bool wg = s == 4 && !grouped && (D == 64 || D == 128) && (r == 4 || r == 8) && n_raw < r;
  if (wg && r == 8)
    rc = launch_prefill_wg<8>(a, dk, q_dtype, stream_dtype, nblocks, st);
  else if (wg && r == 4)
    rc = launch_prefill_wg<4>(a, dk, q_dtype, stream_dtype, nblocks, st);
  else if (s == 4 && r == 8)
    rc = launch_prefill<4, 8>(a, dk, q_dtype, stream_dtype, grouped, nblocks, st);
  else if (s == 4 && r == 4)
    rc = launch_prefill<4, 4>(a, dk, q_dtype, stream_dtype, grouped, nblocks, st);
  else if (s == 4 && r == 16)
    rc = launch_prefill<4, 16>(a, dk, q_dtype, stream_dtype, grouped, nblocks, st);
  else
    rc = prefill_with_int<1, 2, 4>(s, [&](auto sc) {
      return launch_prefill<decltype(sc)::value, 0>(a, dk, q_dtype, stream_dtype, grouped,
                                                     nblocks, st);
    });
  if (rc != FC_OK) return rc;
  return check_launch();
}

}  // extern "C"
