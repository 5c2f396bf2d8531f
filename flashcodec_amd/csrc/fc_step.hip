// Fused decode step of one attention layer on a codec KV cache (gfx950).
//
// One call per layer and step: the new key and value tokens are written
// into their streams' tail buffers (one launch for both streams), a tail
// that completes a block is archived with the archive kernels of
// fc_codec.hip, and the decode attention of fc_attention.hip /
// fc_attn_mfma.hip runs over the archive plus the tail.  The reference does
// the same work as two _CodecStream.append calls (cat, archive, contiguous
// copy) and a codec_decode_attention call (flashcodec/cache.py:143-159,
// flashcodec/attention.py:64-140, driven by
// flashcodec/patch_attention.py:95-98); here the host crosses into the
// library once.
#include <hip/hip_runtime.h>

#include "fc_attn_internal.h"
#include "fc_common.h"

namespace fc {

constexpr int kTailThreads = 64;

// fc_last_step_single_launch: how the calling thread's last step ran
thread_local int g_last_step_single = -1;

struct TailArgs {
  const void* tok[2];  // new token of the key / value stream, (B, H, 1, D)
  int64_t tsb[2], tsh[2];
  void* tail[2];  // (B, H, r, D) contiguous tail buffers
  int64_t H, D, r, t;
  const int64_t* state;  // device (n_blocks, n_tail): t = state[1] (or NULL)
};

// tail[s][b][h][t][:] = tok[s][b][h][:]; blockIdx.x = b * H + h,
// blockIdx.y = stream (0: key, 1: value).  T is a storage word of the
// element size (the copy moves bits).
template <typename T>
__global__ __launch_bounds__(kTailThreads) void tail_append_kernel(TailArgs a) {
  const int s = blockIdx.y;
  const int64_t bh = blockIdx.x;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int64_t t = a.state ? a.state[1] : a.t;
  if (t < 0 || t >= a.r) return;  // a tail row exists only for 0 <= t < r
  const T* src = static_cast<const T*>(a.tok[s]) + b * a.tsb[s] + h * a.tsh[s];
  T* dst = static_cast<T*>(a.tail[s]) + (bh * a.r + t) * a.D;
  for (int64_t d = threadIdx.x; d < a.D; d += kTailThreads) dst[d] = src[d];
}

// state = (n_blocks, n_tail, overflow) after the step's token: one lane per
// word, so the update goes out as ordinary vector stores.  A block that
// completes past the archives' capacity `cap` was not written by the gated
// archive kernels (and the attention reads at most `cap` blocks): the
// overflow word records it, sticky, for the host to check.
__global__ void state_advance_kernel(int64_t* state, int64_t r, int64_t cap) {
  const int i = threadIdx.x;
  if (i >= 3) return;
  const int64_t nb = state[0], t = state[1] + 1;
  const bool full = t == r;
  const bool over = full && nb + 1 > cap;
  const int64_t v[3] = {full ? nb + 1 : nb, full ? 0 : t, (state[2] != 0 || over) ? 1 : 0};
  state[i] = v[i];
}

// The whole step as one launch of the matrix-core decode attention: split
// 0's workgroups append the tokens to the tails (or archive the block they
// complete, attending it from its fresh codes) before their passes over the
// blocks already archived; with a device state the launch's last workgroup
// advances it.  FC_ERR_UNSUPPORTED when the step's shape does not allow it
// (then the step takes the multi-launch path).
static int step_single_launch(const fc_step_args* a, const int64_t* state) {
  const bool grouped = a->store_kind == FC_STORE_JPEG_I8G;
  const bool fp = a->store_kind == FC_STORE_JPEG_FP;  // fp16 / bf16 coefficient rows
  const bool png = a->store_kind == FC_STORE_PNG;     // anchors and fp32 deltas
  const bool pk = a->store_kind == FC_STORE_PNG_PACKED;  // anchors, kept values, masks
  // (fp32 queries: int8 archives; fp coefficient rows need queries in their
  // own dtype, which split_fpj_mfma_supported checks)
  if ((a->store_kind != FC_STORE_JPEG_I8 && !grouped && !fp && !png && !pk) ||
      (!fp && !png && !pk && a->quant_bits != 8) || !mfma_split_allowed())
    return FC_ERR_UNSUPPORTED;
  // (fp32 coefficient archives run on the png pass: its step holds blocks of
  // up to 16 tokens in LDS)
  if (fp && a->stream_dtype == FC_F32 && a->r > 16) return FC_ERR_UNSUPPORTED;
  const int64_t B = a->B, Hq = a->Hq, Hkv = a->Hkv, D = a->D;
  const int r = a->r;
  const int64_t G = Hq / Hkv;
  const int64_t nb = a->n_blocks;  // host counters: blocks before the step; state: split hint
  if (nb < 1) return FC_ERR_UNSUPPORTED;
  const fc_step_stream* st[2] = {&a->key, &a->value};
  fc_stream_view v[2]{};
  for (int i = 0; i < 2; ++i) {
    v[i].rows = st[i]->rows;
    v[i].scales = st[i]->scales;
    v[i].anchors = png || pk ? st[i]->anchors : nullptr;
    v[i].masks = pk ? st[i]->masks : nullptr;
    v[i].cap = st[i]->cap;
    v[i].raw = st[i]->tail;
    v[i].raw_sb = Hkv * r * D;
    v[i].raw_sh = (int64_t)r * D;
    v[i].raw_st = D;
  }
  if (pk ? !split_pngpk_supported(a->q, a->q_dtype, a->q_sb, a->q_sh, D, r, a->keep_m,
                                  a->stream_dtype, &v[0], &v[1])
      : png ? !split_png_mfma_supported(a->q, a->q_dtype, a->q_sb, a->q_sh, D, r,
                                        a->stream_dtype, &v[0], &v[1])
      : fp ? !split_fpj_mfma_supported(a->q, a->q_dtype, a->q_sb, a->q_sh, D, a->s,
                                       a->stream_dtype, &v[0], &v[1])
           : !i8_mfma_takes(a->store_kind, a->q, a->q_dtype, a->q_sb, a->q_sh, D, a->s, &v[0],
                            &v[1]))
    return FC_ERR_UNSUPPORTED;
  const int64_t mstride = counter_stride(2 * B * Hkv * ((G + 15) / 16));
  if (mstride == 0) return FC_ERR_UNSUPPORTED;
  const int n_splits = fc_attention_splits(a->store_kind, a->stream_dtype, a->q_dtype, a->s, nb,
                                           B, Hkv, G, D, a->n_cu);
  // (the png passes hold the step's rows in LDS buffers of their own)
  if (n_splits < 1 ||
      (pk    ? n_splits > kFuseMaxSplitsPk
       : png ? !split_i8_mfma_fusable(n_splits)
             : !step_i8_mfma_supported(a->stream_dtype, r, D, n_splits)))
    return FC_ERR_UNSUPPORTED;
  if (!a->workspace || fc_attention_workspace_bytes(B, Hq, D, n_splits) > a->workspace_bytes)
    return FC_ERR_ARG;
  const WsLayout ws = ws_layout(a->workspace, B, Hq, n_splits);
  MfmaFuse fz{};
  fz.raw_dtype = a->stream_dtype;
  fz.n_raw = 0;
  fz.out = a->out;
  fz.o_sb = a->o_sb;
  fz.o_sh = a->o_sh;
  fz.state = state;
  fz.step = true;
  fz.ktok = a->key.token;
  fz.vtok = a->value.token;
  fz.kt_sb = a->key.tok_sb;
  fz.kt_sh = a->key.tok_sh;
  fz.vt_sb = a->value.tok_sb;
  fz.vt_sh = a->value.tok_sh;
  fz.basis = a->basis;
  fz.step_t = a->n_tail;
  fz.step_nb = a->n_blocks;
  fz.done = ws.done;
  fz.keep_m = a->keep_m;
  if (pk)
    return launch_split_pngpk(a->q, a->q_dtype, a->q_sb, a->q_sh, B, Hq, Hkv, D, r, a->keep_m,
                              a->stream_dtype, nb, &v[0], &v[1], a->scale * 1.4426950408889634f,
                              ws.pm, ws.pl, ws.pacc, n_splits, ws.counters, kCounterWords,
                              mstride, &fz, state, (hipStream_t)a->stream);
  if (png)
    return launch_split_png_mfma(a->q, a->q_dtype, a->q_sb, a->q_sh, B, Hq, Hkv, D, r, nb,
                                 &v[0], &v[1],
                                 a->scale * 1.4426950408889634f, ws.pm, ws.pl, ws.pacc, n_splits,
                                 ws.counters, kCounterWords, mstride, &fz, state,
                                 (hipStream_t)a->stream);
  if (fp)
    return launch_split_fpj_mfma(a->q, a->q_dtype, a->q_sb, a->q_sh, B, Hq, Hkv, D, r, a->s, nb,
                                 &v[0], &v[1], a->A, a->scale * 1.4426950408889634f, ws.pm,
                                 ws.pl, ws.pacc, n_splits, ws.counters, kCounterWords, mstride,
                                 &fz, state, (hipStream_t)a->stream);
  return launch_split_i8_mfma(a->q, a->q_dtype, a->q_sb, a->q_sh, B, Hq, Hkv, D, r, a->s, nb,
                              &v[0], &v[1], a->A, a->scale * 1.4426950408889634f, ws.pm, ws.pl,
                              ws.pacc, n_splits, ws.counters, kCounterWords, mstride,
                              &fz, (hipStream_t)a->stream, grouped);
}

// The step with its counters on the device (a->state): every launch reads
// them there, so one captured graph of the step is valid at every step.
static int decode_step_state(const fc_step_args* a) {
  const int kind = a->store_kind;
  if ((kind == FC_STORE_JPEG_I8 || kind == FC_STORE_JPEG_I8G) && a->quant_bits != 8)
    return FC_ERR_ARG;
  if (kind != FC_STORE_JPEG_I8 && kind != FC_STORE_JPEG_FP && kind != FC_STORE_PNG &&
      kind != FC_STORE_JPEG_I8G && kind != FC_STORE_PNG_PACKED)
    return FC_ERR_ARG;
  if (a->n_blocks < 1) return FC_ERR_ARG;  // the archive holds a block before capture
  const int one = step_single_launch(a, a->state);
  if (one != FC_ERR_UNSUPPORTED) {
    if (one == FC_OK) g_last_step_single = 1;
    return one;
  }
  const int64_t B = a->B, Hkv = a->Hkv, D = a->D;
  const int r = a->r;
  hipStream_t stream = (hipStream_t)a->stream;
  const fc_step_stream* st[2] = {&a->key, &a->value};
  TailArgs ta{};
  for (int i = 0; i < 2; ++i) {
    ta.tok[i] = st[i]->token;
    ta.tsb[i] = st[i]->tok_sb;
    ta.tsh[i] = st[i]->tok_sh;
    ta.tail[i] = st[i]->tail;
  }
  ta.H = Hkv;
  ta.D = D;
  ta.r = r;
  ta.t = 0;
  ta.state = a->state;
  const dim3 grid((unsigned)(B * Hkv), 2);
  if (esize_of(a->stream_dtype) == 4)
    tail_append_kernel<uint32_t><<<grid, kTailThreads, 0, stream>>>(ta);
  else
    tail_append_kernel<uint16_t><<<grid, kTailThreads, 0, stream>>>(ta);
  int rc = check_launch();
  if (rc != FC_OK) return rc;
  const int64_t tsb = Hkv * r * D, tsh = (int64_t)r * D;
  for (int i = 0; i < 2; ++i) {
    if (kind == FC_STORE_PNG || kind == FC_STORE_PNG_PACKED)
      rc = png_encode_gated(st[i]->tail, a->stream_dtype, B, Hkv, tsb, tsh, D, D, r, a->keep_m,
                            static_cast<float*>(st[i]->rows), st[i]->anchors, st[i]->cap,
                            a->stream, a->state,
                            kind == FC_STORE_PNG_PACKED ? st[i]->masks : nullptr);
    else
      rc = jpeg_encode_gated(st[i]->tail, a->stream_dtype, B, Hkv, tsb, tsh, D, D, r, a->s,
                             a->basis, st[i]->rows, st[i]->scales, st[i]->cap,
                             kind == FC_STORE_JPEG_FP ? 0 : 8, a->stream, a->state,
                             kind == FC_STORE_JPEG_I8G ? 32 : 0);
    if (rc != FC_OK) return rc;
  }
  fc_stream_view v[2]{};
  for (int i = 0; i < 2; ++i) {
    v[i].rows = st[i]->rows;
    v[i].scales = st[i]->scales;
    v[i].anchors = st[i]->anchors;
    v[i].cap = st[i]->cap;
    v[i].raw = st[i]->tail;
    v[i].raw_sb = tsb;
    v[i].raw_sh = tsh;
    v[i].raw_st = D;
    v[i].masks = st[i]->masks;
  }
  rc = decode_attention_state(a->q, a->q_dtype, a->q_sb, a->q_sh, B, a->Hq, Hkv, D, kind,
                              a->stream_dtype, r, a->s, a->n_blocks, &v[0], &v[1], a->A, a->scale,
                              a->out, a->o_sb, a->o_sh, a->workspace, a->workspace_bytes,
                              a->n_cu, a->state, a->stream);
  if (rc != FC_OK) return rc;
  state_advance_kernel<<<1, 64, 0, stream>>>(const_cast<int64_t*>(a->state), r,
                                             a->key.cap < a->value.cap ? a->key.cap
                                                                       : a->value.cap);
  rc = check_launch();
  if (rc == FC_OK) g_last_step_single = 0;
  return rc;
}

}  // namespace fc

using namespace fc;

extern "C" {

int fc_decode_step(const fc_step_args* a) {
  if (!a) return FC_ERR_ARG;
  const int64_t B = a->B, Hq = a->Hq, Hkv = a->Hkv, D = a->D;
  const int r = a->r;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || Hq % Hkv) return FC_ERR_ARG;
  if (r < 1 || r > FC_MAX_BLOCK || a->n_tail < 0 || a->n_tail >= r || a->n_blocks < 0)
    return FC_ERR_ARG;
  const int es = esize_of(a->stream_dtype);
  if (es == 0 || a->stream_dtype == FC_I8) return FC_ERR_ARG;
  const fc_step_stream* st[2] = {&a->key, &a->value};
  for (const fc_step_stream* x : st)
    if (!x->token || !x->tail || !x->rows) return FC_ERR_ARG;
  if ((a->store_kind == FC_STORE_JPEG_I8 || a->store_kind == FC_STORE_JPEG_I8G) &&
      (!a->key.scales || !a->value.scales))
    return FC_ERR_ARG;
  const bool png = a->store_kind == FC_STORE_PNG || a->store_kind == FC_STORE_PNG_PACKED;
  if (png && (!a->key.anchors || !a->value.anchors)) return FC_ERR_ARG;
  if (a->store_kind == FC_STORE_PNG_PACKED && (!a->key.masks || !a->value.masks))
    return FC_ERR_ARG;
  if (!png && !a->basis) return FC_ERR_ARG;
  if (a->state) return decode_step_state(a);
  const bool completes = a->n_tail + 1 == r;
  if (completes && (a->n_blocks + 1 > a->key.cap || a->n_blocks + 1 > a->value.cap))
    return FC_ERR_ARG;  // the caller grows the archives first
  const int one = step_single_launch(a, nullptr);
  if (one != FC_ERR_UNSUPPORTED) {
    if (one == FC_OK) g_last_step_single = 1;
    return one;
  }
  hipStream_t stream = (hipStream_t)a->stream;

  // 1. the new tokens into the tails
  TailArgs ta{};
  for (int i = 0; i < 2; ++i) {
    ta.tok[i] = st[i]->token;
    ta.tsb[i] = st[i]->tok_sb;
    ta.tsh[i] = st[i]->tok_sh;
    ta.tail[i] = st[i]->tail;
  }
  ta.H = Hkv;
  ta.D = D;
  ta.r = r;
  ta.t = a->n_tail;
  ta.state = nullptr;  // host counters
  const dim3 grid((unsigned)(B * Hkv), 2);
  if (es == 4)
    tail_append_kernel<uint32_t><<<grid, kTailThreads, 0, stream>>>(ta);
  else
    tail_append_kernel<uint16_t><<<grid, kTailThreads, 0, stream>>>(ta);
  int rc = check_launch();
  if (rc != FC_OK) return rc;

  // 2. a completed tail becomes block n_blocks of each archive
  int64_t nb = a->n_blocks, nt = a->n_tail + 1;
  const int64_t tsb = Hkv * r * D, tsh = (int64_t)r * D;
  if (completes) {
    for (int i = 0; i < 2; ++i) {
      const fc_step_stream* x = st[i];
      if (a->store_kind == FC_STORE_PNG_PACKED)
        rc = fc_png_encode_packed(x->tail, a->stream_dtype, B, Hkv, tsb, tsh, D, r, 1, D, r,
                                  a->keep_m, static_cast<float*>(x->rows), x->masks, x->anchors,
                                  x->cap, nb, a->stream);
      else if (a->store_kind == FC_STORE_PNG)
        rc = fc_png_encode(x->tail, a->stream_dtype, B, Hkv, tsb, tsh, D, r, 1, D, r, a->keep_m,
                           static_cast<float*>(x->rows), x->anchors, x->cap, nb, a->stream);
      else if (a->store_kind == FC_STORE_JPEG_I8G)
        rc = fc_jpeg_encode_grouped(x->tail, a->stream_dtype, B, Hkv, tsb, tsh, D, r, 1, D, r,
                                    a->s, a->basis, static_cast<int8_t*>(x->rows), x->scales,
                                    x->cap, nb, 32, a->stream);
      else
        rc = fc_jpeg_encode(x->tail, a->stream_dtype, B, Hkv, tsb, tsh, D, r, 1, D, r, a->s,
                            a->basis, x->rows, x->scales, x->cap, nb, a->quant_bits, a->stream);
      if (rc != FC_OK) return rc;
    }
    ++nb;
    nt = 0;
  }

  // 3. attention over the archive and the tail
  fc_stream_view v[2]{};
  for (int i = 0; i < 2; ++i) {
    v[i].rows = st[i]->rows;
    v[i].scales = st[i]->scales;
    v[i].anchors = st[i]->anchors;
    v[i].cap = st[i]->cap;
    v[i].raw = nt ? st[i]->tail : nullptr;
    v[i].raw_sb = tsb;
    v[i].raw_sh = tsh;
    v[i].raw_st = D;
    v[i].masks = st[i]->masks;
  }
  int n_splits = 0;
  if (nb > 0) {
    n_splits = fc_attention_splits(a->store_kind, a->stream_dtype, a->q_dtype, a->s, nb, B, Hkv,
                                   Hq / Hkv, D, a->n_cu);
    if (!a->workspace || fc_attention_workspace_bytes(B, Hq, D, n_splits) > a->workspace_bytes)
      return FC_ERR_ARG;
  }
  rc = fc_decode_attention(a->q, a->q_dtype, a->q_sb, a->q_sh, B, Hq, Hkv, D, a->store_kind,
                           a->stream_dtype, r, a->s, nb, &v[0], &v[1], nt, a->A, a->scale,
                           a->out, a->o_sb, a->o_sh, a->workspace, n_splits, a->stream);
  if (rc == FC_OK) g_last_step_single = 0;
  return rc;
}

int fc_last_step_single_launch(void) { return g_last_step_single; }

}  // extern "C"
