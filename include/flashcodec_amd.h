/*
 * flashcodec_amd — C ABI of the MI355X (gfx950) KV-codec hot path.
 *
 * Every entry point is stateless apart from the basis/launch configuration
 * the caller passes in, takes raw device pointers, element strides and
 * sizes, enqueues its kernels on the given HIP stream (`stream` is a
 * hipStream_t; NULL = the default stream) and returns an int status:
 * FC_OK (0) or one of the negative FC_ERR_* codes below.  Nothing here
 * allocates device memory, throws or synchronises a stream.
 *
 * Layout conventions (all element strides, innermost dimension D is
 * contiguous, i.e. stride 1):
 *   sequence input  x[b][h][t][d]      at x + b*x_sb + h*x_sh + t*x_ss + d
 *   coefficient store   (B*H, cap, k, D)   contiguous (jpeg)
 *   scale store         (B*H, cap, k)      contiguous fp32 (jpeg int8)
 *   delta store         (B*H, cap, r-1, D) contiguous fp32 (png)
 *   anchor store        (B*H, cap, D)      contiguous, stream dtype (png)
 * which are exactly the reference buffers `_coeffs`, `_scales`, `_deltas`,
 * `_anchors` of flashcodec/cache.py:94-104 (the trailing size-1 axis of
 * `_scales` is dropped because it has no extent).
 *
 * dtype codes: FC_F32, FC_F16, FC_BF16 for floating tensors, FC_I8 for int8.
 */
#ifndef FLASHCODEC_AMD_H
#define FLASHCODEC_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FC_F32 = 0,
  FC_F16 = 1,
  FC_BF16 = 2,
  FC_I8 = 3
};

enum {
  FC_OK = 0,
  FC_ERR_ARG = -1,         /* invalid argument (shape, dtype, pointer)       */
  FC_ERR_UNSUPPORTED = -2, /* valid but outside this build's kernel limits   */
  FC_ERR_HIP = -3,         /* a HIP runtime call failed (see fc_last_hip_error) */
  FC_ERR_SCRATCH = -5      /* the call needs more scratch than the static array of
                              fc_decode_attention_noalloc holds */
};

/* Limits of the kernels in this library. */
#define FC_MAX_BLOCK 64    /* block size r (tokens per archived block)    */
#define FC_MAX_HEAD_DIM 512

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int fc_version(void);

/* Human-readable text for a status code. */
const char* fc_status_string(int status);

/* hipError_t of the last failing HIP call in this thread (0 if none). */
int fc_last_hip_error(void);

/*
 * JPEG-mode archive: blockwise orthonormal DCT-II along the token axis, keep
 * the lowest k frequencies, optionally quantise them to int8 with one fp32
 * scale per (block, frequency).
 *
 * Encodes m blocks of r tokens for each of the B*H sequences of x (tokens
 * t >= s_valid are treated as zeros, which is the reference's zero padding)
 * and writes them at block offset n0 of a store with capacity `cap` blocks.
 * quant_bits == 0: `coeffs` has x's dtype.  quant_bits == 8: `coeffs` is
 * int8 and `scales` receives the fp32 scales.  `basis` is the k x r fp32
 * DCT-II matrix (row-major, device memory).
 *
 * Replaces dct_compress + quantize_coeffs + the in-place slice copies of
 * _CodecStream._archive (flashcodec/codecs/jpeg.py:55-67, 85-100;
 * flashcodec/cache.py:123-136), and dct_compress alone when quant_bits == 0.
 */
int fc_jpeg_encode(const void* x, int x_dtype, int64_t B, int64_t H,
                   int64_t x_sb, int64_t x_sh, int64_t x_ss, int64_t s_valid,
                   int64_t m, int64_t D, int r, int k, const float* basis,
                   void* coeffs, float* scales, int64_t cap, int64_t n0,
                   int quant_bits, void* stream);

/*
 * JPEG-mode reconstruction of blocks [a, a+nblk) of every sequence of a
 * store (dtype store_dtype: FC_I8 with `scales`, or a float dtype with
 * scales == NULL) into out[b][h][t][d] (dtype out_dtype, element strides
 * o_sb, o_sh, o_ss), token t = block*r + row.  Tokens t >= out_len are not
 * written (the reference's out_len trim).
 *
 * Replaces dequantize_coeffs + dct_decompress and the copy into the
 * memoised view of _CodecStream._decode_pending
 * (flashcodec/codecs/jpeg.py:70-82, 103-105; flashcodec/cache.py:182-192).
 */
int fc_jpeg_decode(const void* store, int store_dtype, const float* scales,
                   int64_t B, int64_t H, int64_t cap, int64_t a, int64_t nblk,
                   int64_t D, int r, int k, const float* basis, void* out,
                   int out_dtype, int64_t o_sb, int64_t o_sh, int64_t o_ss,
                   int64_t out_len, void* stream);

/*
 * JPEG-mode int8 archive with one fp32 scale per `group` features of each
 * (block, frequency) row instead of one per row: the per-32 absmax
 * coefficient quantizer (group must be 32, D a multiple of it).  Same
 * transform, rounding and code rule as fc_jpeg_encode with quant_bits 8;
 * the scale of features [32 g, 32 g + 32) of row j of block n is
 * scales[((b*H + h)*cap + n)*k + j][g] of a (B*H, cap, k, D/32) fp32 store.
 * No reference counterpart as a library format: flashcodec documents it as
 * the quantizer that makes the coefficient archive competitive
 * (README.md:487-494) without shipping it.
 */
int fc_jpeg_encode_grouped(const void* x, int x_dtype, int64_t B, int64_t H,
                           int64_t x_sb, int64_t x_sh, int64_t x_ss,
                           int64_t s_valid, int64_t m, int64_t D, int r, int k,
                           const float* basis, int8_t* codes, float* scales,
                           int64_t cap, int64_t n0, int group, void* stream);

/*
 * Reconstruction of blocks [a, a+nblk) of a per-`group` scaled int8 store
 * (fc_jpeg_encode_grouped) into out, as fc_jpeg_decode.
 */
int fc_jpeg_decode_grouped(const int8_t* codes, const float* scales,
                           int64_t B, int64_t H, int64_t cap, int64_t a,
                           int64_t nblk, int64_t D, int r, int k, int group,
                           const float* basis, void* out, int out_dtype,
                           int64_t o_sb, int64_t o_sh, int64_t o_ss,
                           int64_t out_len, void* stream);

/*
 * Symmetric int8 quantisation of coefficient rows: n_rows rows of D values
 * (dtype c_dtype, row stride c_rs elements) -> int8 codes (contiguous
 * rows of D) and one fp32 scale per row.
 * Replaces quantize_coeffs (flashcodec/codecs/jpeg.py:85-100).
 */
int fc_quantize_rows(const void* c, int c_dtype, int64_t n_rows, int64_t c_rs,
                     int64_t D, int8_t* codes, float* scales, void* stream);

/*
 * Dequantisation q.to(dtype) * scale.to(dtype): n_rows rows of D int8
 * codes with one fp32 scale per row -> out (dtype out_dtype, contiguous).
 * Replaces dequantize_coeffs (flashcodec/codecs/jpeg.py:103-105).
 */
int fc_dequantize_rows(const int8_t* codes, const float* scales, int64_t n_rows,
                       int64_t D, void* out, int out_dtype, void* stream);

/*
 * PNG-mode archive: per block an anchor (token 0, stored in x's dtype) and
 * r-1 fp32 first-order deltas; when 0 < keep_m < r-1 only the keep_m
 * largest |delta| per (block, feature) survive, the others are multiplied
 * by 0 (sign kept).  Ties at the cut are resolved exactly as the
 * reference's CPU topk resolves them.
 * Replaces png_filter + the slice copies of _CodecStream._archive
 * (flashcodec/codecs/png.py:36-60; flashcodec/cache.py:137-140).
 */
int fc_png_encode(const void* x, int x_dtype, int64_t B, int64_t H,
                  int64_t x_sb, int64_t x_sh, int64_t x_ss, int64_t s_valid,
                  int64_t m, int64_t D, int r, int keep_m, float* deltas,
                  void* anchors, int64_t cap, int64_t n0, void* stream);

/*
 * PNG-mode reconstruction (anchor + running sum of deltas) of blocks
 * [a, a+nblk) into out (anchor dtype), as fc_jpeg_decode.
 * Replaces png_reconstruct + the view copy (flashcodec/codecs/png.py:63-74;
 * flashcodec/cache.py:189-192).
 */
int fc_png_decode(const float* deltas, const void* anchors, int anchor_dtype,
                  int64_t B, int64_t H, int64_t cap, int64_t a, int64_t nblk,
                  int64_t D, int r, void* out, int64_t o_sb, int64_t o_sh,
                  int64_t o_ss, int64_t out_len, void* stream);

/*
 * Host-side (CPU) evaluation of the exact tie-aware Top-M rule the png
 * kernel applies to one (block, feature) column: bit i of the result is set
 * when step i of the n (<= 63) deltas survives keep_m.  Same source as the
 * kernel's tie path; exported so the selection can be checked without a
 * GPU.  Restates the topk selection of flashcodec/codecs/png.py:54-58.
 */
uint64_t fc_png_topm_mask_host(const float* delta, int n, int keep_m);

/*
 * Packed png archive (no reference code: the fixed-rate, block-addressable
 * form of png_filter's Top-M output that the reference leaves to a future
 * entropy coder, flashcodec/README.md:580-583).  Per (block, feature) the
 * keep_m deltas png_filter keeps (flashcodec/codecs/png.py:36-60), in step
 * order, as fp32 values `vals` (B*H, cap, keep_m, D), and one mask word
 * (B*H, cap, D): bit i set = step i (delta i, token i + 1) kept; bit 16 + i
 * = the sign bit of step i when it is not kept (png_filter stores a pruned
 * delta as delta * 0, a signed zero).  Kept steps are the non-zero deltas
 * of the Top-M selection, then the lowest-index zero steps until keep_m
 * (a kept and a pruned zero unpack to the same bits).  Unpacking gives
 * png_filter's dense deltas bit for bit (finite inputs: a pruned delta that
 * is not finite, which png_filter turns into NaN, unpacks as a signed
 * zero).  Anchors as the dense archive.  2 <= r <= 16, 1 <= keep_m <= r - 1.
 * Same arguments as fc_png_encode with the packed stores in place of the
 * delta store.
 */
int fc_png_encode_packed(const void* x, int x_dtype, int64_t B, int64_t H,
                         int64_t x_sb, int64_t x_sh, int64_t x_ss,
                         int64_t s_valid, int64_t m, int64_t D, int r,
                         int keep_m, float* vals, uint32_t* masks,
                         void* anchors, int64_t cap, int64_t n0,
                         void* stream);

/*
 * png_reconstruct of blocks [a, a + nblk) of a packed archive, as
 * fc_png_decode (fp64 running sum of the unpacked deltas, bit for bit the
 * dense archive's reconstruction).  Replaces png_reconstruct
 * (flashcodec/codecs/png.py:63-74) for packed stores.
 */
int fc_png_decode_packed(const float* vals, const uint32_t* masks,
                         const void* anchors, int anchor_dtype, int64_t B,
                         int64_t H, int64_t cap, int64_t a, int64_t nblk,
                         int64_t D, int r, int keep_m, void* out, int64_t o_sb,
                         int64_t o_sh, int64_t o_ss, int64_t out_len,
                         void* stream);

/*
 * Dense deltas (B*H, d_cap, r-1, D) fp32 at blocks [a, a + nblk) from a
 * packed archive: png_filter's delta output bit for bit (the layout of
 * fc_png_encode's delta store).  No reference counterpart (the reference
 * stores only the dense form); for callers converting packed archives.
 */
int fc_png_unpack(const float* vals, const uint32_t* masks, int64_t B, int64_t H,
                  int64_t cap, int64_t a, int64_t nblk, int64_t D, int r,
                  int keep_m, float* deltas, int64_t d_cap, void* stream);

/* Archive kind of a stream for fc_decode_attention. */
enum {
  FC_STORE_JPEG_I8 = 0,  /* rows: int8 coeffs x fp32 scale, s = k      */
  FC_STORE_JPEG_FP = 1,  /* rows: coeffs in the stream dtype, s = k    */
  FC_STORE_PNG = 2,      /* rows: anchor (stream dtype) + r-1 fp32 deltas, s = r */
  FC_STORE_JPEG_I8G = 3, /* rows: int8 coeffs x one fp32 scale per 32 features
                            (scales (B*H, cap, k, D/32)), s = k */
  FC_STORE_PNG_PACKED = 4 /* rows: anchor (stream dtype) + the packed Top-M
                            deltas of fc_png_encode_packed (vals (B*H, cap,
                            keep_m, D) fp32 in `rows`, mask words (B*H, cap,
                            D) in `masks`), s = keep_m */
};

/* One KV stream as seen by the decode attention. */
typedef struct fc_stream_view {
  const void* rows;      /* jpeg: coeffs (B*H, cap, k, D); png: deltas (B*H, cap, r-1, D) */
  const float* scales;   /* jpeg int8: (B*H, cap, k); per-32: (B*H, cap, k, D/32); else NULL */
  const void* anchors;   /* png: (B*H, cap, D); else NULL */
  int64_t cap;           /* capacity of the store in blocks */
  const void* raw;       /* raw tail (B, H, n_raw, D) in the stream dtype, or NULL */
  int64_t raw_sb, raw_sh, raw_st; /* element strides of the raw tail */
  const uint32_t* masks; /* packed png: mask words (B*H, cap, D); else NULL */
} fc_stream_view;

/*
 * Bytes of device workspace fc_decode_attention needs for B*Hq query heads,
 * head size D and n_splits splits (0 when n_splits == 0).  The workspace
 * must be zero-filled before its first use: it starts with arrival counters
 * that every call returns to zero, so one workspace (of the largest size
 * needed) serves any number of calls ordered on one stream.  Calls that may
 * run concurrently need separate workspaces.
 */
int64_t fc_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t D,
                                     int n_splits);

/*
 * Split count the library would choose for nb archived blocks spread over
 * B*Hkv kv heads with G query heads each on a device with n_cu compute
 * units (>= 1 whenever nb > 0; 0 when nb == 0).
 */
int fc_attention_default_splits(int64_t nb, int64_t B, int64_t Hkv, int64_t G,
                                 int n_cu);

/*
 * Split count for a fc_decode_attention call over stores of `store_kind`
 * (stream dtype, query dtype, s stored rows per block, head size D): one
 * round of workgroups of the split pass that will run — the matrix-core
 * passes for int8 jpeg archives (one scale per row or per 32 features) with
 * fp16/bf16/fp32 queries, for fp16/bf16/fp32 coefficient archives queried
 * in their dtype at D = 64/128, and for png (fp32/fp16/bf16 streams
 * queried in their dtype) at r = 4/8/16 (two workgroups per compute unit,
 * but at least one pass per wavefront and at most max(16, passes / 10)
 * splits), the packed png pass, otherwise the vector-ALU pass at the
 * occupancy it reaches on the current device.  0 when nb == 0.
 * Replaces the split heuristic ns = max(1, min(32, ceil(n / 64))) of
 * flashcodec/triton_attention.py:191.
 */
int fc_attention_splits(int store_kind, int stream_dtype, int q_dtype, int s,
                        int64_t nb, int64_t B, int64_t Hkv, int64_t G, int64_t D,
                        int n_cu);

/*
 * Materialisation-free decode attention of one query token per sequence:
 *   q (B, Hq, 1, D) in q_dtype with element strides q_sb, q_sh
 *   K/V archives of nb blocks with s stored rows each, synthesis matrix
 *   A (r x s, fp32 row-major, device) and raw tails of n_raw tokens,
 *   out (B, Hq, 1, D) in q_dtype with element strides o_sb, o_sh.
 * Query head hq reads kv head hq / G (G = Hq / Hkv).  Scores are
 * scale * q . (A S)[p]; softmax in fp32; output (p A) S + p_raw V_raw.
 * Every query head reads its kv head's rows once per group of up to 16
 * query heads.  `workspace` must hold fc_attention_workspace_bytes(...) and
 * follow its zero-fill rule.  With archived blocks the call is normally
 * one launch: the split pass's last workgroup per (batch, kv head, head
 * group) merges the partials and the raw tail into `out`.  Shapes beyond
 * the workspace's counters or the fused merge's split limit run the merge
 * pass as a second launch; a tail-only call (nb == 0) is one merge launch.
 *
 * Replaces codec_decode_attention's jpeg Triton path and its png / torch
 * path (flashcodec/attention.py:64-140;
 * flashcodec/triton_attention.py:34-222).
 */
int fc_decode_attention(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                        int store_kind, int stream_dtype, int r, int s,
                        int64_t nb, const fc_stream_view* key,
                        const fc_stream_view* value, int64_t n_raw,
                        const float* A, float scale, void* out, int64_t o_sb,
                        int64_t o_sh, void* workspace, int n_splits,
                        void* stream);

/*
 * The two passes of fc_decode_attention as separate entry points (same
 * arguments): _split enqueues the pass over the archived blocks that fills
 * the workspace partials, _merge the pass that combines them with the raw
 * tail into `out`.  Calling _split then _merge on one stream equals
 * fc_decode_attention; callers use them to time or overlap the passes.
 * No reference counterpart (the Triton path launches its split and combine
 * kernels back to back, flashcodec/triton_attention.py:199-221).
 */
int fc_decode_attention_split(const void* q, int q_dtype, int64_t q_sb,
                              int64_t q_sh, int64_t B, int64_t Hq, int64_t Hkv,
                              int64_t D, int store_kind, int stream_dtype,
                              int r, int s, int64_t nb,
                              const fc_stream_view* key,
                              const fc_stream_view* value, int64_t n_raw,
                              const float* A, float scale, void* out,
                              int64_t o_sb, int64_t o_sh, void* workspace,
                              int n_splits, void* stream);
int fc_decode_attention_merge(const void* q, int q_dtype, int64_t q_sb,
                              int64_t q_sh, int64_t B, int64_t Hq, int64_t Hkv,
                              int64_t D, int store_kind, int stream_dtype,
                              int r, int s, int64_t nb,
                              const fc_stream_view* key,
                              const fc_stream_view* value, int64_t n_raw,
                              const float* A, float scale, void* out,
                              int64_t o_sb, int64_t o_sh, void* workspace,
                              int n_splits, void* stream);

/*
 * Gather of per-(row, head) byte segments on the device, for batch-major
 * buffers (every archive buffer, tail buffer and reconstruction of a
 * stream): for b in [0, B_out) and h in [0, H),
 *   dst[b*d_sb + h*d_sh + i] = src[idx[b]*s_sb + h*s_sh + i],  i in [0, len)
 * with strides and len in bytes, idx B_out int64 device indices into src's
 * B_src rows (NULL: idx[b] = b).  dst == src (same strides, B_out == B_src)
 * gathers in place: every source segment of a column is read before any
 * destination in it is written, so any idx (a permutation, repeats) is
 * valid; other overlaps are not allowed.  Indices outside [0, B_src) leave
 * their destination segment unwritten.  No allocation, no host
 * synchronisation: a captured HIP graph can replay it with new indices.
 * FC_ERR_UNSUPPORTED when an in-place gather has more than 2048 rows.
 * Replaces the index_select gathers of _CodecStream.select_batch and the
 * verbatim prefix copy of _CodecStream._grow (flashcodec/cache.py:106-121,
 * 259-301).
 */
int fc_gather_segments(void* dst, int64_t d_sb, int64_t d_sh, const void* src,
                       int64_t s_sb, int64_t s_sh, const int64_t* idx,
                       int64_t B_out, int64_t B_src, int64_t H, int64_t len,
                       void* stream);

/* Bytes of the static scratch array of fc_decode_attention_noalloc (one per
 * GPU, held until the process ends). */
#define FC_NOALLOC_SCRATCH_BYTES (16 << 20)

/*
 * fc_decode_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the workspace is a static device
 * array of this library, FC_NOALLOC_SCRATCH_BYTES per GPU, looked up on the
 * first call on a device; nothing is allocated, ever.  Arguments, results
 * and split count rules as fc_decode_attention (the caller still passes q,
 * the stores and out).  A call whose fc_attention_workspace_bytes(B, Hq, D,
 * n_splits) exceeds FC_NOALLOC_SCRATCH_BYTES returns FC_ERR_SCRATCH.  All
 * calls on one GPU share the array (the last call's contents stay in it;
 * every call returns its counters to zero): calls that overlap on one GPU
 * (several streams or threads) race and must not be issued.
 * No counterpart in the reference; it exists for the callers that cannot
 * allocate.
 */
int fc_decode_attention_noalloc(const void* q, int q_dtype, int64_t q_sb,
                                int64_t q_sh, int64_t B, int64_t Hq,
                                int64_t Hkv, int64_t D, int store_kind,
                                int stream_dtype, int r, int s, int64_t nb,
                                const fc_stream_view* key,
                                const fc_stream_view* value, int64_t n_raw,
                                const float* A, float scale, void* out,
                                int64_t o_sb, int64_t o_sh, int n_splits,
                                void* stream);

/* Split pass selection for fc_decode_attention / fc_decode_step. */
enum {
  FC_PASS_AUTO = 0,   /* matrix-core passes for the archives they support,
                         its passes handed out by a queue (outputs may differ in
                         the last bits between calls: fp32 summation order) */
  FC_PASS_VECTOR = 1, /* vector-ALU pass for every store (A/B measurements) */
  FC_PASS_STATIC = 2  /* as FC_PASS_AUTO with a fixed pass order: bitwise
                         reproducible outputs, at some cost in balance */
};

/*
 * Process-wide split pass selection (FC_PASS_*; FC_ERR_ARG otherwise) and
 * its current value.  The initial value comes from the environment when
 * the library is loaded (FLASHCODEC_AMD_ATTN=valu selects FC_PASS_VECTOR);
 * calls never read the environment.  Changing it while calls are in flight
 * on other threads is a race.  No reference counterpart (the reference picks
 * Triton or torch per call through `impl`, flashcodec/attention.py:91-99).
 */
int fc_set_attention_pass(int pass);
int fc_get_attention_pass(void);

/*
 * Causal prefill attention on int8 jpeg archives without the reconstructed
 * view: the Sq query tokens q (B, Hq, Sq, D) (q_dtype FC_F16 / FC_BF16,
 * element strides q_sb, q_sh, q_st) sit at positions P0 .. P0+Sq-1 of the
 * streams (P0 + Sq <= nb * r + n_raw), and query token i attends every
 * cached token at a position <= P0 + i: archived blocks through their
 * stored rows (codes x scales: store_kind FC_STORE_JPEG_I8, one scale per
 * row, or FC_STORE_JPEG_I8G, one per 32 features, whose scale stores must
 * be 16-byte aligned; synthesis matrix A r x s) in the coefficient
 * domain, raw-tail tokens at full precision.  Softmax in fp32; out
 * (B, Hq, Sq, D) in q_dtype, strides o_sb, o_sh, o_st.  GQA as
 * fc_decode_attention.  Supports D in {64, 128, 256} and s in {1, 2, 4}
 * (FC_ERR_UNSUPPORTED otherwise), 16-byte aligned q and stores.  One
 * launch, no workspace.
 * Replaces the reference's prefill attention on the materialised view
 * (the read() view SDPA attends, flashcodec/cache.py:203-220 through
 * flashcodec/patch_attention.py:58-61; flashcodec/attention.py:24-26 names
 * the gap).
 */
int fc_prefill_attention(const void* q, int q_dtype, int64_t q_sb,
                         int64_t q_sh, int64_t q_st, int64_t B, int64_t Hq,
                         int64_t Hkv, int64_t Sq, int64_t D, int64_t P0,
                         int stream_dtype, int store_kind, int r, int s,
                         int64_t nb, const fc_stream_view* key,
                         const fc_stream_view* value, int64_t n_raw,
                         const float* A, float scale, void* out,
                         int64_t o_sb, int64_t o_sh, int64_t o_st,
                         void* stream);

/*
 * One stream (key or value) of a layer for fc_decode_step: its archive
 * buffers (as fc_stream_view), its (B, H, r, D) contiguous tail buffer in
 * the stream dtype (the raw tail is its first n_tail token rows), and the
 * step's new token (B, H, 1, D) with element strides tok_sb, tok_sh.
 */
typedef struct fc_step_stream {
  void* rows;            /* jpeg: (B*H, cap, s, D) codes / coefficients; png: deltas */
  float* scales;         /* jpeg int8: (B*H, cap, s); else NULL */
  void* anchors;         /* png: (B*H, cap, D); else NULL */
  int64_t cap;           /* capacity of the archive in blocks */
  void* tail;            /* (B, H, r, D) tail buffer */
  const void* token;     /* the new token */
  int64_t tok_sb, tok_sh;
  uint32_t* masks;       /* packed png: mask words (B*H, cap, D); else NULL */
} fc_step_stream;

typedef struct fc_step_args {
  const void* q;         /* (B, Hq, 1, D) query, element strides q_sb, q_sh */
  int q_dtype;
  int64_t q_sb, q_sh;
  int64_t B, Hq, Hkv, D;
  int store_kind;        /* FC_STORE_* */
  int stream_dtype;      /* dtype of the tokens, tails (and jpeg fp stores) */
  int r;                 /* block size */
  int s;                 /* stored rows per block: keep_freqs (jpeg) or r (png) */
  int quant_bits;        /* jpeg: 0 or 8 */
  int keep_m;            /* png: deltas kept per (block, feature) */
  int64_t n_blocks;      /* archived blocks before the step */
  int64_t n_tail;        /* tail tokens before the step (< r) */
  const float* basis;    /* jpeg: k x r DCT-II basis (device); png: NULL */
  const float* A;        /* r x s synthesis matrix (device) */
  float scale;           /* attention scale */
  void* out;             /* (B, Hq, 1, D) output in q_dtype, strides o_sb, o_sh */
  int64_t o_sb, o_sh;
  void* workspace;       /* decode-attention workspace (zero-fill rule) */
  int64_t workspace_bytes;
  int n_cu;              /* compute units of the device (split count) */
  void* stream;          /* hipStream_t */
  fc_step_stream key, value;
  int64_t* state;        /* device (n_blocks, n_tail, overflow), or NULL: see below */
} fc_step_args;

/*
 * One decode step of one attention layer: appends the new key and value
 * tokens to their tails; if that completes a block (n_tail + 1 == r) both
 * tails are archived as block n_blocks (the caller grows the archives
 * beforehand; cap <= n_blocks is FC_ERR_ARG) and the tails become empty;
 * then the decode attention runs over the archives and tails as
 * fc_decode_attention with the split count of fc_attention_splits
 * (workspace_bytes must cover fc_attention_workspace_bytes for it).  After
 * the call the caller's state is n_tail' = (n_tail + 1) % r and
 * n_blocks' = n_blocks + (n_tail + 1 == r).
 * Replaces the decode-step sequence key_stream.append(k);
 * value_stream.append(v); codec_decode_attention(q, ...) of
 * flashcodec/patch_attention.py:95-98 (flashcodec/cache.py:143-159,
 * flashcodec/attention.py:64-140) with one call.
 */
int fc_decode_step(const fc_step_args* args);
/*
 * With args->state != NULL (any store kind), the step takes n_blocks and
 * n_tail from the first two of the three int64 words at `state` on the
 * device and advances them there (n_tail + 1 == r moves a block into the
 * archive), so the enqueued work is the same at every step and a captured
 * HIP graph of it stays valid: the archive kernels run gated on the state,
 * the attention is one launch with its merge fused.  args->n_blocks (>= 1)
 * then only sizes the split count.  The archives must hold every block the
 * replayed steps will add: a block past `cap` is not written, the attention
 * reads at most `cap` blocks, and the third word (overflow, zero when the
 * caller sets up the state) becomes 1 and stays 1, for the caller to check.
 */

/*
 * How the calling thread's last successful fc_decode_step call ran: 1 when
 * the whole step was one kernel launch (int8 jpeg archives with one scale
 * per row or per 32 features, fp16 / bf16 / fp32 queries and stream; jpeg
 * archives of fp16 / bf16 / fp32 coefficients with queries and stream of
 * their dtype, fp32 with blocks of up to 16 tokens; png archives with
 * queries and stream of one dtype; packed Top-M png archives; a matrix-core
 * pass's shapes), 0 when it took the multi-launch form (token append,
 * archive, attention, state advance), -1 before any such call.  No counterpart in the reference (its
 * step is always two appends and an attention call); for callers and tests
 * that report or check launches per decode step.
 */
int fc_last_step_single_launch(void);
#ifdef __cplusplus
}
#endif

#endif /* FLASHCODEC_AMD_H */
