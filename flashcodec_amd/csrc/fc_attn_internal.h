// Declarations shared by the decode-attention sources (fc_attention.hip:
// argument checks, vector-ALU split pass, merge pass; fc_attn_mfma.hip:
// matrix-core split pass for int8 jpeg archives).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flashcodec_amd.h"

namespace fc {

typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kBufWord3 = 0x00020000;  // raw buffer descriptor: 32-bit data format
constexpr int kCachePolicySc1 = 16;    // buffer load cache policy: device scope (sc1)
constexpr int kWaitVmcnt0 = 0x0F70;    // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15)

// buffer descriptor over `bytes` bytes at `base`: loads at offsets past the
// end return zero
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, kBufWord3);
}

int check_launch();
int hip_status(hipError_t e);  // FC_OK, or FC_ERR_HIP with the error recorded
int esize_of(int dt);

// Process-wide settings, read once when the library loads
// (FLASHCODEC_AMD_ATTN=valu selects the vector-ALU split pass) and
// changeable through fc_set_attention_pass.
bool mfma_split_allowed();
bool static_pass_order();  // matrix-core pass without its dynamic pass queue

// Decode-attention workspace: a header line (the fused step's count of
// finished workgroups), the counter region (pass queues and arrival counts;
// zero between calls), then the split partials pm | pl | pacc.
constexpr int64_t kWsCounterRegionWords = 262144;  // 1 MiB
constexpr int64_t kWsHeadWords = 64;                // done count + padding (two lines)
constexpr int64_t kCounterWords = kWsCounterRegionWords - kWsHeadWords;
constexpr int64_t kCounterBytes = kWsCounterRegionWords * 4;
constexpr int64_t kCounterStride = 32;  // words between counters (no two share a line)
constexpr int64_t kCounterStrideMax = 256;  // 1 KiB
// Words between the counters of consecutive groups of the matrix-core
// passes (`slots` counters: two per group): as far apart as the counter
// region allows, up to 1 KiB, never closer than one 128-byte line.  Counters
// packed into a few KiB put every group's atomics on a few memory channels
// and slowed the streams through those channels (C3: 0.56 us per call).
// 0 when the region cannot hold the counters.
inline int64_t counter_stride(int64_t slots) {
  int64_t st = kCounterStrideMax;
  while (st > kCounterStride && slots * st > kCounterWords) st >>= 1;
  return slots * st <= kCounterWords ? st : 0;
}
struct WsLayout {
  unsigned int* done;      // fused decode step: workgroups finished (zero between calls)
  unsigned int* counters;  // kCounterWords words
  float* pm;
  float* pl;
  float* pacc;
};
WsLayout ws_layout(void* workspace, int64_t B, int64_t Hq, int n_splits);

// Fused merge of the matrix-core split pass: the last workgroup of each
// (batch, kv head, head group) combines the split partials with the raw
// tail and writes the output.
struct MfmaFuse {
  int raw_dtype;
  int64_t n_raw;
  void* out;
  int64_t o_sb, o_sh;
  // decode-step state on the device, (n_blocks, n_tail) before the step's
  // token, or NULL: the kernel then takes the block and tail counts from it
  const int64_t* state = nullptr;
  // fused decode step in the same launch (see fc_decode_step): the step's
  // tokens, the writable archives, the basis and the host counters (used
  // when state is NULL); `done` counts finished workgroups for the state
  // advance
  bool step = false;
  const void* ktok = nullptr;
  const void* vtok = nullptr;
  int64_t kt_sb = 0, kt_sh = 0, vt_sb = 0, vt_sh = 0;
  const float* basis = nullptr;
  int64_t step_t = 0, step_nb = 0;
  unsigned int* done = nullptr;
  int keep_m = 0;  // png: kept deltas per (block, feature)
};

// Whether fc_decode_step can run as one launch of the matrix-core pass for
// this step (int8 jpeg, the matrix-core pass's shapes, fp16 / bf16 stream,
// the step's rows fit the kernel's LDS scratch, fused merge).
bool step_i8_mfma_supported(int stream_dtype, int r, int64_t D, int n_splits);

// Query dtype, head size and stored rows per block of the matrix-core pass.
bool mfma_shape_supported(int q_dtype, int64_t D, int s);
bool split_i8_mfma_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                             int s, const fc_stream_view* key, const fc_stream_view* value);
bool split_i8_mfma_fusable(int n_splits);
bool mfma_group_shape_supported(int q_dtype, int64_t D, int s);
bool i8_mfma_takes(int store_kind, const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                   int64_t D, int s, const fc_stream_view* key, const fc_stream_view* value);
// counters: counter_words zero words (zero again when the work is done): two
// per (batch, kv head, group of <= 16 query heads), `stride` words apart.
// fuse == nullptr: write the split partials only (pm, pl, pacc).
int launch_split_i8_mfma(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t D, int r, int s, int64_t nb,
                         const fc_stream_view* key, const fc_stream_view* value, const float* A,
                         float scale_log2, float* pm, float* pl, float* pacc, int n_splits,
                         unsigned int* counters, int64_t counter_words, int64_t stride,
                         const MfmaFuse* fuse, hipStream_t st, bool grouped = false);

// The png matrix-core split pass (fc_attn_png.hip): queries in the stream's
// dtype (fp32, fp16, bf16; anchors in it, deltas fp32), D in {64, 128}, r in
// {4, 8, 16}; `state` as the fused decode step's device counters (or NULL).
bool png_mfma_shape_supported(int q_dtype, int stream_dtype, int64_t D, int r);
constexpr int kPngWgPerCu = 2;  // workgroups per compute unit of the png pass
// jpeg archives of fp16 / bf16 coefficients on the matrix cores
// (fc_attn_fpj.hip): queries in the stream dtype, D = 64 / 128, s = 1 / 2 /
// 3 / 4 / 8; fp32 coefficients with fp32 queries (the png pass's fp32
// products), s = 1 / 2 / 4 / 8 / 16.
bool fpj_mfma_shape_supported(int q_dtype, int stream_dtype, int64_t D, int s);
bool split_fpj_mfma_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                              int s, int stream_dtype, const fc_stream_view* key,
                              const fc_stream_view* value);
int launch_split_fpj_mfma(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                          int64_t Hq, int64_t Hkv, int64_t D, int r, int s, int64_t nb,
                          const fc_stream_view* key, const fc_stream_view* value, const float* A,
                          float scale_log2, float* pm, float* pl, float* pacc, int n_splits,
                          unsigned int* counters, int64_t counter_words, int64_t stride,
                          const MfmaFuse* fuse, const int64_t* state, hipStream_t st);
bool split_png_mfma_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                              int r, int stream_dtype, const fc_stream_view* key,
                              const fc_stream_view* value);
int launch_split_png_mfma(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                          int64_t Hq, int64_t Hkv, int64_t D, int r, int64_t nb,
                          const fc_stream_view* key,
                          const fc_stream_view* value, float scale_log2, float* pm, float* pl,
                          float* pacc, int n_splits, unsigned int* counters,
                          int64_t counter_words, int64_t stride, const MfmaFuse* fuse,
                          const int64_t* state, hipStream_t st);

// The packed png split pass (fc_attn_pngpk.hip): fp32 / fp16 / bf16
// queries and anchors, D in {64, 128, 256}, r <= 16, keep_m <= 8; `state`
// as the fused decode step's device counters (or NULL).
constexpr int kFuseMaxSplitsPk = 64;  // the fused merge's split limit (kFuseMaxSplits)
bool pngpk_shape_supported(int q_dtype, int stream_dtype, int64_t D, int r, int keep_m);
bool split_pngpk_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                           int r, int keep_m, int stream_dtype, const fc_stream_view* key,
                           const fc_stream_view* value);
int launch_split_pngpk(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                       int64_t Hq, int64_t Hkv, int64_t D, int r, int keep_m, int stream_dtype,
                       int64_t nb, const fc_stream_view* key, const fc_stream_view* value,
                       float scale_log2, float* pm, float* pl, float* pacc, int n_splits,
                       unsigned int* counters, int64_t counter_words, int64_t stride,
                       const MfmaFuse* fuse, const int64_t* state, hipStream_t st);

// fc_decode_attention's body: validates the arguments and enqueues the
// requested parts (kPartSplit: the split pass over the archived blocks;
// kPartMerge: the merge of the split partials with the raw tail, fused into
// the split pass where it can be) with `workspace` as scratch.
constexpr int kPartSplit = 1, kPartMerge = 2;
int decode_attention_parts(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                           int64_t Hq, int64_t Hkv, int64_t D, int store_kind, int stream_dtype,
                           int r, int s, int64_t nb, const fc_stream_view* key,
                           const fc_stream_view* value, int64_t n_raw, const float* A,
                           float scale, void* out, int64_t o_sb, int64_t o_sh, void* workspace,
                           int n_splits, void* stream, int parts);

// Decode attention over a graph-capturable decode step (fc_decode_step with
// a device state): one launch with the merge fused (matrix-core pass for
// int8 jpeg archives it supports, else the vector-ALU pass), block and tail
// counts read from `state` on the device; nb_hint (> 0) sizes the split
// count.
int decode_attention_state(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                           int64_t Hq, int64_t Hkv, int64_t D, int store_kind, int stream_dtype,
                           int r, int s, int64_t nb_hint, const fc_stream_view* key,
                           const fc_stream_view* value, const float* A, float scale, void* out,
                           int64_t o_sb, int64_t o_sh, void* workspace, int64_t workspace_bytes,
                           int n_cu, const int64_t* state, void* stream);

// png archive of one block of a decode step's tail, gated like
// jpeg_encode_gated.
// masks != NULL: the packed layout (deltas = the value store).
int png_encode_gated(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb,
                     int64_t x_sh, int64_t x_ss, int64_t D, int r, int keep_m, float* deltas,
                     void* anchors, int64_t cap, void* stream, const int64_t* gate,
                     uint32_t* masks = nullptr);

// jpeg archive of one block of a decode step's tail, gated on the device:
// runs only when gate[1] == r - 1 and writes block gate[0] (< cap).
int jpeg_encode_gated(const void* x, int x_dtype, int64_t B, int64_t H, int64_t x_sb,
                      int64_t x_sh, int64_t x_ss, int64_t D, int r, int k, const float* basis,
                      void* coeffs, float* scales, int64_t cap, int quant_bits, void* stream,
                      const int64_t* gate, int group = 0);

}  // namespace fc
