// Declarations shared by the decode-attention sources (fc_attention.hip:
// argument checks, vector-ALU split pass, merge pass; fc_attn_mfma.hip:
// matrix-core split pass for int8 jpeg archives).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flashcodec_amd.h"

namespace fc {

int check_launch();
int esize_of(int dt);

// Fused merge of the matrix-core split pass: the last workgroup of each
// (batch, kv head, head group) combines the split partials with the raw
// tail and writes the output.
struct MfmaFuse {
  int raw_dtype;
  int64_t n_raw;
  void* out;
  int64_t o_sb, o_sh;
};

bool split_i8_mfma_supported(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t D,
                             int s, const fc_stream_view* key, const fc_stream_view* value);
bool split_i8_mfma_fusable(int n_splits);
// counters: counter_words zero words (zero again when the work is done): two
// per (batch, kv head, group of <= 16 query heads), `stride` words apart.
// fuse == nullptr: write the split partials only (pm, pl, pacc).
int launch_split_i8_mfma(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh, int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t D, int r, int s, int64_t nb,
                         const fc_stream_view* key, const fc_stream_view* value, const float* A,
                         float scale_log2, float* pm, float* pl, float* pacc, int n_splits,
                         unsigned int* counters, int64_t counter_words, int64_t stride,
                         const MfmaFuse* fuse, hipStream_t st);

}  // namespace fc
