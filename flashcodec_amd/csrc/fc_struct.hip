// Structural operations on codec archives, device side (gfx950): batch
// gathers for beam-search reorders and batch selection / expansion, and the
// verbatim prefix copy of a capacity growth.
//
// Every archive buffer of a stream ((B, H, cap, s, D) codes or
// coefficients, (B, H, cap, s) scales, (B, H, cap, r-1, D) deltas,
// (B, H, cap, D) anchors, the (B, H, r, D) tail buffer, the (B, H, T, D)
// reconstruction) is, per (batch row, head), one contiguous run of bytes
// whose live part is a prefix.  So all of them are the same operation: a
// gather of (row, head) byte segments, dst(b, h) = src(idx[b], h).
//
// In place (dst == src), a gather with repeated or permuted indices must
// read every source segment before it overwrites any: one workgroup owns a
// column (head h, byte chunk c) across all batch rows, stages the chunk of
// every source row in LDS, and writes after a barrier.  Columns are
// disjoint, so workgroups never race.  Out of place, threads copy straight.
// Indices outside [0, B_src) are skipped (the destination segment keeps
// its bytes), so no index can make a kernel read outside `src`.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <initializer_list>

#include "fc_attn_internal.h"
#include "fc_common.h"

namespace fc {

constexpr int kStructThreads = 256;
constexpr int kStageBytes = 32768;  // LDS staging of an in-place column

template <int VB>
struct word_of;
template <>
struct word_of<16> {
  typedef uint4 type;
};
template <>
struct word_of<4> {
  typedef uint32_t type;
};
template <>
struct word_of<1> {
  typedef uint8_t type;
};

struct GatherArgs {
  char* dst;
  const char* src;
  int64_t d_sb, d_sh, s_sb, s_sh;  // bytes
  const int64_t* idx;              // B_out indices, or NULL (identity)
  int64_t B_out, B_src, H, len;    // len: bytes per segment
  int64_t chunk;                   // in-place: bytes of a column chunk
};

__device__ __forceinline__ int64_t src_row(const GatherArgs& a, int64_t b) {
  const int64_t s = a.idx ? a.idx[b] : b;
  return (s >= 0 && s < a.B_src) ? s : -1;
}

// Out of place: one thread per word of a (b, h) segment, grid-stride.
template <int VB>
__global__ __launch_bounds__(kStructThreads) void gather_copy_kernel(GatherArgs a) {
  typedef typename word_of<VB>::type W;
  const int64_t words = a.len / VB;
  const int64_t total = a.B_out * a.H * words;
  for (int64_t i = blockIdx.x * (int64_t)kStructThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kStructThreads) {
    const int64_t seg = i / words, w = i - seg * words;
    const int64_t b = seg / a.H, h = seg - b * a.H;
    const int64_t s = src_row(a, b);
    if (s < 0) continue;
    const W v = *reinterpret_cast<const W*>(a.src + s * a.s_sb + h * a.s_sh + w * VB);
    *reinterpret_cast<W*>(a.dst + b * a.d_sb + h * a.d_sh + w * VB) = v;
  }
}

// In place: workgroup (chunk c, head h) stages bytes [c * chunk, ...) of
// every source row in LDS, then writes every destination row.
template <int VB>
__global__ __launch_bounds__(kStructThreads) void gather_inplace_kernel(GatherArgs a) {
  typedef typename word_of<VB>::type W;
  __shared__ __attribute__((aligned(16))) char stage[kStageBytes];
  const int64_t h = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * a.chunk;
  const int64_t cw = (min(a.chunk, a.len - c0)) / VB;  // words of this chunk per row
  const int64_t n = a.B_out * cw;
  W* st = reinterpret_cast<W*>(stage);
  const int64_t row_words = a.chunk / VB;  // LDS row pitch
  for (int64_t i = threadIdx.x; i < n; i += kStructThreads) {
    const int64_t b = i / cw, w = i - b * cw;
    const int64_t s = src_row(a, b);
    if (s >= 0)
      st[b * row_words + w] =
          *reinterpret_cast<const W*>(a.src + s * a.s_sb + h * a.s_sh + c0 + w * VB);
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < n; i += kStructThreads) {
    const int64_t b = i / cw, w = i - b * cw;
    if (src_row(a, b) >= 0)
      *reinterpret_cast<W*>(a.dst + b * a.d_sb + h * a.d_sh + c0 + w * VB) = st[b * row_words + w];
  }
}

static bool fits(int vb, const void* p, std::initializer_list<int64_t> v) {
  if (reinterpret_cast<uintptr_t>(p) % vb) return false;
  for (int64_t x : v)
    if (x % vb) return false;
  return true;
}

}  // namespace fc

using namespace fc;

extern "C" {

int fc_gather_segments(void* dst, int64_t d_sb, int64_t d_sh, const void* src, int64_t s_sb,
                       int64_t s_sh, const int64_t* idx, int64_t B_out, int64_t B_src,
                       int64_t H, int64_t len, void* stream) {
  if (B_out < 0 || B_src < 0 || H < 0 || len < 0) return FC_ERR_ARG;
  if (B_out == 0 || H == 0 || len == 0) return FC_OK;
  if (!dst || !src || B_src == 0) return FC_ERR_ARG;
  const bool inplace = dst == src;
  if (inplace && (d_sb != s_sb || d_sh != s_sh || B_out != B_src)) return FC_ERR_ARG;
  if (!inplace && !idx && B_out > B_src) return FC_ERR_ARG;
  const int vb = (fits(16, dst, {d_sb, d_sh, len}) && fits(16, src, {s_sb, s_sh})) ? 16
                 : (fits(4, dst, {d_sb, d_sh, len}) && fits(4, src, {s_sb, s_sh})) ? 4
                                                                                    : 1;
  GatherArgs a{static_cast<char*>(dst), static_cast<const char*>(src), d_sb, d_sh, s_sb, s_sh,
               idx, B_out, B_src, H, len, 0};
  hipStream_t st = (hipStream_t)stream;
  if (inplace) {
    // a column chunk of every row must fit the LDS stage
    int64_t chunk = (kStageBytes / B_out) / 16 * 16;
    if (chunk < 16) return FC_ERR_UNSUPPORTED;
    chunk = std::min<int64_t>(chunk, 4096);
    a.chunk = chunk;
    const dim3 grid((unsigned)((len + chunk - 1) / chunk), (unsigned)H);
    if (grid.y > 65535) return FC_ERR_UNSUPPORTED;
    if (vb == 16)
      gather_inplace_kernel<16><<<grid, kStructThreads, 0, st>>>(a);
    else if (vb == 4)
      gather_inplace_kernel<4><<<grid, kStructThreads, 0, st>>>(a);
    else
      gather_inplace_kernel<1><<<grid, kStructThreads, 0, st>>>(a);
    return check_launch();
  }
  const int64_t total = B_out * H * (len / vb);
  const int64_t blocks = std::min<int64_t>((total + kStructThreads - 1) / kStructThreads, 4096);
  if (vb == 16)
    gather_copy_kernel<16><<<(unsigned)blocks, kStructThreads, 0, st>>>(a);
  else if (vb == 4)
    gather_copy_kernel<4><<<(unsigned)blocks, kStructThreads, 0, st>>>(a);
  else
    gather_copy_kernel<1><<<(unsigned)blocks, kStructThreads, 0, st>>>(a);
  return check_launch();
}

}  // extern "C"
