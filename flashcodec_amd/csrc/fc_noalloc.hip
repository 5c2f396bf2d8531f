// Decode attention for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc): fc_decode_attention with its workspace taken from a static
// device array of this library instead of an argument.
//
// The array, `scratch`, is one per GPU (the runtime gives every device its
// own copy when it loads the code object) and lives until the process ends.
// Host code never passes the array's name to a kernel or a copy: the name
// is a host-side stand-in, not a device address.  On a device's first call
// its address is looked up with hipGetSymbolAddress (with that device
// current) and kept per device; kernels receive that pointer exactly as they
// receive a caller's workspace.
//
// What must start at zero (the fused step's done count and the pass-queue /
// arrival counters at the head of the array) is zero when the code
// object is loaded, is cleared once more by a fill kernel at set-up, and is
// returned to zero by every call.  Every call on a GPU shares that GPU's
// array: calls that overlap on one GPU (other streams, other threads) race
// and must not be issued.
#include <hip/hip_runtime.h>

#include <mutex>

#include "fc_attn_internal.h"
#include "fc_common.h"

namespace fc {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[FC_NOALLOC_SCRATCH_BYTES];

static void* g_scratch_ptr[kMaxDevices] = {};
static std::mutex g_scratch_mutex;

// zero words [0, n) of the scratch (the header line and the counters)
__global__ void scratch_clear_kernel(unsigned int* words, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    words[i] = 0u;
}

// Device address of the current device's scratch array (set up on the first
// call on that device), or NULL with *rc set.
static void* noalloc_scratch(hipStream_t stream, int* rc) {
  int dev = -1;
  *rc = hip_status(hipGetDevice(&dev));
  if (*rc != FC_OK) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = FC_ERR_UNSUPPORTED;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
  void* ptr = nullptr;
  *rc = hip_status(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  if (*rc != FC_OK) return nullptr;
  if (!ptr) {
    *rc = FC_ERR_HIP;
    return nullptr;
  }
  // a fill kernel, not hipMemsetAsync: the first call may be under capture
  scratch_clear_kernel<<<64, 256, 0, stream>>>(static_cast<unsigned int*>(ptr),
                                               kWsCounterRegionWords);
  *rc = check_launch();
  if (*rc != FC_OK) return nullptr;
  g_scratch_ptr[dev] = ptr;
  return ptr;
}

}  // namespace fc

using namespace fc;

extern "C" {

int fc_decode_attention_noalloc(const void* q, int q_dtype, int64_t q_sb, int64_t q_sh,
                                int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int store_kind,
                                int stream_dtype, int r, int s, int64_t nb,
                                const fc_stream_view* key, const fc_stream_view* value,
                                int64_t n_raw, const float* A, float scale, void* out,
                                int64_t o_sb, int64_t o_sh, int n_splits, void* stream) {
  if (B <= 0 || Hq <= 0 || D <= 0 || nb < 0) return FC_ERR_ARG;
  if (nb > 0 && fc_attention_workspace_bytes(B, Hq, D, n_splits) > FC_NOALLOC_SCRATCH_BYTES)
    return FC_ERR_SCRATCH;
  int rc = FC_OK;
  void* ws = noalloc_scratch((hipStream_t)stream, &rc);
  if (!ws) return rc;
  return decode_attention_parts(q, q_dtype, q_sb, q_sh, B, Hq, Hkv, D, store_kind, stream_dtype,
                                r, s, nb, key, value, n_raw, A, scale, out, o_sb, o_sh, ws,
                                n_splits, stream, kPartSplit | kPartMerge);
}

}  // extern "C"
