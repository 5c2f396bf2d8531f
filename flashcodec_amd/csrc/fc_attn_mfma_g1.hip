// Instantiations of the matrix-core decode attention over per-32 scales for
// 1 stored row per block (one translation unit per row count and scale
// layout keeps the builds parallel).
#include "fc_attn_mfma_kernel.h"

namespace fc {
template int launch_mfma_rows_g<1>(const MfmaArgs&, int, int, dim3, hipStream_t);
}  // namespace fc
