// Instantiations of the matrix-core decode attention for 2 stored rows per
// block (one translation unit per row count keeps the builds parallel).
#include "fc_attn_mfma_kernel.h"

namespace fc {
template int launch_mfma_rows<2>(const MfmaArgs&, int, int, dim3, hipStream_t);
}  // namespace fc
