// Instantiations of the packed png decode attention for blocks of up to
// 4 tokens with up to 4 kept deltas per feature (one translation unit
// per bucket keeps the builds parallel).
#include "fc_attn_pngpk.h"

namespace fc {
template int launch_pngpk_rows<4, 4>(const MfmaArgs&, int, int, bool, dim3, hipStream_t);
}  // namespace fc
