// Instantiations of the packed png decode attention for blocks of up to
// 8 tokens with up to 8 kept deltas per feature (one translation unit
// per bucket keeps the builds parallel).
#include "fc_attn_pngpk.h"

namespace fc {
template int launch_pngpk_rows<8, 8>(const MfmaArgs&, int, int, bool, dim3, hipStream_t);
}  // namespace fc
