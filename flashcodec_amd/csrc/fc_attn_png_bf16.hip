// The png matrix-core pass for bf16 streams and queries (fc_attn_png_kernel.h).
#include "fc_attn_png_kernel.h"

namespace fc {

template int launch_png_t<bf16_t>(const MfmaArgs&, int, int, int, dim3, hipStream_t);

}  // namespace fc
