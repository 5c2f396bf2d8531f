// Prefill kernel variants with the matrix-core softmax, blocks of 16 tokens
// from 4 stored rows (the kernel: fc_prefill_kernel.h).
#include "fc_prefill_kernel.h"

namespace fc {

template int launch_prefill<4, 16>(const PrefillArgs&, int, int, int, bool, unsigned, hipStream_t);

}  // namespace fc
