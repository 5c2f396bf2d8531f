// Workgroup-shared prefill kernel variants, blocks of 4 or 8 tokens from 4
// stored rows (the kernel: fc_prefill_wg.h).
#include "fc_prefill_wg.h"

namespace fc {

template int launch_prefill_wg<4>(const PrefillArgs&, int, int, int, unsigned, hipStream_t);
template int launch_prefill_wg<8>(const PrefillArgs&, int, int, int, unsigned, hipStream_t);

}  // namespace fc
