// vws_row_f16.hip -- the sampling kernel (vws_sample_row.h) for f16 logits, without and
// with raw logprobs, and with an allowed-token mask.
#include "vws_sample_row.h"

namespace vws {
template __global__ void row_kernel<_Float16, false, false>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<_Float16, true, false>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<_Float16, false, true>(const void*, int64_t, int, int, KArgs);
}  // namespace vws
