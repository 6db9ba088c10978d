// vws_row_f32.hip -- the sampling kernel (vws_sample_row.h) for fp32 logits, without and
// with raw logprobs, and with an allowed-token mask.
#include "vws_sample_row.h"

namespace vws {
template __global__ void row_kernel<float, false, false>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, true, false>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, false, true>(const void*, int64_t, int, int, KArgs);
}  // namespace vws
