// vws_row_bf16.hip -- the sampling kernel (vws_sample_row.h) for bf16 logits, without and
// with raw logprobs, and with an allowed-token mask.
#include "vws_sample_row.h"

namespace vws {
template __global__ void row_kernel<uint16_t, false, false>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<uint16_t, true, false>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<uint16_t, false, true>(const void*, int64_t, int, int, KArgs);
}  // namespace vws
