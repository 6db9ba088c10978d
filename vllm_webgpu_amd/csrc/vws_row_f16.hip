// vws_row_f16.hip -- the sampling kernel (vws_sample_row.h) for f16 logits: plain, with raw
// logprobs, with an allowed-token mask (without and with raw logprobs), and under the logit
// soft cap (without and with raw logprobs).
#include "vws_sample_row.h"

namespace vws {
template __global__ void row_kernel<_Float16, false, kXfNone>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<_Float16, true, kXfNone>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<_Float16, false, kXfMask>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<_Float16, true, kXfMask>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<_Float16, false, kXfCap>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<_Float16, true, kXfCap>(const void*, int64_t, int, int, KArgs);
}  // namespace vws
