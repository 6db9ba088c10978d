// vws_row_f32.hip -- the sampling kernel (vws_sample_row.h) for fp32 logits, without and
// with raw logprobs, with an allowed-token mask, and under the logit soft cap (with and
// without raw logprobs).
#include "vws_sample_row.h"

namespace vws {
template __global__ void row_kernel<float, false, kXfNone>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, true, kXfNone>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, false, kXfMask>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, false, kXfCap>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, true, kXfCap>(const void*, int64_t, int, int, KArgs);
}  // namespace vws
