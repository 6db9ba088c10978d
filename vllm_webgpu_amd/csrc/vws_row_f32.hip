// vws_row_f32.hip -- the sampling kernel (vws_sample_row.h) for fp32 logits: plain, with raw
// logprobs, with an allowed-token mask (without and with raw logprobs), and under the logit
// soft cap (without and with raw logprobs).
#include "vws_sample_row.h"

namespace vws {
template __global__ void row_kernel<float, false, kXfNone>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, true, kXfNone>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, false, kXfMask>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, true, kXfMask>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, false, kXfCap>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<float, true, kXfCap>(const void*, int64_t, int, int, KArgs);
}  // namespace vws
