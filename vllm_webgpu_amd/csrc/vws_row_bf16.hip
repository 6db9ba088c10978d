// vws_row_bf16.hip -- the sampling kernel (vws_sample_row.h) for bf16 logits: plain, with raw
// logprobs, with an allowed-token mask (without and with raw logprobs), and under the logit
// soft cap (without and with raw logprobs).
#include "vws_sample_row.h"

namespace vws {
template __global__ void row_kernel<uint16_t, false, kXfNone>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<uint16_t, true, kXfNone>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<uint16_t, false, kXfMask>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<uint16_t, true, kXfMask>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<uint16_t, false, kXfCap>(const void*, int64_t, int, int, KArgs);
template __global__ void row_kernel<uint16_t, true, kXfCap>(const void*, int64_t, int, int, KArgs);
}  // namespace vws
