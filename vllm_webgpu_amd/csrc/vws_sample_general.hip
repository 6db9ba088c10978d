// vws_sample_general.hip -- the multi-pass kernel as its own launch (one 1024-thread workgroup per
// row), used by the top-k operation for the rows its single-pass kernel leaves over.
#include "vws_general.h"

namespace vws {

template <typename T>
__global__ __launch_bounds__(kGenThreads) void general_kernel(KArgs a) {
    __shared__ GenSmem sm;
    const int r = blockIdx.x;
    if (r >= a.B) return;
    const RowP prm = row_params(a, r);
    const bool need = fast_k(a, prm) == 0 || a.row_state[r] != 0u;
    if (!need) return;
    __syncthreads();
    if (threadIdx.x == 0) a.row_state[r] = 0u;
    if (a.mode == kModeTopK) general_topk_row<T>(a, sm, r);
    else general_row<T>(a, sm, r, prm);
}

template __global__ void general_kernel<float>(KArgs);
template __global__ void general_kernel<uint16_t>(KArgs);
template __global__ void general_kernel<_Float16>(KArgs);

}  // namespace vws
