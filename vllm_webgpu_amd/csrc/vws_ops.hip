// vws_ops.hip -- the standalone row operations of the library: batched argmax (the argmax.wgsl
// contract), row softmax with temperature (softmax.wgsl), in-place penalties, and the device
// self-test of the sampler arithmetic.
#include "vws_device.h"
#include "vws_internal.h"
#include "vws_sampler.h"

namespace vws {

constexpr int kOpThreads = 1024;
constexpr int kOpWaves = kOpThreads / 64;

__device__ __forceinline__ uint64_t op_block_max(uint64_t v, uint64_t* red) {
    v = wave_max_u64(v);
    __syncthreads();
    if (lane_id() == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < kOpWaves; ++i) t = t > red[i] ? t : red[i];
    return t;
}

__device__ __forceinline__ double op_block_sum_f64(double v, double* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    __syncthreads();
    if (lane_id() == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < kOpWaves; ++i) t += red[i];
    return t;
}

// One workgroup per row; (key << 32 | 0x7FFFFFFF - index) max = largest value, lowest index.
template <typename T>
__global__ __launch_bounds__(kOpThreads) void argmax_kernel(const T* logits, int64_t stride, int V,
                                                             int32_t* out) {
    __shared__ uint64_t red[kOpWaves];
    const int r = blockIdx.x;
    Slice<T> sl;
    sl.init(logits + (size_t)r * stride, 0, V);
    constexpr int VEC = Elem<T>::kVec;
    uint64_t best = 0;
    for (int c = threadIdx.x; c < sl.nchunks(); c += kOpThreads) {
        float v[VEC];
        const int i0 = sl.load(c, v);
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const uint64_t pk = ((uint64_t)key_of(v[j]) << 32) | (uint32_t)(0x7FFFFFFF - (i0 + j));
            best = best > pk ? best : pk;
        }
    }
    best = op_block_max(best, red);
    if (threadIdx.x == 0) {
        int32_t tok = (int32_t)(0x7FFFFFFF - (uint32_t)(best & 0xFFFFFFFFu));
        if ((best >> 32) == 0u || tok >= V) tok = 0;  // every element NaN
        out[r] = tok;
    }
}

// probs = exp_det(x/T - m) / S, m = max x/T, S = sum exp_det(x/T - m); one workgroup per row.
// Rows of up to 32 values per thread (V <= 32768: 8 chunks of fp32, 4 of 16-bit values) are
// read once: each thread keeps its chunks in registers through the max, the sum and the write
// (one read and one write of the row).  Longer rows are read twice: the maximum and S together
// (an online merge of per-thread running maxima and sums), then the write.  S is summed in
// double, in a different order than the sequential oracle (and, for long rows, with rescaled
// partial sums); each probability is e * fl64(1 / S): the probabilities agree with the oracle's
// to within a few fp32 ulps.
template <typename T>
__global__ __launch_bounds__(kOpThreads) void softmax_kernel(const T* logits, int64_t stride, int V,
                                                              const float* temperature, float* probs,
                                                              float* row_max, float* log_sum) {
    __shared__ uint64_t red[kOpWaves];
    __shared__ double redd[kOpWaves];
    const int r = blockIdx.x;
    const float Tt = temperature ? temperature[r] : 1.0f;
    Slice<T> sl;
    sl.init(logits + (size_t)r * stride, 0, V);
    constexpr int VEC = Elem<T>::kVec;
    constexpr int kSoftmaxRegs = 32 / VEC;  // chunks a thread keeps in registers
    const int nch = sl.nchunks();
    // element i of chunk c (head and tail chunks are NaN-padded) lies in the row
    auto inside = [&](int c, int i) {
        const bool in = (c == 0) ? (i < sl.a) : (c <= sl.nbody ? true : i < V);
        return c <= sl.nbody + 1 && in && i < V;
    };
    float* out = probs + (size_t)r * V;
    uint64_t mk = 0;
    double s = 0.0;
    float m;
    double S;
    if (nch <= kSoftmaxRegs * kOpThreads) {
        // the row in registers: y = fl(x / T) once, then e = exp(y - m) in place of y, then
        // the probabilities e * fl64(1 / S) (within an ulp of e / S)
        float v[kSoftmaxRegs][VEC];
#pragma unroll
        for (int q = 0; q < kSoftmaxRegs; ++q) {
            const int c = threadIdx.x + q * kOpThreads;
            if (c < nch) {
                sl.load(c, v[q]);
            } else {
#pragma unroll
                for (int j = 0; j < VEC; ++j) v[q][j] = __builtin_nanf("");
            }
        }
        if (Tt != 1.0f) {
#pragma unroll
            for (int q = 0; q < kSoftmaxRegs; ++q)
#pragma unroll
                for (int j = 0; j < VEC; ++j) v[q][j] = v[q][j] / Tt;
        }
#pragma unroll
        for (int q = 0; q < kSoftmaxRegs; ++q)
#pragma unroll
            for (int j = 0; j < VEC; ++j) { const uint64_t k = key_of(v[q][j]); mk = mk > k ? mk : k; }
        mk = op_block_max(mk, red);
        m = mk ? val_of((uint32_t)mk) : -__builtin_inff();  // (a row of NaN: the empty maximum)
#pragma unroll
        for (int q = 0; q < kSoftmaxRegs; ++q)
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                // exp_det is 0 for NaN (NaN logits, padding, y - m of infinities)
                const float e = exp_det(v[q][j] - m);
                v[q][j] = e;
                const int c = threadIdx.x + q * kOpThreads;
                const int i0 = c == 0 ? 0 : sl.a + (c - 1) * VEC;
                if (c < nch && inside(c, i0 + j)) s += (double)e;
            }
        S = op_block_sum_f64(s, redd);
        const double inv = 1.0 / S;
#pragma unroll
        for (int q = 0; q < kSoftmaxRegs; ++q) {
            const int c = threadIdx.x + q * kOpThreads;
            // first element of chunk c: the row's start (head), the body vectors, the tail
            const int i0 = c == 0 ? 0 : sl.a + (c - 1) * VEC;
#pragma unroll
            for (int j = 0; j < VEC; ++j)
                if (c < nch && inside(c, i0 + j)) out[i0 + j] = (float)((double)v[q][j] * inv);
        }
    } else {
        // longer rows: the maximum and the normaliser in one pass (each thread keeps a running
        // maximum mt of its finite values and its sum st of exp(y - mt), rescaled when mt
        // rises; the workgroup merges them as sum st * exp(mt - m)), then a second pass writes
        // the probabilities.  Only finite values add a term: exp_det is 0 for NaN, for -inf
        // and for y - m of infinities, so S is 0 when m is not finite.
        float mt = -__builtin_inff();
        double st = 0.0;
        for (int c = threadIdx.x; c < nch; c += kOpThreads) {
            float v[VEC];
            const int i0 = sl.load(c, v);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const float y = v[j] / Tt;
                const uint64_t k = key_of(y);
                mk = mk > k ? mk : k;
                if (!inside(c, i0 + j)) continue;  // padding of the head and tail chunks
                if (!(__builtin_fabsf(y) < __builtin_inff())) continue;
                if (y > mt) {
                    st = st * (double)exp_det(mt - y) + 1.0;
                    mt = y;
                } else {
                    st += (double)exp_det(y - mt);
                }
            }
        }
        mk = op_block_max(mk, red);
        m = mk ? val_of((uint32_t)mk) : -__builtin_inff();  // (a row of NaN: the empty maximum)
        const bool mfin = __builtin_fabsf(m) < __builtin_inff();
        S = op_block_sum_f64(mfin && mt > -__builtin_inff() ? st * (double)exp_det(mt - m) : 0.0, redd);
        const double inv = 1.0 / S;
        for (int c = threadIdx.x; c < nch; c += kOpThreads) {
            float v[VEC];
            const int i0 = sl.load(c, v);
#pragma unroll
            for (int j = 0; j < VEC; ++j)
                if (inside(c, i0 + j)) out[i0 + j] = (float)((double)exp_det(v[j] / Tt - m) * inv);
        }
    }
    if (threadIdx.x == 0) {
        if (row_max) row_max[r] = m;
        if (log_sum) log_sum[r] = (float)log(S);
    }
}

// In-place vLLM-v1 penalties on fp32 rows: one workgroup per row, history deduplicated in a
// per-row hash in the workspace.
__global__ __launch_bounds__(kOpThreads) void penalties_kernel(KArgs a, float* logits) {
    const int r = blockIdx.x;
    const float rep = a.rep ? a.rep[r] : 1.0f;
    const float pres = a.pres ? a.pres[r] : 0.0f;
    const float freq = a.freq ? a.freq[r] : 0.0f;
    const float inv_rep = 1.0f / rep;
    const int np = a.prompt ? (a.plens ? min(max(a.plens[r], 0), a.pwidth) : a.pwidth) : 0;
    const int no = a.output ? (a.olens ? min(max(a.olens[r], 0), a.owidth) : a.owidth) : 0;
    const int hs = a.hs_row;
    if (hs == 0 || (np == 0 && no == 0)) return;
    uint32_t* hkey = a.hist_hash + (size_t)r * (size_t)hs * 4;
    uint32_t* hval = hkey + hs;
    for (int i = threadIdx.x; i < hs; i += kOpThreads) { hkey[i] = 0u; hval[i] = 0u; }
    __threadfence();
    __syncthreads();
    auto insert = [&](int t, uint32_t inc) {
        uint32_t s = ((uint32_t)t * 2654435761u) & (uint32_t)(hs - 1);
        for (int probe = 0; probe < hs; ++probe) {
            const uint32_t prev = atomicCAS(&hkey[s], 0u, (uint32_t)t + 1u);
            if (prev == 0u || prev == (uint32_t)t + 1u) {
                if (inc & 0x80000000u) atomicOr(&hval[s], 0x80000000u);
                else atomicAdd(&hval[s], inc);
                return;
            }
            s = (s + 1u) & (uint32_t)(hs - 1);
        }
    };
    for (int i = threadIdx.x; i < np; i += kOpThreads) {
        const int t = a.prompt[(size_t)r * a.pstride + i];
        if (t >= 0 && t < a.V) insert(t, 0x80000000u);
    }
    for (int i = threadIdx.x; i < no; i += kOpThreads) {
        const int t = a.output[(size_t)r * a.ostride + i];
        if (t >= 0 && t < a.V) insert(t, 1u);
    }
    __threadfence();
    __syncthreads();
    float* row = logits + (size_t)r * a.lstride;
    for (int s = threadIdx.x; s < hs; s += kOpThreads) {
        const uint32_t kk = __hip_atomic_load(&hkey[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (!kk) continue;
        const uint32_t v = __hip_atomic_load(&hval[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int t = (int)kk - 1;
        row[t] = apply_penalty(row[t], (v >> 31) != 0u, v & 0x7FFFFFFFu, rep, inv_rep, freq, pres);
    }
    // The workspace is left as it was found (zeros): the top-k operation keeps its per-row part
    // counters at the start of the same buffer, and a non-zero counter there would stop its
    // last-part election from ever firing.
    __syncthreads();
    for (int i = threadIdx.x; i < hs; i += kOpThreads) { hkey[i] = 0u; hval[i] = 0u; }
}

// Hash of f(x) over every fp32 x whose order key lies in [klo, khi]; same accumulation as the
// CPU oracle's checker (sum over inputs of bits(f(x)) * golden ^ bits(x)).
__global__ __launch_bounds__(256) void selftest_kernel(int fn, uint32_t klo, uint32_t khi,
                                                       unsigned long long* out) {
    __shared__ uint64_t red[4][2];
    uint64_t h = 0, c = 0;
    const uint64_t n = (uint64_t)khi - klo + 1ull;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const uint32_t key = klo + (uint32_t)i;
        const uint32_t bits = (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
        const float x = u2f(bits);
        const float y = fn == 0 ? exp_det(x)
                      : (fn == 1 ? log_det(x) : (fn == 2 ? softcap_det(x, 1.0f, 1.0f) : round_f16(x)));
        h += ((uint64_t)f2u(y) * 0x9E3779B97F4A7C15ull) ^ (uint64_t)bits;
        c++;
    }
    h = wave_sum_u64(h);
    c = wave_sum_u64(c);
    if (lane_id() == 0) { red[threadIdx.x >> 6][0] = h; red[threadIdx.x >> 6][1] = c; }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t th = 0, tc = 0;
        for (int w = 0; w < 4; ++w) { th += red[w][0]; tc += red[w][1]; }
        atomicAdd(&out[0], (unsigned long long)th);
        atomicAdd(&out[1], (unsigned long long)tc);
    }
}

__global__ void fill_u32_kernel(uint32_t* p, size_t n, uint32_t v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

// vws_token_state_update: one id per thread, counted (output) or flagged (prompt) in its row's
// word with a vector atomic (ids and rows may repeat within a call).
__global__ void token_state_kernel(uint32_t* st, int64_t stride, uint32_t* bits, int64_t bstride,
                                   int V, int n, const int32_t* rows, int row, const int32_t* tok,
                                   int kind) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= n) return;
    const int t = tok[i];
    const int rr = rows ? rows[i] : row;
    if (t < 0 || t >= V || rr < 0) return;
    uint32_t* w = st + (size_t)rr * (size_t)stride + (uint32_t)t;
    if (kind == VWS_STATE_OUTPUT) atomicAdd(w, 1u);
    else atomicOr(w, 0x80000000u);
    if (bits) atomicOr(bits + (size_t)rr * (size_t)bstride + ((uint32_t)t >> 5), 1u << (t & 31));
}

template __global__ void argmax_kernel<float>(const float*, int64_t, int, int32_t*);
template __global__ void argmax_kernel<uint16_t>(const uint16_t*, int64_t, int, int32_t*);
template __global__ void softmax_kernel<float>(const float*, int64_t, int, const float*, float*, float*, float*);
template __global__ void softmax_kernel<uint16_t>(const uint16_t*, int64_t, int, const float*, float*, float*, float*);
template __global__ void argmax_kernel<_Float16>(const _Float16*, int64_t, int, int32_t*);
template __global__ void softmax_kernel<_Float16>(const _Float16*, int64_t, int, const float*, float*, float*, float*);

}  // namespace vws
