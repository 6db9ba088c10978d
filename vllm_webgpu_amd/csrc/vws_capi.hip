// vws_capi.hip -- extern "C" entry points of _vws.so: argument validation (pure host code),
// workspace layout, shape-dependent launch decisions and kernel launches on the caller's stream.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "vws_internal.h"
#include "vws_sampler.h"

namespace vws {
template <typename T> __global__ void fast_kernel(KArgs);
template <typename T> __global__ void general_kernel(KArgs);
template <typename T, bool LP, int XF> __global__ void row_kernel(const void*, int64_t, int, int, KArgs);
template <typename T> __global__ void argmax_kernel(const T*, int64_t, int, int32_t*);
template <typename T>
__global__ void softmax_kernel(const T*, int64_t, int, const float*, float*, float*, float*);
__global__ void penalties_kernel(KArgs, float*);
__global__ void selftest_kernel(int, uint32_t, uint32_t, unsigned long long*);
__global__ void fill_u32_kernel(uint32_t*, size_t, uint32_t);
__global__ void token_state_kernel(uint32_t*, int64_t, uint32_t*, int64_t, int, int, const int32_t*, int,
                                   const int32_t*, int);
}  // namespace vws

using namespace vws;

// Static device scratch of vws_sample_noalloc (one copy per GPU, held until the process ends).
// Host code never uses this name as an address: the per-device address comes from
// hipGetSymbolAddress (scratch_address below) and only that pointer is handed to kernels.
static __device__ __align__(256) unsigned char scratch[VWS_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_err;

// Bound of a top-p row's wait for the chunks of its cooperative passes run by other workgroups
// (vws_set_coop_wait_polls), read at every launch.
std::atomic<int> g_coop_wait_polls{kCoopWaitPolls};
// Whether rows may take the single pass (vws_set_single_pass), read at every launch.
std::atomic<int> g_single_pass{1};

#ifdef VWS_TRACE
// Trace build: the record buffer of vws_trace_set and its workgroup count, read at every launch.
std::mutex g_trace_mu;
uint64_t* g_trace_buf = nullptr;
int g_trace_wgs = 0;
#endif

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return VWS_OK;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(VWS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return VWS_OK;
}

struct DeviceInfo {
    int cus = 0;
    int fast_blocks_per_cu = 0;
    int row_blocks_per_cu = 0;  // sampling workgroups resident per CU at once
};

DeviceInfo device_info() {
    static std::mutex mu;
    static DeviceInfo cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    std::lock_guard<std::mutex> lock(mu);
    DeviceInfo& d = cache[dev];
    if (d.cus == 0) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) == hipSuccess) d.cus = prop.multiProcessorCount;
        if (d.cus <= 0) d.cus = 256;
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fast_kernel<float>, kFastThreads, 0) != hipSuccess || n <= 0) n = 4;
        d.fast_blocks_per_cu = n;
        int nr = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nr, row_kernel<float, false, kXfNone>, kGenThreads, 0) != hipSuccess || nr <= 0) nr = 1;
        d.row_blocks_per_cu = nr;
        (void)hipGetLastError();
    }
    return d;
}

// Parts per row for the split-row top-k kernel: enough workgroups to fill every slot of the chip
// once, with at least 4096 elements per part.
void choose_parts(int B, int V, int esize, int* S, int* part_len) {
    const DeviceInfo d = device_info();
    const int slots = d.cus * d.fast_blocks_per_cu;
    int s = slots / (B > 0 ? B : 1);
    if (s < 1) s = 1;
    if (s > kMaxParts) s = kMaxParts;
    const int max_by_len = V / 4096 > 0 ? V / 4096 : 1;
    if (s > max_by_len) s = max_by_len;
    const int min_parts = (V + kPartMax - 1) / kPartMax;  // kMaxParts parts cover VWS_MAX_VOCAB
    if (s < min_parts) s = min_parts;
    int len = (V + s - 1) / s;
    const int align = 64;  // elements; keeps every part start 16-byte aligned
    len = (len + align - 1) / align * align;
    if (len > kPartMax) len = kPartMax;
    (void)esize;
    s = (V + len - 1) / len;
    *S = s;
    *part_len = len;
}

int esize_of(int dtype) { return dtype == VWS_DTYPE_F32 ? 4 : 2; }

// Per-device address of `scratch`, looked up once per device with that device current and
// cleared once by a fill kernel on the caller's stream (the kernels also clear what they use).
// The array is zero when the code object is loaded (static storage), which is the state the
// kernels need; the first call outside graph capture also clears it once and waits for that
// clear before any call can use the address, so that a first call from another stream cannot
// overtake it.  Under capture nothing is enqueued (the clear would otherwise be recorded into
// the caller's graph and replayed with it).
struct ScratchSlot {
    void* ptr = nullptr;
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[64];

int scratch_address(hipStream_t s, void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return fail(VWS_ERR_HIP, "vws_sample_noalloc: no current HIP device (or device index >= 64)");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ScratchSlot& slot = g_scratch[dev];
    if (!slot.ptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(VWS_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &cs) != hipSuccess) cs = hipStreamCaptureStatusNone;
        (void)hipGetLastError();
        if (cs == hipStreamCaptureStatusNone) {
            const size_t n = VWS_NOALLOC_SCRATCH_BYTES / 4;
            hipLaunchKernelGGL(fill_u32_kernel, dim3(1024), dim3(256), 0, s, static_cast<uint32_t*>(p), n, 0u);
            if (int st = check_launch("vws_sample_noalloc (scratch clear)")) return st;
            const hipError_t se = hipStreamSynchronize(s);
            if (se != hipSuccess)
                return fail(VWS_ERR_HIP, "vws_sample_noalloc (scratch clear): %s", hipGetErrorString(se));
        }
        slot.ptr = p;
    }
    *out = slot.ptr;
    return VWS_OK;
}

// ---- optional per-kernel event timing (vws_profile_begin / vws_profile_end) ----
struct Profiler {
    std::mutex mu;
    bool on = false;
    int cap = 0, n = 0;
    hipEvent_t* ev = nullptr;
    int* kind = nullptr;
};
Profiler g_prof;

// The event pair of the next launch while profiling is on (else both null).
void prof_events(int kind, hipEvent_t* e0, hipEvent_t* e1) {
    *e0 = *e1 = nullptr;
    std::lock_guard<std::mutex> lock(g_prof.mu);
    if (!g_prof.on || g_prof.n >= g_prof.cap) return;
    const int i = g_prof.n++;
    g_prof.kind[i] = kind;
    *e0 = g_prof.ev[2 * i];
    *e1 = g_prof.ev[2 * i + 1];
}

// Launches kernel k on stream s.  While profiling is on, the launch carries its own event pair
// (hipExtLaunchKernel), which the runtime stamps when the kernel begins and ends: the elapsed
// time is the kernel's duration, as a kernel trace reports it, with no marker packets between
// back-to-back launches.
template <typename F, typename... A>
void launch(int kind, F k, dim3 g, dim3 b, hipStream_t s, A... args) {
    hipEvent_t e0, e1;
    prof_events(kind, &e0, &e1);
    if (e0) hipExtLaunchKernelGGL(k, g, b, 0, s, e0, e1, 0u, args...);
    else hipLaunchKernelGGL(k, g, b, 0, s, args...);
}

int validate_rows(const void* logits, int32_t dtype, int32_t B, int32_t V, int64_t stride) {
    if (!logits) return fail(VWS_ERR_INVALID_ARGUMENT, "logits is NULL");
    if (B < 1) return fail(VWS_ERR_INVALID_ARGUMENT, "batch must be >= 1 (got %d)", B);
    if (V < 1 || V > VWS_MAX_VOCAB)
        return fail(VWS_ERR_LIMIT, "vocab must be in [1, %d] (got %d)", VWS_MAX_VOCAB, V);
    if (dtype != VWS_DTYPE_F32 && dtype != VWS_DTYPE_BF16 && dtype != VWS_DTYPE_F16)
        return fail(VWS_ERR_UNSUPPORTED_DTYPE, "unsupported logits dtype %d", dtype);
    if (stride < V) return fail(VWS_ERR_INVALID_ARGUMENT, "logits_row_stride %lld < vocab %d", (long long)stride, V);
    return VWS_OK;
}

int validate_history(const int32_t* ids, int64_t stride, int32_t width, const char* name) {
    if (!ids) return VWS_OK;
    if (width < 0) return fail(VWS_ERR_INVALID_ARGUMENT, "%s_width must be >= 0", name);
    if (stride < width) return fail(VWS_ERR_INVALID_ARGUMENT, "%s_row_stride < %s_width", name, name);
    if (width > (1 << 24)) return fail(VWS_ERR_LIMIT, "%s_width too large", name);
    return VWS_OK;
}

// History entries a row can put into the hash: prompt, output and processor tokens.
int sample_history_width(const vws_sample_args* a) {
    return (a->prompt_ids ? a->prompt_width : 0) + (a->output_ids ? a->output_width : 0) +
           (a->adjust_ids ? a->adjust_width : 0);
}

int validate_sample(const vws_sample_args* a) {
    if (!a) return fail(VWS_ERR_INVALID_ARGUMENT, "args is NULL");
    if (a->struct_size != sizeof(vws_sample_args))
        return fail(VWS_ERR_INVALID_ARGUMENT, "struct_size %u != %zu (ABI mismatch)", a->struct_size, sizeof(vws_sample_args));
    int st = validate_rows(a->logits, a->dtype, a->batch, a->vocab, a->logits_row_stride);
    if (st) return st;
    if (!a->sampled) return fail(VWS_ERR_INVALID_ARGUMENT, "sampled is NULL");
    if (a->temperature) {
        if (!a->uniforms && !a->rng_seeds && !a->rng_key_set)
            return fail(VWS_ERR_INVALID_ARGUMENT,
                        "uniforms, rng_seeds or rng_key_set is required when temperature is given");
        if (a->uniforms && a->uniforms_row_stride < a->vocab)
            return fail(VWS_ERR_INVALID_ARGUMENT, "uniforms_row_stride < vocab");
    }
    if (a->num_logprobs < -1 || a->num_logprobs > VWS_MAX_LOGPROBS)
        return fail(VWS_ERR_LIMIT, "num_logprobs must be in [-1, %d] (got %d)", VWS_MAX_LOGPROBS, a->num_logprobs);
    if (a->num_logprobs > a->vocab) return fail(VWS_ERR_INVALID_ARGUMENT, "num_logprobs > vocab");
    if (a->num_logprobs >= 0 && (!a->logprob_ids || !a->logprob_vals || !a->logprob_ranks))
        return fail(VWS_ERR_INVALID_ARGUMENT, "logprob outputs are NULL while num_logprobs >= 0");
    if ((st = validate_history(a->prompt_ids, a->prompt_row_stride, a->prompt_width, "prompt"))) return st;
    if ((st = validate_history(a->output_ids, a->output_row_stride, a->output_width, "output"))) return st;
    if ((st = validate_history(a->adjust_ids, a->adjust_row_stride, a->adjust_width, "adjust"))) return st;
    if (a->adjust_ids && !a->adjust_vals) return fail(VWS_ERR_INVALID_ARGUMENT, "adjust_vals is NULL while adjust_ids is set");
    if (a->token_state) {
        if (a->prompt_ids || a->output_ids)
            return fail(VWS_ERR_INVALID_ARGUMENT, "token_state replaces prompt_ids/output_ids: pass one or the other");
        if (a->token_state_row_stride < a->vocab)
            return fail(VWS_ERR_INVALID_ARGUMENT, "token_state_row_stride < vocab");
        if (a->token_state_bits && a->token_state_bits_stride < (int64_t)(a->vocab + 31) / 32)
            return fail(VWS_ERR_INVALID_ARGUMENT, "token_state_bits_stride < ceil(vocab / 32) words");
    } else if (a->token_state_bits) {
        return fail(VWS_ERR_INVALID_ARGUMENT, "token_state_bits is set without token_state");
    }
    if (!(a->logit_softcap >= 0.0f) || a->logit_softcap == __builtin_inff())
        return fail(VWS_ERR_INVALID_ARGUMENT, "logit_softcap must be finite and >= 0 (got %g)", (double)a->logit_softcap);
    if (a->allowed_mask && a->allowed_row_stride < (int64_t)(a->vocab + 31) / 32)
        return fail(VWS_ERR_INVALID_ARGUMENT, "allowed_row_stride < ceil(vocab / 32) words");
    const int hw = sample_history_width(a);
    const size_t need = ws_layout(a->batch, a->vocab, hw, false).total;
    // without a history the workspace carries only the cooperative region: a NULL or smaller
    // workspace turns the cooperative passes off (sample_workspace)
    if (hw == 0 && (!a->workspace || a->workspace_bytes < need)) return VWS_OK;
    if (!a->workspace) return fail(VWS_ERR_WORKSPACE_TOO_SMALL, "workspace is NULL (need %zu bytes)", need);
    if (a->workspace_bytes < need)
        return fail(VWS_ERR_WORKSPACE_TOO_SMALL, "workspace has %zu bytes, need %zu", a->workspace_bytes, need);
    if (reinterpret_cast<uintptr_t>(a->workspace) & 255u)
        return fail(VWS_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    return VWS_OK;
}

// The workspace vws_sample uses (after validate_sample): NULL when it is absent or too small to
// hold the cooperative region of a launch without a history.
void* sample_workspace(const vws_sample_args* a, int hw) {
    const size_t need = ws_layout(a->batch, a->vocab, hw, false).total;
    return (a->workspace && a->workspace_bytes >= need) ? a->workspace : nullptr;
}

KArgs make_kargs(int B, int V, const void* logits, int64_t stride, void* ws, int hw, bool parts) {
    KArgs k;
    std::memset(&k, 0, sizeof(k));
    k.logits = logits;
    k.lstride = stride;
    k.B = B;
    k.V = V;
    k.L = -1;
    const WsLayout w = ws_layout(B, V, hw, parts);
    char* base = static_cast<char*>(ws);
    if (parts) {
        k.row_counter = reinterpret_cast<uint32_t*>(base + w.counter);
        k.row_state = reinterpret_cast<uint32_t*>(base + w.state);
        k.part_meta = reinterpret_cast<uint32_t*>(base + w.meta);
        k.part_list = reinterpret_cast<uint2*>(base + w.list);
    }
    k.hist_hash = w.hs_row ? reinterpret_cast<uint32_t*>(base + w.hash) : nullptr;
    k.hs_row = w.hs_row;
    if (!parts && ws) k.coop = reinterpret_cast<CoopState*>(base + w.coop);
    return k;
}

}  // namespace

extern "C" {

int32_t vws_abi_version(void) { return VWS_ABI_VERSION; }

const char* vws_last_error(void) { return g_err.c_str(); }

size_t vws_sample_workspace_size(int32_t batch, int32_t vocab, int32_t history_width) {
    if (batch < 1 || vocab < 1 || history_width < 0) return 0;
    return ws_layout(batch, vocab, history_width, false).total;
}

int vws_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
    if (!workspace) return fail(VWS_ERR_INVALID_ARGUMENT, "workspace is NULL");
    const size_t n = workspace_bytes / 4;
    if (n == 0) return ok();
    const int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                       static_cast<uint32_t*>(workspace), n, 0u);
    if (int st = check_launch("vws_workspace_init")) return st;
    return ok();
}

int vws_validate_sample_args(const vws_sample_args* args) {
    const int st = validate_sample(args);
    return st ? st : ok();
}

int vws_sample(const vws_sample_args* a) {
    int st = validate_sample(a);
    if (st) return st;
    const int hw = sample_history_width(a);
    KArgs k = make_kargs(a->batch, a->vocab, a->logits, a->logits_row_stride, sample_workspace(a, hw), hw, false);
    k.temperature = a->temperature;
    k.top_k = a->top_k;
    k.top_p = a->top_p;
    k.min_p = a->min_p;
    k.rep = a->repetition_penalty;
    k.pres = a->presence_penalty;
    k.freq = a->frequency_penalty;
    k.prompt = a->prompt_ids;
    k.pstride = a->prompt_row_stride;
    k.pwidth = a->prompt_ids ? a->prompt_width : 0;
    k.plens = a->prompt_lens;
    k.output = a->output_ids;
    k.ostride = a->output_row_stride;
    k.owidth = a->output_ids ? a->output_width : 0;
    k.olens = a->output_lens;
    k.tstate = a->token_state;
    k.tstride = a->token_state_row_stride;
    k.trows = a->token_state_rows;
    k.tbits = a->token_state ? a->token_state_bits : nullptr;
    k.tbstride = a->token_state_bits_stride;
    k.allowed = a->allowed_mask;
    k.astride = a->allowed_row_stride;
    k.adj_ids = a->adjust_ids;
    k.adj_vals = a->adjust_vals;
    k.adjstride = a->adjust_row_stride;
    k.adjwidth = a->adjust_ids ? a->adjust_width : 0;
    k.adjlens = a->adjust_lens;
    k.softcap = a->logit_softcap;
    k.inv_softcap = a->logit_softcap > 0.0f ? 1.0f / a->logit_softcap : 0.0f;
    k.softcap_f16 = (a->logit_softcap > 0.0f && a->logit_softcap_f16) ? 1 : 0;
    k.u = a->uniforms;
    k.ustride = a->uniforms_row_stride;
    k.rng_seed = a->uniforms ? nullptr : a->rng_seeds;
    k.rng_offset = a->uniforms ? nullptr : a->rng_offsets;
    k.rng_key = a->rng_key;
    k.sampled = a->sampled;
    k.flags = a->row_flags;
    k.nkept = a->num_kept;
    k.L = a->num_logprobs;
    k.lp_ids = a->logprob_ids;
    k.lp_vals = a->logprob_vals;
    k.lp_ranks = a->logprob_ranks;
    // more rows than workgroups resident at once: the kernel counts its workgroups, so that one
    // whose row is done waits for other rows' passes only once no workgroup is left to start
    const int grid = a->batch;
    if (k.coop) {
        const DeviceInfo d = device_info();
        if (a->batch > kCoopMaxGrid) k.coop = nullptr;
        else if (a->batch > d.cus * d.row_blocks_per_cu) k.coop_count = 1;
    }
    k.coop_wait_polls = g_coop_wait_polls.load(std::memory_order_relaxed);
    // the single pass switched off (vws_set_single_pass(0)): rows go straight to the top-p
    // stream or the general path, without the single pass's first loads
    k.nofast = g_single_pass.load(std::memory_order_relaxed) ? 0 : 1;
#ifdef VWS_TRACE
    {
        std::lock_guard<std::mutex> lock(g_trace_mu);
        k.trace = g_trace_buf;
        k.trace_wgs = g_trace_wgs;
    }
#endif
    const int cf = (k.coop ? 1 : 0) | (k.coop_count ? 2 : 0) |
                   ((k.coop_count && a->batch <= kRowOrderMaxBatch) ? 4 : 0);
    hipStream_t s = (hipStream_t)a->stream;
    // the kernels with the raw-logprob epilogue only for launches that ask for logprobs, those
    // with an allowed mask only for launches that have one (without logprobs it masks as it
    // streams, with them it masks the candidates of the single pass), those whose top-p path
    // caps as it streams only for launches with the soft cap and no mask
    const int K = VWS_KERNEL_SAMPLE;
    const bool lp = a->num_logprobs >= 0;
    const bool cap = a->logit_softcap > 0.0f && !a->allowed_mask;
    const int var = (lp ? 1 : 0) | (a->allowed_mask ? 2 : 0) | (cap ? 4 : 0);
    using Kern = void (*)(const void*, int64_t, int, int, KArgs);
    auto pick = [var](auto tag) -> Kern {
        using T = decltype(tag);
        switch (var) {
        case 1: return row_kernel<T, true, kXfNone>;
        case 2: return row_kernel<T, false, kXfMask>;
        case 3: return row_kernel<T, true, kXfMask>;
        case 4: return row_kernel<T, false, kXfCap>;
        case 5: return row_kernel<T, true, kXfCap>;
        default: return row_kernel<T, false, kXfNone>;
        }
    };
    Kern kern;
    if (a->dtype == VWS_DTYPE_F32) kern = pick(float{});
    else if (a->dtype == VWS_DTYPE_BF16) kern = pick(uint16_t{});
    else kern = pick(_Float16{});
    launch(K, kern, dim3(grid), dim3(kGenThreads), s, k.logits, k.lstride, k.V, cf, k);
    if ((st = check_launch("vws_sample"))) return st;
    return ok();
}

int vws_sample_noalloc(const vws_sample_args* a) {
    if (!a) return fail(VWS_ERR_INVALID_ARGUMENT, "args is NULL");
    if (a->struct_size != sizeof(vws_sample_args))
        return fail(VWS_ERR_INVALID_ARGUMENT, "struct_size %u != %zu (ABI mismatch)", a->struct_size, sizeof(vws_sample_args));
    if (a->batch < 1 || a->vocab < 1)
        return validate_sample(a);  // reports the shape error
    const int hw = sample_history_width(a);
    if (hw < 0) return validate_sample(a);
    const size_t need = ws_layout(a->batch, a->vocab, hw, false).total;
    if (need > (size_t)VWS_NOALLOC_SCRATCH_BYTES)
        return fail(VWS_ERR_LIMIT,
                    "vws_sample_noalloc: this batch needs %zu bytes of scratch (batch %d, history width %d); "
                    "the static scratch holds %zu (use vws_sample with a caller workspace)",
                    need, a->batch, hw, (size_t)VWS_NOALLOC_SCRATCH_BYTES);
    vws_sample_args b = *a;
    b.workspace = nullptr;
    b.workspace_bytes = 0;
    if (need) {
        // arguments first (host only), so a bad call touches no device state
        b.workspace = reinterpret_cast<void*>(uintptr_t(256));
        b.workspace_bytes = VWS_NOALLOC_SCRATCH_BYTES;
        if (int st = validate_sample(&b)) return st;
        void* p = nullptr;
        if (int st = scratch_address((hipStream_t)a->stream, &p)) return st;
        b.workspace = p;
    }
    return vws_sample(&b);
}

int vws_token_state_update(uint32_t* state, int64_t row_stride, uint32_t* bits,
                           int64_t bits_stride, int32_t vocab, int32_t n, const int32_t* rows,
                           int32_t row, const int32_t* tokens, int32_t kind, void* stream) {
    if (!state) return fail(VWS_ERR_INVALID_ARGUMENT, "state is NULL");
    if (vocab < 1 || vocab > VWS_MAX_VOCAB)
        return fail(VWS_ERR_LIMIT, "vocab must be in [1, %d] (got %d)", VWS_MAX_VOCAB, vocab);
    if (row_stride < vocab) return fail(VWS_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %d", (long long)row_stride, vocab);
    if (bits && bits_stride < (vocab + 31) / 32)
        return fail(VWS_ERR_INVALID_ARGUMENT, "bits_stride %lld < ceil(vocab / 32) = %d", (long long)bits_stride, (vocab + 31) / 32);
    if (n < 0) return fail(VWS_ERR_INVALID_ARGUMENT, "n must be >= 0 (got %d)", n);
    if (kind != VWS_STATE_OUTPUT && kind != VWS_STATE_PROMPT)
        return fail(VWS_ERR_INVALID_ARGUMENT, "kind must be VWS_STATE_OUTPUT or VWS_STATE_PROMPT (got %d)", kind);
    if (n == 0) return ok();
    if (!tokens) return fail(VWS_ERR_INVALID_ARGUMENT, "tokens is NULL");
    if (!rows && row < 0) return fail(VWS_ERR_INVALID_ARGUMENT, "row must be >= 0 when rows is NULL (got %d)", row);
    launch(VWS_KERNEL_OTHER, token_state_kernel, dim3((n + 255) / 256), dim3(256), (hipStream_t)stream,
           state, row_stride, bits, bits_stride, (int)vocab, (int)n, rows, (int)row, tokens, (int)kind);
    if (int st = check_launch("vws_token_state_update")) return st;
    return ok();
}

int vws_argmax(const void* logits, int32_t dtype, int32_t batch, int32_t vocab, int64_t row_stride,
               int32_t* out_ids, void* stream) {
    int st = validate_rows(logits, dtype, batch, vocab, row_stride);
    if (st) return st;
    if (!out_ids) return fail(VWS_ERR_INVALID_ARGUMENT, "out_ids is NULL");
    hipStream_t s = (hipStream_t)stream;
    const int K = VWS_KERNEL_ARGMAX;
    if (dtype == VWS_DTYPE_F32)
        launch(K, argmax_kernel<float>, dim3(batch), dim3(1024), s,
               static_cast<const float*>(logits), row_stride, vocab, out_ids);
    else if (dtype == VWS_DTYPE_BF16)
        launch(K, argmax_kernel<uint16_t>, dim3(batch), dim3(1024), s,
               static_cast<const uint16_t*>(logits), row_stride, vocab, out_ids);
    else
        launch(K, argmax_kernel<_Float16>, dim3(batch), dim3(1024), s,
               static_cast<const _Float16*>(logits), row_stride, vocab, out_ids);
    if ((st = check_launch("vws_argmax"))) return st;
    return ok();
}

size_t vws_topk_workspace_size(int32_t batch, int32_t vocab, int32_t k) {
    (void)k;
    if (batch < 1 || vocab < 1) return 0;
    return ws_layout(batch, vocab, 0, true).total;
}

int vws_topk(const void* logits, int32_t dtype, int32_t batch, int32_t vocab, int64_t row_stride,
             int32_t k, float* out_vals, int32_t* out_ids, void* workspace, size_t workspace_bytes,
             void* stream) {
    int st = validate_rows(logits, dtype, batch, vocab, row_stride);
    if (st) return st;
    if (k < 1 || k > kKMax || k > vocab) return fail(VWS_ERR_LIMIT, "k must be in [1, min(%d, vocab)] (got %d)", kKMax, k);
    if (!out_vals || !out_ids) return fail(VWS_ERR_INVALID_ARGUMENT, "outputs are NULL");
    const size_t need = vws_topk_workspace_size(batch, vocab, k);
    if (!workspace || workspace_bytes < need)
        return fail(VWS_ERR_WORKSPACE_TOO_SMALL, "workspace has %zu bytes, need %zu", workspace_bytes, need);
    KArgs ka = make_kargs(batch, vocab, logits, row_stride, workspace, 0, true);
    ka.topk_k = k;
    ka.topk_vals = out_vals;
    ka.topk_ids = out_ids;
    choose_parts(batch, vocab, esize_of(dtype), &ka.S, &ka.part_len);
    hipStream_t s = (hipStream_t)stream;
    const int bp = (batch + 7) / 8 * 8;
    const int K = VWS_KERNEL_TOPK;
    if (dtype == VWS_DTYPE_F32)
        launch(K, fast_kernel<float>, dim3(bp * ka.S), dim3(kFastThreads), s, ka);
    else if (dtype == VWS_DTYPE_BF16)
        launch(K, fast_kernel<uint16_t>, dim3(bp * ka.S), dim3(kFastThreads), s, ka);
    else
        launch(K, fast_kernel<_Float16>, dim3(bp * ka.S), dim3(kFastThreads), s, ka);
    if ((st = check_launch("vws_topk"))) return st;
    // rows whose single-pass candidate lists overflowed (ties) are finished exactly here
    if (dtype == VWS_DTYPE_F32)
        launch(K, general_kernel<float>, dim3(batch), dim3(kGenThreads), s, ka);
    else if (dtype == VWS_DTYPE_BF16)
        launch(K, general_kernel<uint16_t>, dim3(batch), dim3(kGenThreads), s, ka);
    else
        launch(K, general_kernel<_Float16>, dim3(batch), dim3(kGenThreads), s, ka);
    if ((st = check_launch("vws_topk (general kernel)"))) return st;
    return ok();
}

int vws_softmax(const void* logits, int32_t dtype, int32_t batch, int32_t vocab, int64_t row_stride,
                const float* temperature, float* probs, float* row_max, float* log_sum, void* stream) {
    int st = validate_rows(logits, dtype, batch, vocab, row_stride);
    if (st) return st;
    if (!probs) return fail(VWS_ERR_INVALID_ARGUMENT, "probs is NULL");
    hipStream_t s = (hipStream_t)stream;
    const int K = VWS_KERNEL_SOFTMAX;
    if (dtype == VWS_DTYPE_F32)
        launch(K, softmax_kernel<float>, dim3(batch), dim3(1024), s,
               static_cast<const float*>(logits), row_stride, vocab, temperature, probs, row_max, log_sum);
    else if (dtype == VWS_DTYPE_BF16)
        launch(K, softmax_kernel<uint16_t>, dim3(batch), dim3(1024), s,
               static_cast<const uint16_t*>(logits), row_stride, vocab, temperature, probs, row_max, log_sum);
    else
        launch(K, softmax_kernel<_Float16>, dim3(batch), dim3(1024), s,
               static_cast<const _Float16*>(logits), row_stride, vocab, temperature, probs, row_max, log_sum);
    if ((st = check_launch("vws_softmax"))) return st;
    return ok();
}

int vws_apply_penalties(float* logits, int32_t batch, int32_t vocab, int64_t row_stride,
                        const float* repetition, const float* presence, const float* frequency,
                        const int32_t* prompt_ids, int64_t prompt_row_stride, int32_t prompt_width,
                        const int32_t* prompt_lens, const int32_t* output_ids,
                        int64_t output_row_stride, int32_t output_width,
                        const int32_t* output_lens, void* workspace, size_t workspace_bytes,
                        void* stream) {
    int st = validate_rows(logits, VWS_DTYPE_F32, batch, vocab, row_stride);
    if (st) return st;
    if ((st = validate_history(prompt_ids, prompt_row_stride, prompt_width, "prompt"))) return st;
    if ((st = validate_history(output_ids, output_row_stride, output_width, "output"))) return st;
    const int hw = (prompt_ids ? prompt_width : 0) + (output_ids ? output_width : 0);
    if (hw == 0) return ok();  // nothing to penalise: the workspace is not touched
    const size_t need = ws_layout(batch, vocab, hw, false).total;
    if (!workspace || workspace_bytes < need)
        return fail(VWS_ERR_WORKSPACE_TOO_SMALL, "workspace has %zu bytes, need %zu", workspace_bytes, need);
    KArgs k = make_kargs(batch, vocab, logits, row_stride, workspace, hw, false);
    k.rep = repetition;
    k.pres = presence;
    k.freq = frequency;
    k.prompt = prompt_ids;
    k.pstride = prompt_row_stride;
    k.pwidth = prompt_ids ? prompt_width : 0;
    k.plens = prompt_lens;
    k.output = output_ids;
    k.ostride = output_row_stride;
    k.owidth = output_ids ? output_width : 0;
    k.olens = output_lens;
    launch(VWS_KERNEL_PENALTIES, penalties_kernel, dim3(batch), dim3(1024), (hipStream_t)stream, k, logits);
    if ((st = check_launch("vws_apply_penalties"))) return st;
    return ok();
}

int vws_math_selftest(int32_t fn, uint32_t key_lo, uint32_t key_hi, uint64_t* out2, void* stream) {
    if (fn < 0 || fn > 3) return fail(VWS_ERR_INVALID_ARGUMENT, "fn must be 0 (exp), 1 (log), 2 (soft cap) or 3 (f16 rounding)");
    if (!out2) return fail(VWS_ERR_INVALID_ARGUMENT, "out2 is NULL");
    if (key_hi < key_lo) return fail(VWS_ERR_INVALID_ARGUMENT, "key_hi < key_lo");
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, s, reinterpret_cast<uint32_t*>(out2), (size_t)4, 0u);
    int st = check_launch("vws_math_selftest (clear)");
    if (st) return st;
    hipLaunchKernelGGL(selftest_kernel, dim3(4096), dim3(256), 0, s, fn, key_lo, key_hi,
                       reinterpret_cast<unsigned long long*>(out2));
    if ((st = check_launch("vws_math_selftest"))) return st;
    return ok();
}

int32_t vws_set_coop_wait_polls(int32_t polls) {
    if (polls < 0) {
        fail(VWS_ERR_INVALID_ARGUMENT, "polls must be >= 0 (got %d)", polls);
        return -1;
    }
    return g_coop_wait_polls.exchange(polls);
}

int32_t vws_set_single_pass(int32_t enabled) {
    if (enabled != 0 && enabled != 1) {
        fail(VWS_ERR_INVALID_ARGUMENT, "enabled must be 0 or 1 (got %d)", enabled);
        return -1;
    }
    return g_single_pass.exchange(enabled);
}

int vws_trace_set(uint64_t* buf, int32_t max_workgroups) {
#ifdef VWS_TRACE
    if (max_workgroups < 0 || (max_workgroups > 0 && !buf))
        return fail(VWS_ERR_INVALID_ARGUMENT, "trace: a buffer of max_workgroups >= 0 records");
    std::lock_guard<std::mutex> lock(g_trace_mu);
    g_trace_buf = max_workgroups > 0 ? buf : nullptr;
    g_trace_wgs = max_workgroups;
    return ok();
#else
    (void)buf;
    (void)max_workgroups;
    return fail(VWS_ERR_UNSUPPORTED, "vws_trace_set: not the trace build of the library "
                                     "(vllm_webgpu_amd/_vws_trace.so records phase stamps)");
#endif
}

int vws_profile_begin(int32_t max_launches) {
    if (max_launches < 1 || max_launches > (1 << 20))
        return fail(VWS_ERR_INVALID_ARGUMENT, "max_launches must be in [1, 2^20]");
    std::lock_guard<std::mutex> lock(g_prof.mu);
    if (g_prof.on) return fail(VWS_ERR_INVALID_ARGUMENT, "profiling already active");
    g_prof.ev = new hipEvent_t[2 * (size_t)max_launches];
    g_prof.kind = new int[max_launches];
    for (int i = 0; i < 2 * max_launches; ++i) {
        if (hipEventCreate(&g_prof.ev[i]) != hipSuccess) {
            for (int j = 0; j < i; ++j) (void)hipEventDestroy(g_prof.ev[j]);
            delete[] g_prof.ev;
            delete[] g_prof.kind;
            g_prof.ev = nullptr;
            g_prof.kind = nullptr;
            return fail(VWS_ERR_HIP, "hipEventCreate failed");
        }
    }
    g_prof.cap = max_launches;
    g_prof.n = 0;
    g_prof.on = true;
    return ok();
}

int vws_profile_end(double* ms, int32_t* count) {
    std::lock_guard<std::mutex> lock(g_prof.mu);
    if (!g_prof.on) return fail(VWS_ERR_INVALID_ARGUMENT, "profiling is not active");
    for (int k = 0; k < VWS_KERNEL_KINDS; ++k) {
        if (ms) ms[k] = 0.0;
        if (count) count[k] = 0;
    }
    int st = VWS_OK;
    for (int i = 0; i < g_prof.n; ++i) {
        float t = 0.0f;
        if (hipEventSynchronize(g_prof.ev[2 * i + 1]) != hipSuccess ||
            hipEventElapsedTime(&t, g_prof.ev[2 * i], g_prof.ev[2 * i + 1]) != hipSuccess) {
            st = fail(VWS_ERR_HIP, "event timing failed");
            continue;
        }
        const int k = g_prof.kind[i];
        if (ms) ms[k] += (double)t;
        if (count) count[k] += 1;
    }
    for (int i = 0; i < 2 * g_prof.cap; ++i) (void)hipEventDestroy(g_prof.ev[i]);
    delete[] g_prof.ev;
    delete[] g_prof.kind;
    g_prof.ev = nullptr;
    g_prof.kind = nullptr;
    g_prof.on = false;
    g_prof.cap = g_prof.n = 0;
    return st ? st : ok();
}

}  // extern "C"
