// vws_row.h -- per-row sampling parameters as the kernels see them, and the rule that sends a
// row to the single-pass kernel or to the general kernel.
#pragma once

#include "vws_device.h"
#include "vws_internal.h"
#include "vws_sampler.h"

namespace vws {

// Trace build (-DVWS_TRACE) only: lane 0 of the workgroup's last wave stores the device clock
// (s_memrealtime, 100 MHz) or a value into slot s of the workgroup's record (vws_trace_set).
// The last wave, because the wait for the clock read delays the wave that stores it: wave 0
// does the workgroup's serial work (edges, selections) and more often sets a phase's end.
// VWS_TRACE_MARK_AFTER first waits for dep, a value the phase produced, so that the stamp
// cannot be taken before the phase's loads have landed.
#ifdef VWS_TRACE
__device__ __forceinline__ bool trace_lane(const KArgs& a) {
    return a.trace && threadIdx.x == blockDim.x - 64u && (int)blockIdx.x < a.trace_wgs;
}
__device__ __forceinline__ void trace_put(const KArgs& a, int s, uint64_t v) {
    if (trace_lane(a)) a.trace[(size_t)blockIdx.x * VWS_TRACE_SLOTS + s] = v;
}
// the clock is read by the stamping wave alone (the others issue nothing)
__device__ __forceinline__ void trace_mark(const KArgs& a, int s) {
    if (trace_lane(a)) a.trace[(size_t)blockIdx.x * VWS_TRACE_SLOTS + s] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ uint64_t trace_clock() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ uint32_t trace_xcc() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xFu;
}
#define VWS_TRACE_MARK(a, s) ::vws::trace_mark((a), (s))
#define VWS_TRACE_MARK_AFTER(a, s, dep)                        \
    do {                                                       \
        asm volatile("" : : "v"((uint32_t)(dep)));             \
        VWS_TRACE_MARK(a, s);                                  \
    } while (0)
#define VWS_TRACE_PUT(a, s, v) ::vws::trace_put((a), (s), (uint64_t)(v))
#else
#define VWS_TRACE_MARK(a, s) ((void)0)
#define VWS_TRACE_MARK_AFTER(a, s, dep) ((void)0)
#define VWS_TRACE_PUT(a, s, v) ((void)0)
#endif

struct RowP {
    float T, top_p, min_p, rep, pres, freq, inv_rep;
    int k, np, no;
    int na;          // logits-processor entries (bans, logit bias) of the row
    int trow;        // the row's row of the token-state table
    bool greedy;
    bool has_hist;   // penalties apply: a history and not every penalty the identity
    bool tab;        // ... read from the token-state table (no history lists)
    bool need_hash;  // the row's hash holds history or processor tokens
};

__device__ __forceinline__ RowP row_params(const KArgs& a, int r) {
    RowP p;
    p.T = a.temperature ? a.temperature[r] : 0.0f;
    p.greedy = is_greedy(p.T);
    p.k = a.top_k ? a.top_k[r] : 0;
    p.top_p = a.top_p ? a.top_p[r] : 1.0f;
    p.min_p = a.min_p ? a.min_p[r] : 0.0f;
    p.rep = a.rep ? a.rep[r] : 1.0f;
    p.pres = a.pres ? a.pres[r] : 0.0f;
    p.freq = a.freq ? a.freq[r] : 0.0f;
    p.inv_rep = 1.0f / p.rep;
    // prompt tokens take only the repetition penalty: at r = 1 (x * 1 and x * fl(1 / 1) are x)
    // they change nothing and are not hashed
    p.np = (a.prompt && p.rep != 1.0f) ? (a.plens ? min(max(a.plens[r], 0), a.pwidth) : a.pwidth) : 0;
    p.no = a.output ? (a.olens ? min(max(a.olens[r], 0), a.owidth) : a.owidth) : 0;
    // vLLM skips the penalty step when every penalty is the identity; the result is the same
    const bool identity = (p.rep == 1.0f && p.pres == 0.0f && p.freq == 0.0f);
    p.tab = a.tstate != nullptr && !identity;
    p.trow = a.trows ? a.trows[r] : r;
    p.has_hist = p.tab || ((p.np > 0 || p.no > 0) && !identity);
    p.na = a.adj_ids ? (a.adjlens ? min(max(a.adjlens[r], 0), a.adjwidth) : a.adjwidth) : 0;
    p.need_hash = (p.has_hist && !p.tab) || p.na > 0;
    return p;
}

// The token-state word of token t in table row trow (prompt flag | output count).
__device__ __forceinline__ uint32_t state_word(const KArgs& a, int trow, int t) {
    return a.tstate[(size_t)trow * (size_t)a.tstride + (uint32_t)t] & kStateMask;
}

// The race's uniform of token t in row r: the caller's [B, V] uniforms, or the generated one
// (philox_uniform of the row's key and offset) when the caller passes keys instead, or one key
// for the launch (offset r).
__device__ __forceinline__ uint64_t row_rng_seed(const KArgs& a, int r) {
    return a.rng_seed ? a.rng_seed[r] : a.rng_key;
}
__device__ __forceinline__ uint64_t row_rng_offset(const KArgs& a, int r) {
    return a.rng_seed ? (a.rng_offset ? a.rng_offset[r] : 0ull) : (uint64_t)(uint32_t)r;
}
__device__ __forceinline__ float row_uniform(const KArgs& a, int r, int t) {
    if (a.u) return a.u[(size_t)r * a.ustride + t];
    return philox_uniform(row_rng_seed(a, r), row_rng_offset(a, r), (uint32_t)t);
}

// k served by the single-pass kernel for this row, or 0 when the row needs another path (top-k
// off or above kKMax; an allowed mask together with logprobs).  With raw logprobs the single
// pass keeps at least L candidates and finishes the logprobs from them (row_logprobs_entry);
// with an allowed mask it masks every element as it streams.
// CM: the kernel masks the candidates of its single pass (launches with an allowed mask and raw
// logprobs); no other kernel serves such a launch's rows on the single pass.
template <bool CM>
__device__ __forceinline__ int fast_k(const KArgs& a, const RowP& p) {
    if (!CM && a.allowed && a.L >= 0) return 0;
    if (p.greedy) return 1;
    if (p.k > 0 && p.k < a.V && p.k <= kKMax) return p.k;
    return 0;
}

// The race over the kept survivors and the diagnostics of the top-p cut.
struct RowRace {
    uint64_t best = 0;     // (key bits << 32) | (0x7FFFFFFF - index), 0 = none
    uint64_t last = 0;     // max (key(y) << 32 | index) over kept survivors
    uint64_t cprev = 0;    // largest cumulative mass among removed survivors
    uint64_t cat = ~0ull;  // smallest cumulative mass among kept survivors
    uint32_t second = 0;   // key bits + 1 of the best non-winning key, 0 = none
    uint32_t nkept = 0;
    uint32_t nrem = 0;     // survivors removed by top-p
    __device__ __forceinline__ void add_key(float key, int idx) {
        if (!(key >= 0.0f)) return;  // NaN keys never win
        const uint64_t pk = ((uint64_t)f2u(key) << 32) | (uint32_t)(0x7FFFFFFF - idx);
        if (pk > best) {
            if (best) { const uint32_t o = (uint32_t)(best >> 32) + 1u; second = second > o ? second : o; }
            best = pk;
        } else {
            const uint32_t o = f2u(key) + 1u;
            second = second > o ? second : o;
        }
    }
    __device__ __forceinline__ void merge(const RowRace& o) {
        const uint64_t hi = best > o.best ? best : o.best;
        const uint64_t lo = best > o.best ? o.best : best;
        const uint32_t l = lo ? (uint32_t)(lo >> 32) + 1u : 0u;
        second = second > o.second ? second : o.second;
        second = second > l ? second : l;
        best = hi;
        last = last > o.last ? last : o.last;
        cprev = cprev > o.cprev ? cprev : o.cprev;
        cat = cat < o.cat ? cat : o.cat;
        nkept += o.nkept;
        nrem += o.nrem;
    }
    __device__ __forceinline__ void shfl_merge(int off) {
        RowRace o;
        o.best = lane_xor64(best, off);
        o.last = lane_xor64(last, off);
        o.cprev = lane_xor64(cprev, off);
        o.cat = lane_xor64(cat, off);
        o.second = lane_xor(second, off);
        o.nkept = lane_xor(nkept, off);
        o.nrem = lane_xor(nrem, off);
        merge(o);
    }
};

}  // namespace vws
