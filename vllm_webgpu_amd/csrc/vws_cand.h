// vws_cand.h -- per-wave threshold-filtered candidate buffer (LDS) used to find the top-k of a
// streamed row slice in one pass.
//
// Each wave keeps (key, index) pairs of elements whose order key is >= its threshold tau.  When
// the buffer would overflow, the wave computes the exact k-th largest key of its buffer with a
// radix select, drops everything below it and raises tau to it.  Any wave's tau is a lower
// bound on the k-th largest value of the whole slice, so waves share the largest one through
// LDS (`shared_tau`) and filter with it too.  After the stream, the buffer holds every element
// of the wave's share that is >= the final threshold, which always includes its exact top-k
// with all ties at the k-th value.
#pragma once

#include "vws_device.h"

namespace vws {

struct CandBuf {
    uint32_t* ck;         // keys [cap]
    int32_t* ci;          // indices [cap]
    uint32_t* hist;       // 256 words of wave-private LDS for the radix select
    uint32_t* shared_tau; // LDS word shared by the workgroup (atomicMax)
    int cap;
    int k;
    int cnt;              // wave-uniform
    uint32_t tau;         // wave-uniform threshold key
    float tauf;           // value form of tau (-inf when tau admits every non-NaN)
    bool ovf;             // wave-uniform: capacity exceeded (ties)
    bool compacted;       // wave-uniform: at least one compaction dropped entries

    __device__ __forceinline__ void init(uint32_t* ck_, int32_t* ci_, uint32_t* hist_, uint32_t* st, int cap_,
                         int k_) {
        ck = ck_; ci = ci_; hist = hist_; shared_tau = st; cap = cap_; k = k_;
        cnt = 0; tau = 0; tauf = -__builtin_inff(); ovf = false; compacted = false;
    }

    __device__ __forceinline__ void set_tau(uint32_t t) {
        if (t > tau) {
            tau = t;
            tauf = (tau > 0x007FFFFFu) ? val_of(tau) : -__builtin_inff();
        }
    }

    // Picks up a higher threshold published by another wave.
    __device__ __forceinline__ void refresh() {
        const uint32_t st = __builtin_amdgcn_readfirstlane(__hip_atomic_load(shared_tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        set_tau(st);
    }

    // Keeps the exact top-k (with ties) of the buffer; wave-uniform call.
    __device__ __forceinline__ void compact() {
        if (cnt <= k) return;
        const int lane = lane_id();
        const uint32_t kth = wave_kth_largest(ck, cnt, k, hist);
        int out = 0;
        for (int base = 0; base < cnt; base += kWave) {
            const int i = base + lane;
            bool keep = false;
            uint32_t kk = 0;
            int32_t ii = 0;
            if (i < cnt) { kk = ck[i]; ii = ci[i]; keep = kk >= kth; }
            const uint64_t bal = wave_ballot(keep);
            if (keep) { const int pos = out + lane_prefix(bal); ck[pos] = kk; ci[pos] = ii; }
            out += __popcll(bal);
            wave_sync();
        }
        if (out < cnt) compacted = true;
        cnt = out;
        set_tau(kth);
        atomicMax(shared_tau, kth);
        wave_sync();
    }

    // Appends (kk, idx) from the lanes where c holds; wave-uniform call.  Callers pass
    // c = (value >= tauf) already (NaN values never pass).
    __device__ __forceinline__ void append(bool c, uint32_t kk, int32_t idx) {
        uint64_t bal = wave_ballot(c);
        if (!bal || ovf) return;
        int n = __popcll(bal);
        if (cnt + n > cap) {
            compact();
            c = c && kk >= tau;
            bal = wave_ballot(c);
            n = __popcll(bal);
            if (cnt + n > cap) { ovf = true; return; }
        }
        if (c) { const int pos = cnt + lane_prefix(bal); ck[pos] = kk; ci[pos] = idx; }
        cnt += n;
        wave_sync();
    }
};

// k-th largest key over the concatenation of nreg LDS regions (region w starts at
// base + w * stride and holds cnts[w] keys); one whole wave; requires 1 <= k <= total.
__device__ __forceinline__ uint32_t wave_kth_largest_multi(const uint32_t* base, int stride,
                                                           const int* cnts, int nreg, int k,
                                                           uint32_t* hist) {
    const int lane = lane_id();
    uint32_t prefix = 0, pmask = 0;
    uint32_t rem = (uint32_t)k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int b = lane; b < 256; b += kWave) hist[b] = 0;
        wave_sync();
        for (int w = 0; w < nreg; ++w) {
            const uint32_t* keys = base + (size_t)w * stride;
            const int n = cnts[w];
            for (int i = lane; i < n; i += kWave) {
                const uint32_t kk = keys[i];
                if ((kk & pmask) == prefix) atomicAdd(&hist[(kk >> shift) & 255u], 1u);
            }
        }
        wave_sync();
        const uint32_t c0 = hist[255 - 4 * lane], c1 = hist[254 - 4 * lane];
        const uint32_t c2 = hist[253 - 4 * lane], c3 = hist[252 - 4 * lane];
        const uint32_t s = c0 + c1 + c2 + c3;
        const uint32_t incl = wave_incl_scan(s);
        const uint32_t excl = incl - s;
        const uint64_t hit = wave_ballot(excl < rem && rem <= incl);
        const int L = __ffsll((unsigned long long)hit) - 1;
        uint32_t bin = 0, r = rem - excl;
        if (r <= c0) bin = 255 - 4 * lane;
        else if ((r -= c0) <= c1) bin = 254 - 4 * lane;
        else if ((r -= c1) <= c2) bin = 253 - 4 * lane;
        else { r -= c2; bin = 252 - 4 * lane; }
        bin = __builtin_amdgcn_readlane(bin, L);  // L is wave-uniform
        rem = __builtin_amdgcn_readlane(r, L);
        prefix |= bin << shift;
        pmask |= 255u << shift;
        wave_sync();
    }
    return prefix;
}

}  // namespace vws
