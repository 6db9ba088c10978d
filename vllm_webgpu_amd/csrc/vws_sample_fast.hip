// vws_sample_fast.hip -- single-pass split-row sampler for greedy rows and top-k rows (k <= 256),
// and the top-k operation.
//
// Grid: B' x S workgroups of 256 threads (B' = B rounded up to 8).  Workgroup b serves row r,
// part p: xcd = b % 8, slot = b / 8, p = slot % S, r = (slot / S) * 8 + xcd, so the parts of a
// row are dispatched to one XCD.  Each part streams its slice of the row once in 16-byte loads
// (8 in flight per lane) and keeps every element at or above a threshold in per-wave LDS
// candidate buffers.  The threshold starts from the first iteration's values (a 2-level
// histogram estimate of the slice's 4k-th largest) and rises when a buffer fills (exact radix
// select).  The part then publishes its exact top-k, all ties included, to the workspace.  The
// last part of a row to arrive (atomic counter) merges the S lists and finishes the row:
// temperature, min-p, top-k, top-p over exact integer masses, and the exponential race over the
// survivors' uniforms.  Rows it cannot finish exactly (tie overflow, too many survivors,
// non-finite max) are handed to the general kernel through row_state.
//
// Penalties: each part loads the history ids before its first logits and marks the tokens of
// its slice in an LDS hash (counts, prompt flag) and an LDS bitmap.  When no penalty can raise
// a logit (repetition >= 1, presence >= 0, frequency >= 0), a history element can only be a
// candidate if its raw value passes the threshold, so candidates at marked positions are
// penalised on the spot and tested again.  Otherwise the part gathers the raw logits of its
// history tokens up front, seeds the buffers with the penalised values and skips marked
// positions in the stream.
#include "vws_cand.h"
#include "vws_internal.h"
#include "vws_row.h"

namespace vws {

constexpr int kBitmapWordsFast = kPartMax / 32;
constexpr int kSpec = 64;  // list entries per part read speculatively with the metas

struct FastSmem {
    uint32_t ckey[kFastWaves][kCapW];  // candidate keys (also: seed histograms, merged keys)
    int32_t cidx[kFastWaves][kCapW];   // candidate indices (also: merged indices)
    uint32_t hist[kFastWaves][256];    // per-wave radix-select scratch
    union {
        struct {
            uint32_t key[kHashSlots];  // token + 1, 0 = empty
            uint32_t val[kHashSlots];  // output count | prompt flag << 31
            float pen[kHashSlots];     // penalised value (gather path)
            uint32_t bits[kBitmapWordsFast];
        } h;
        struct {
            float u[kMergeCap];        // uniforms of the merged candidates
            uint32_t ky[kKeepCap];     // survivors: key(y), index, race key, mass
            int32_t idx[kKeepCap];
            float rk[kKeepCap];
            uint64_t w[kKeepCap];
        } k;
    } u;
    uint64_t red[kFastWaves][8];
    uint32_t tau;
    uint32_t status;
    uint32_t nhash;
    uint32_t outcnt;
    uint32_t kth_part;
    uint32_t last;
    uint32_t nkeep;
    uint32_t maxkey;
    int cnt[kFastWaves];
    uint32_t pcnt[kMaxParts];
    uint32_t pkth[kMaxParts];
    uint32_t poff[kMaxParts + 1];
    uint32_t bcast[8];
};

// Cross-workgroup hand-off of the part lists.  Stores and loads are agent-scope atomics, which
// the memory model makes coherent across XCD L2s without whole-cache writeback/invalidate; the
// arrival counter is incremented only after every store of the workgroup has completed
// (s_waitcnt), so the last arriver, which reads with agent-scope atomic loads after seeing the
// final count, observes all lists.
__device__ __forceinline__ void publish_u32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t fetch_u32(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t fetch_u64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stores_complete() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ uint32_t fast_hash(int t) {
    return ((uint32_t)t * 2654435761u) >> (32 - 10);  // kHashSlots = 1024
}

// Inserts history token t (count increment, or the prompt bit) and marks it in the bitmap.
__device__ __forceinline__ void fhash_insert(FastSmem& sm, int t, int lo, uint32_t inc) {
    uint32_t s = fast_hash(t);
    for (int probe = 0; probe < kHashSlots; ++probe) {
        const uint32_t prev = atomicCAS(&sm.u.h.key[s], 0u, (uint32_t)t + 1u);
        if (prev == 0u) {
            if (atomicAdd(&sm.nhash, 1u) >= (uint32_t)kHashFill) atomicOr(&sm.status, 1u);
            atomicOr(&sm.u.h.bits[(t - lo) >> 5], 1u << ((t - lo) & 31));
        }
        if (prev == 0u || prev == (uint32_t)t + 1u) {
            if (inc & 0x80000000u) atomicOr(&sm.u.h.val[s], 0x80000000u);
            else atomicAdd(&sm.u.h.val[s], inc);
            return;
        }
        s = (s + 1u) & (kHashSlots - 1);
    }
    atomicOr(&sm.status, 1u);
}

// count | prompt << 31 of history token t (0 if absent)
__device__ __forceinline__ uint32_t fhash_value(const FastSmem& sm, int t) {
    uint32_t s = fast_hash(t);
    for (int probe = 0; probe < kHashSlots; ++probe) {
        const uint32_t k = sm.u.h.key[s];
        if (k == (uint32_t)t + 1u) return sm.u.h.val[s];
        if (k == 0u) return 0u;
        s = (s + 1u) & (kHashSlots - 1);
    }
    return 0u;
}

__device__ __forceinline__ bool fbit(const FastSmem& sm, int i, int lo) {
    return (sm.u.h.bits[(i - lo) >> 5] >> ((i - lo) & 31)) & 1u;
}

template <typename T>
__device__ __forceinline__ int body_index(const Slice<T>& sl, int vi) {
    return sl.a + vi * Elem<T>::kVec;
}

// ---- block reductions for 256 threads ----------------------------------------------------

__device__ __forceinline__ uint64_t fblock_max(uint64_t v, FastSmem& sm) {
    v = wave_max_u64(v);
    __syncthreads();
    if (lane_id() == 0) sm.red[threadIdx.x >> 6][0] = v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < kFastWaves; ++i) t = t > sm.red[i][0] ? t : sm.red[i][0];
    return t;
}

__device__ __forceinline__ uint64_t fblock_sum(uint64_t v, FastSmem& sm) {
    v = wave_sum_u64(v);
    __syncthreads();
    if (lane_id() == 0) sm.red[threadIdx.x >> 6][0] = v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < kFastWaves; ++i) t += sm.red[i][0];
    return t;
}

// The race over a set of kept tokens: the best (key bits << 32 | 0x7FFFFFFF - index), the best
// key among the others (bits + 1, 0 = none), and the diagnostics of the top-p cut.
struct RaceSum {
    uint64_t best = 0, last = 0, cprev = 0, cat = ~0ull;
    uint32_t second = 0, nkept = 0, nrem = 0;
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
    __device__ __forceinline__ void merge(const RaceSum& o) {
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
        RaceSum o;
        o.best = __shfl_xor(best, off, kWave);
        o.last = __shfl_xor(last, off, kWave);
        o.cprev = __shfl_xor(cprev, off, kWave);
        o.cat = __shfl_xor(cat, off, kWave);
        o.second = __shfl_xor(second, off, kWave);
        o.nkept = __shfl_xor(nkept, off, kWave);
        o.nrem = __shfl_xor(nrem, off, kWave);
        merge(o);
    }
};

// ---- the part: stream a slice, publish its top-k list -----------------------------------

template <typename T>
__device__ __forceinline__ void fast_stream_part(const KArgs& a, FastSmem& sm, int r, int p,
                                                 const RowP& prm, int k) {
    constexpr int NT = kFastThreads;
    constexpr int VEC = Elem<T>::kVec;
    constexpr int U = 32 / VEC;  // 16-byte loads in flight per lane per iteration
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const T* row = reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride;
    const int lo = p * a.part_len;
    const int hi = min(a.V, lo + a.part_len);
    const bool hh = prm.has_hist;
    // penalties that never raise a logit let history candidates be found by their raw value
    const bool mono = prm.rep >= 1.0f && prm.pres >= 0.0f && prm.freq >= 0.0f;
    const bool gather = hh && !mono;

    // 1. history ids (first two per thread), then the first iteration of logits
    int hp0 = -1, hp1 = -1, ho0 = -1, ho1 = -1;
    if (hh) {
        const int32_t* pr = a.prompt + (size_t)r * a.pstride;
        const int32_t* ou = a.output + (size_t)r * a.ostride;
        if (tid < prm.np) hp0 = pr[tid];
        if (NT + tid < prm.np) hp1 = pr[NT + tid];
        if (tid < prm.no) ho0 = ou[tid];
        if (NT + tid < prm.no) ho1 = ou[NT + tid];
    }
    Slice<T> sl;
    sl.init(row, lo, hi);
    const int nbody = sl.nbody;
    const int bend = sl.body_end();
    const int nit = (nbody + NT * U - 1) / (NT * U);
    float A[U][VEC], Bq[U][VEC];
    if (nbody > 0) {
#pragma unroll
        for (int q = 0; q < U; ++q) sl.load_body(q * NT + tid, A[q]);
    }
    if (nit > 1) {  // the second iteration stays in flight while the seed is computed
#pragma unroll
        for (int q = 0; q < U; ++q) sl.load_body((U + q) * NT + tid, Bq[q]);
    }

    // 2. clear LDS state
    if (tid == 0) { sm.tau = 0; sm.status = 0; sm.nhash = 0; sm.outcnt = 0; sm.bcast[7] = 0; }
    uint32_t* bins = &sm.ckey[0][0];  // seed histograms (2048 + 256 bins)
    for (int b = tid; b < 2048 + 256; b += NT) bins[b] = 0u;
    if (hh) {
        for (int s = tid; s < kHashSlots; s += NT) { sm.u.h.key[s] = 0; sm.u.h.val[s] = 0; }
        for (int s = tid; s < kBitmapWordsFast; s += NT) sm.u.h.bits[s] = 0;
    }
    __syncthreads();

    // 3. history of this slice -> LDS hash + bitmap
    if (hh) {
        if (hp0 >= lo && hp0 < hi) fhash_insert(sm, hp0, lo, 0x80000000u);
        if (hp1 >= lo && hp1 < hi) fhash_insert(sm, hp1, lo, 0x80000000u);
        if (ho0 >= lo && ho0 < hi) fhash_insert(sm, ho0, lo, 1u);
        if (ho1 >= lo && ho1 < hi) fhash_insert(sm, ho1, lo, 1u);
        const int32_t* pr = a.prompt + (size_t)r * a.pstride;
        const int32_t* ou = a.output + (size_t)r * a.ostride;
        for (int i = 2 * NT + tid; i < prm.np; i += NT) {
            const int t = pr[i];
            if (t >= lo && t < hi) fhash_insert(sm, t, lo, 0x80000000u);
        }
        for (int i = 2 * NT + tid; i < prm.no; i += NT) {
            const int t = ou[i];
            if (t >= lo && t < hi) fhash_insert(sm, t, lo, 1u);
        }
    }

    // 4. seed threshold: lower edge of the key range (11 + 8 bits) holding the `want`-th largest
    //    value of the first iteration; `want` is chosen so that about 4k elements of the slice
    //    are expected above it.  It only saves work: with fewer than k candidates above it at
    //    the end, the slice is streamed again without it.
    const int sample = nbody > 0 ? min(NT * U * VEC, bend - sl.a) : 0;
    const int want = sample > 0 ? (int)(((int64_t)4 * k * sample + (hi - lo) - 1) / (hi - lo)) + 1 : 1;
    const bool seeded = nbody > 0 && want <= sample;
    if (seeded) {
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const int i0 = body_index(sl, q * NT + tid);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const uint32_t kk = key_of(A[q][j]);
                if (kk && i0 + j < bend) atomicAdd(&bins[kk >> 21], 1u);
            }
        }
    }
    __syncthreads();
    if (seeded) {
        // level 1: 2048 bins, 8 per thread, scanned from the top bucket down
        uint32_t c[8], tot = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) { c[i] = bins[2047 - (tid * 8 + i)]; tot += c[i]; }
        const uint32_t incl = wave_incl_scan(tot);
        if (lane == 63) sm.bcast[wave] = incl;
        __syncthreads();
        uint32_t run = incl - tot;
        for (int w = 0; w < wave; ++w) run += sm.bcast[w];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t before = run;
            run += c[i];
            if (before < (uint32_t)want && run >= (uint32_t)want) {
                sm.bcast[4] = (uint32_t)(2047 - (tid * 8 + i));
                sm.bcast[5] = (uint32_t)want - before;  // rank inside that bin
            }
        }
        __syncthreads();
        const uint32_t b1 = sm.bcast[4];
        // level 2: the next 8 key bits inside bin b1
        uint32_t* bins2 = bins + 2048;
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const int i0 = body_index(sl, q * NT + tid);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const uint32_t kk = key_of(A[q][j]);
                if (kk && i0 + j < bend && (kk >> 21) == b1) atomicAdd(&bins2[(kk >> 13) & 255u], 1u);
            }
        }
        __syncthreads();
        if (wave == 0) {
            const uint32_t rem = sm.bcast[5];
            const uint32_t c0 = bins2[255 - 4 * lane], c1 = bins2[254 - 4 * lane];
            const uint32_t c2 = bins2[253 - 4 * lane], c3 = bins2[252 - 4 * lane];
            const uint32_t s4 = c0 + c1 + c2 + c3;
            const uint32_t inc4 = wave_incl_scan(s4);
            const uint32_t exc4 = inc4 - s4;
            if (exc4 < rem && rem <= inc4) {
                uint32_t rr = rem - exc4, bin;
                if (rr <= c0) bin = 255 - 4 * lane;
                else if ((rr -= c0) <= c1) bin = 254 - 4 * lane;
                else if ((rr -= c1) <= c2) bin = 253 - 4 * lane;
                else bin = 252 - 4 * lane;
                sm.bcast[7] = (b1 << 21) | (bin << 13);
            }
        }
    }
    __syncthreads();
    const uint32_t seed = seeded ? sm.bcast[7] : 0u;

    // 5. gather path for penalties that may raise a logit: penalised values seed the buffers
    if (gather) {
        for (int s = tid; s < kHashSlots; s += NT) {
            const uint32_t kk = sm.u.h.key[s];
            if (kk) {
                const int t = (int)kk - 1;
                const uint32_t v = sm.u.h.val[s];
                sm.u.h.pen[s] = apply_penalty(Elem<T>::load1(row + t), (v >> 31) != 0u,
                                              v & 0x7FFFFFFFu, prm.rep, prm.inv_rep, prm.freq,
                                              prm.pres);
            }
        }
    }
    for (int b = tid; b < 2048 + 256; b += NT) bins[b] = 0u;  // the buffers reuse this LDS
    __syncthreads();

    CandBuf cb;
    // candidate test of one element (wave-uniform call)
    auto slot = [&](float v, int idx, bool valid) __attribute__((always_inline)) {
        bool c = valid && v >= cb.tauf;
        if (wave_ballot(c) == 0ull) return;
        if (hh) {
            const bool hit = c && fbit(sm, idx, lo);
            if (wave_ballot(hit) != 0ull) {
                if (gather) {
                    c = c && !hit;
                } else if (hit) {
                    const uint32_t hv = fhash_value(sm, idx);
                    v = apply_penalty(v, (hv >> 31) != 0u, hv & 0x7FFFFFFFu, prm.rep, prm.inv_rep,
                                      prm.freq, prm.pres);
                    c = v >= cb.tauf;
                }
            }
        }
        cb.append(c, key_of(v), idx);
    };
    auto run_stream = [&](uint32_t seed_tau) __attribute__((always_inline)) {
        cb.init(sm.ckey[wave], sm.cidx[wave], sm.hist[wave], &sm.tau, kCapW, k);
        cb.set_tau(seed_tau);
        if (gather && sm.status == 0u) {
            constexpr int per = kHashSlots / kFastWaves;
            for (int s0 = wave * per; s0 < (wave + 1) * per; s0 += 64) {
                const int s = s0 + lane;
                const uint32_t kk = sm.u.h.key[s];
                const uint32_t pk = kk ? key_of(sm.u.h.pen[s]) : 0u;
                cb.append(pk != 0u && pk >= cb.tau, pk, (int32_t)kk - 1);
            }
        }
        if (sm.status != 0u) return;
        {   // unaligned head (thread 0) and tail (thread 1): fewer than 2 vectors in total
            float v[VEC];
            const int i0 = sl.load_edge(tid == 1 ? 1 : 0, v);
            const int end = tid == 0 ? sl.a : hi;
#pragma unroll
            for (int j = 0; j < VEC; ++j) slot(v[j], i0 + j, tid <= 1 && i0 + j < end);
        }
        auto examine = [&](float (&buf)[U][VEC], int it) __attribute__((always_inline)) {
            cb.refresh();
            bool any = false;
#pragma unroll
            for (int q = 0; q < U; ++q)
#pragma unroll
                for (int j = 0; j < VEC; ++j) any |= (buf[q][j] >= cb.tauf);
            if (wave_ballot(any) != 0ull) {
#pragma unroll
                for (int q = 0; q < U; ++q) {
                    const int i0 = body_index(sl, (it * U + q) * NT + tid);
                    const bool ok = i0 < bend;
#pragma unroll
                    for (int j = 0; j < VEC; ++j) slot(buf[q][j], i0 + j, ok);
                }
            }
        };
        if (nit > 0) examine(A, 0);
        if (nit > 1 && !cb.ovf) examine(Bq, 1);
        for (int it = 2; it < nit && !cb.ovf; ++it) {
#pragma unroll
            for (int q = 0; q < U; ++q) sl.load_body((it * U + q) * NT + tid, A[q]);
            examine(A, it);
        }
    };
    run_stream(seed);
    if (lane == 0) sm.cnt[wave] = cb.ovf ? (1 << 28) : cb.cnt;
    __syncthreads();
    uint32_t seed_used = seed;
    if (seed != 0u && sm.status == 0u) {
        int total = 0;
#pragma unroll
        for (int w = 0; w < kFastWaves; ++w) total += sm.cnt[w];
        if (total < k) {
            // fewer than k candidates above the seed: stream the slice again without it
            __syncthreads();
            if (tid == 0) sm.tau = 0u;
            __syncthreads();
            if (nbody > 0) {
#pragma unroll
                for (int q = 0; q < U; ++q) sl.load_body(q * NT + tid, A[q]);
            }
            if (nit > 1) {
#pragma unroll
                for (int q = 0; q < U; ++q) sl.load_body((U + q) * NT + tid, Bq[q]);
            }
            run_stream(0u);
            seed_used = 0u;
            if (lane == 0) sm.cnt[wave] = cb.ovf ? (1 << 28) : cb.cnt;
            __syncthreads();
        }
    }

    // 6. the part's exact top-k (all ties) -> workspace.  Elements left out are below `excl`:
    //    with more than k candidates that is the k-th largest candidate; otherwise the largest
    //    threshold any wave filtered with (0 when nothing was filtered).
    int total = 0;
#pragma unroll
    for (int w = 0; w < kFastWaves; ++w) total += sm.cnt[w];
    if (total >= (1 << 28)) atomicOr(&sm.status, 2u);
    __syncthreads();
    const size_t pm = ((size_t)r * kMaxParts + p) * 4;
    if (sm.status == 0u) {
        if (wave == 0) {
            uint32_t kth = 0;
            if (total > k && total <= 256) {
                uint32_t v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {  // element e of the concatenated wave buffers
                    int e = 4 * lane + i, w = 0;
                    while (w < kFastWaves && e >= sm.cnt[w]) { e -= sm.cnt[w]; ++w; }
                    v[i] = w < kFastWaves ? sm.ckey[w][e] : 0u;
                }
                kth = wave_kth_largest_256(v[0], v[1], v[2], v[3], k);
            } else if (total > k) {
                kth = wave_kth_largest_multi(&sm.ckey[0][0], kCapW, sm.cnt, kFastWaves, k, sm.hist[0]);
            }
            if (lane == 0) sm.kth_part = kth;
        }
        __syncthreads();
        const uint32_t kth = sm.kth_part;
        const uint32_t st = sm.tau;
        const uint32_t excl = total > k ? kth : (seed_used > st ? seed_used : st);
        uint2* out = a.part_list + ((size_t)r * kMaxParts + p) * kPartCap;
        for (int base = 0; base < cb.cnt; base += 64) {
            const int i = base + lane;
            const bool keep = i < cb.cnt && cb.ck[i] >= kth;
            const uint64_t bal = wave_ballot(keep);
            uint32_t off = 0;
            if (lane == 0 && bal) off = atomicAdd(&sm.outcnt, (uint32_t)__popcll(bal));
            off = __shfl(off, 0, 64);
            if (keep) {
                const uint32_t pos = off + (uint32_t)lane_prefix(bal);
                if (pos < (uint32_t)kPartCap) {
                    const uint64_t e = ((uint64_t)(uint32_t)cb.ci[i] << 32) | cb.ck[i];
                    __hip_atomic_store(reinterpret_cast<uint64_t*>(out + pos), e, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        __syncthreads();
        if (tid == 0) {
            const uint32_t n = sm.outcnt;
            publish_u32(&a.part_meta[pm + 0], n);
            publish_u32(&a.part_meta[pm + 1], excl);
            publish_u32(&a.part_meta[pm + 2], (n > (uint32_t)kPartCap) ? 1u : 0u);
        }
    } else if (tid == 0) {
        publish_u32(&a.part_meta[pm + 0], 0u);
        publish_u32(&a.part_meta[pm + 1], 0u);
        publish_u32(&a.part_meta[pm + 2], 1u);
    }
}

// ---- the last part: merge and finish the row -------------------------------------------

__device__ __forceinline__ void fast_hand_to_general(const KArgs& a, int r) {
    if (threadIdx.x == 0) a.row_state[r] = kRowNeedsGeneral;
}

template <typename T>
__device__ __forceinline__ void fast_finish_row(const KArgs& a, FastSmem& sm, int r,
                                                const RowP& prm, int k) {
    constexpr int NT = kFastThreads;
    constexpr int NSPEC = (kMaxParts * kSpec) / NT;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int S = a.S;
    uint32_t* mk = &sm.ckey[0][0];
    int32_t* mi = &sm.cidx[0][0];

    // metas and the first kSpec entries of every list in one round trip
    uint64_t spec[NSPEC];
#pragma unroll
    for (int s = 0; s < NSPEC; ++s) {
        const int e = s * NT + tid, pp = e / kSpec, i = e % kSpec;
        spec[s] = pp < S ? fetch_u64(reinterpret_cast<const uint64_t*>(
                               a.part_list + ((size_t)r * kMaxParts + pp) * kPartCap + i))
                         : 0ull;
    }
    if (tid == 0) { sm.status = 0; sm.maxkey = 0; sm.nkeep = 0; }
    __syncthreads();
    if (tid < S) {
        const size_t pm = ((size_t)r * kMaxParts + tid) * 4;
        sm.pcnt[tid] = fetch_u32(&a.part_meta[pm + 0]);
        sm.pkth[tid] = fetch_u32(&a.part_meta[pm + 1]);
        if (fetch_u32(&a.part_meta[pm + 2])) atomicOr(&sm.status, 4u);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t off = 0;
        for (int pp = 0; pp < S; ++pp) { sm.poff[pp] = off; off += sm.pcnt[pp]; }
        sm.poff[S] = off;
        if (off > (uint32_t)kMergeCap) sm.status |= 8u;
    }
    __syncthreads();
    if (sm.status) { fast_hand_to_general(a, r); return; }
    const int N = (int)sm.poff[S];
    uint32_t mx = 0;
#pragma unroll
    for (int s = 0; s < NSPEC; ++s) {
        const int e = s * NT + tid, pp = e / kSpec, i = e % kSpec;
        if (pp < S && i < (int)sm.pcnt[pp]) {
            const int o = (int)sm.poff[pp] + i;
            mk[o] = (uint32_t)spec[s];
            mi[o] = (int32_t)(uint32_t)(spec[s] >> 32);
            mx = mx > (uint32_t)spec[s] ? mx : (uint32_t)spec[s];
        }
    }
    for (int pp = 0; pp < S; ++pp) {  // lists longer than the speculative window
        const int n = (int)sm.pcnt[pp];
        if (n <= kSpec) continue;
        const uint2* src = a.part_list + ((size_t)r * kMaxParts + pp) * kPartCap;
        for (int i = kSpec + tid; i < n; i += NT) {
            const uint64_t e = fetch_u64(reinterpret_cast<const uint64_t*>(src + i));
            const int o = (int)sm.poff[pp] + i;
            mk[o] = (uint32_t)e;
            mi[o] = (int32_t)(uint32_t)(e >> 32);
            mx = mx > (uint32_t)e ? mx : (uint32_t)e;
        }
    }
    mx = wave_max_u32(mx);
    if (lane == 0) atomicMax(&sm.maxkey, mx);
    __syncthreads();

    if (a.mode == kModeTopK) {
        // ids/values of the k largest, ordered (value desc, index asc)
        if (wave == 0) {
            const uint32_t kth = (N >= k) ? wave_kth_largest(mk, N, k, sm.hist[0]) : 0u;
            if (lane == 0) sm.bcast[0] = kth;
        }
        __syncthreads();
        const uint32_t kth = sm.bcast[0];
        for (int j = tid; j < k; j += NT) {
            a.topk_vals[(size_t)r * k + j] = __builtin_nanf("");
            a.topk_ids[(size_t)r * k + j] = -1;
        }
        __syncthreads();
        for (int j = tid; j < N; j += NT) {
            const uint32_t kj = mk[j];
            if (kj < kth || kj == 0u) continue;
            const int32_t ij = mi[j];
            int rank = 0;
            for (int i = 0; i < N; ++i) {
                const uint32_t ki = mk[i];
                rank += (ki >= kth && ki != 0u && (ki > kj || (ki == kj && mi[i] < ij))) ? 1 : 0;
            }
            if (rank < k) {
                a.topk_vals[(size_t)r * k + rank] = val_of(kj);
                a.topk_ids[(size_t)r * k + rank] = ij;
            }
        }
        return;
    }

    if (prm.greedy) {
        // max key, lowest index
        uint64_t best = 0;
        for (int j = tid; j < N; j += NT) {
            const uint64_t pk = ((uint64_t)mk[j] << 32) | (uint32_t)(0x7FFFFFFF - mi[j]);
            best = best > pk ? best : pk;
        }
        best = fblock_max(best, sm);
        if (tid == 0) {
            const int32_t tok = (best >> 32) ? (int32_t)(0x7FFFFFFF - (uint32_t)(best & 0xFFFFFFFFu)) : 0;
            a.sampled[r] = tok;
            if (a.flags) a.flags[r] = VWS_FLAG_GREEDY;
            if (a.nkept) a.nkept[r] = 1;
        }
        return;
    }

    // uniforms of every merged candidate: issued now, consumed after the k-th value select
    constexpr int NU = kMergeCap / NT;
    float ureg[NU];
#pragma unroll
    for (int s = 0; s < NU; ++s) {
        const int j = s * NT + tid;
        ureg[s] = j < N ? row_uniform(a, r, mi[j]) : 0.5f;
    }

    const float Tt = prm.T;
    if (wave == 0) {
        uint32_t kth = 0;
        if (N >= k && N <= 256) {
            uint32_t v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = 4 * lane + i < N ? mk[4 * lane + i] : 0u;
            kth = wave_kth_largest_256(v[0], v[1], v[2], v[3], k);
        } else if (N >= k) {
            kth = wave_kth_largest(mk, N, k, sm.hist[0]);
        }
        if (lane == 0) sm.bcast[0] = kth;
    }
#pragma unroll
    for (int s = 0; s < NU; ++s) {
        const int j = s * NT + tid;
        if (j < N) sm.u.k.u[j] = ureg[s];
    }
    __syncthreads();
    const uint32_t kth = sm.bcast[0];
    const uint32_t mxk = sm.maxkey;
    const float kth_y = kth ? val_of(kth) / Tt : -__builtin_inff();
    const float m = mxk ? val_of(mxk) / Tt : __builtin_nanf("");
    bool bad = !(m > -__builtin_inff() && m < __builtin_inff());
    for (int pp = 0; pp < S; ++pp) {
        const uint32_t kp = sm.pkth[pp];
        if (kp > 0x007FFFFFu && val_of(kp - 1u) / Tt >= kth_y) bad = true;
    }
    if (bad) { fast_hand_to_general(a, r); return; }

    // survivors of temperature + top-k + min-p, with their masses and race keys
    const float lp_min = (prm.min_p > 0.0f) ? log_det(prm.min_p < 1.0f ? prm.min_p : 1.0f)
                                            : -__builtin_inff();
    uint64_t wsum = 0;
    for (int base = 0; base < N; base += NT) {
        const int j = base + tid;
        float y = 0.0f;
        bool keep = false;
        if (j < N) {
            y = val_of(mk[j]) / Tt;
            keep = key_of(y) != 0u && y >= kth_y && (y - m) >= lp_min;
        }
        const uint64_t bal = wave_ballot(keep);
        uint32_t off = 0;
        if (lane == 0 && bal) off = atomicAdd(&sm.nkeep, (uint32_t)__popcll(bal));
        off = __shfl(off, 0, 64);
        if (keep) {
            const uint32_t pos = off + (uint32_t)lane_prefix(bal);
            if (pos < (uint32_t)kKeepCap) {
                const float e = exp_det(y - m);
                const uint64_t w = mass_of(e);
                sm.u.k.ky[pos] = key_of(y);
                sm.u.k.idx[pos] = mi[j];
                sm.u.k.rk[pos] = e / (0.0f - log_det(sm.u.k.u[j]));
                sm.u.k.w[pos] = w;
                wsum += w;
            }
        }
    }
    const uint64_t W = fblock_sum(wsum, sm);  // its barriers also publish nkeep
    const int n = (int)sm.nkeep;
    if (n > kKeepCap) { fast_hand_to_general(a, r); return; }

    // top-p over exact masses: C_j = sum of w_i over i <= j in (y asc, index asc)
    const float q32 = 1.0f - prm.top_p;
    const bool topp = q32 > 0.0f;
    const bool abl = topp && !(q32 < 1.0f);
    const uint64_t thr = (topp && !abl) ? scale_floor(q32, W) : 0ull;
    RaceSum rs;
    for (int j = tid; j < n; j += NT) {
        const uint32_t kj = sm.u.k.ky[j];
        const int32_t ij = sm.u.k.idx[j];
        bool removed = false;
        uint64_t C = 0;
        if (topp) {
            for (int i = 0; i < n; ++i) {
                const uint32_t ki = sm.u.k.ky[i];
                if (ki < kj || (ki == kj && sm.u.k.idx[i] <= ij)) C += sm.u.k.w[i];
            }
            removed = abl ? (C != W) : (C <= thr && C != W);
        }
        if (removed) {
            rs.nrem++;
            rs.cprev = rs.cprev > C ? rs.cprev : C;
            continue;
        }
        rs.cat = rs.cat < C ? rs.cat : C;
        rs.nkept++;
        const uint64_t lk = ((uint64_t)kj << 32) | (uint32_t)ij;
        rs.last = rs.last > lk ? rs.last : lk;
        rs.add_key(sm.u.k.rk[j], ij);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) rs.shfl_merge(off);
    __syncthreads();
    if (lane == 0) {
        sm.red[wave][0] = rs.best; sm.red[wave][1] = rs.last; sm.red[wave][2] = rs.cprev;
        sm.red[wave][3] = rs.cat; sm.red[wave][4] = rs.second; sm.red[wave][5] = rs.nkept;
        sm.red[wave][6] = rs.nrem;
    }
    __syncthreads();
    if (tid == 0) {
        RaceSum t;
        for (int w = 0; w < kFastWaves; ++w) {
            RaceSum o;
            o.best = sm.red[w][0]; o.last = sm.red[w][1]; o.cprev = sm.red[w][2]; o.cat = sm.red[w][3];
            o.second = (uint32_t)sm.red[w][4]; o.nkept = (uint32_t)sm.red[w][5];
            o.nrem = (uint32_t)sm.red[w][6];
            t.merge(o);
        }
        int32_t tok;
        uint32_t fl = 0;
        if (t.best) {
            tok = (int32_t)(0x7FFFFFFF - (uint32_t)(t.best & 0xFFFFFFFFu));
            const float bk = u2f((uint32_t)(t.best >> 32));
            if (t.second) {
                const float sk = u2f(t.second - 1u);
                if ((double)sk >= (double)bk * (1.0 - 1e-6)) fl |= VWS_FLAG_RACE_NEAR_TIE;
            }
        } else {
            tok = (int32_t)(uint32_t)(t.last & 0xFFFFFFFFu);
        }
        if (topp && !abl) {
            const uint64_t tol = (uint64_t)((double)W * 1e-6);
            if ((t.nrem > 0 && thr - t.cprev <= tol) || (t.cat > thr && t.cat - thr <= tol))
                fl |= VWS_FLAG_TOPP_NEAR_TIE;
        }
        a.sampled[r] = tok;
        if (a.flags) a.flags[r] = fl;
        if (a.nkept) a.nkept[r] = (int32_t)t.nkept;
    }
}

template <typename T>
__global__ __launch_bounds__(kFastThreads) void fast_kernel(KArgs a) {
    __shared__ FastSmem sm;
    const int b = blockIdx.x;
    const int xcd = b & 7, slot = b >> 3;
    const int p = slot % a.S;
    const int r = (slot / a.S) * 8 + xcd;
    if (r >= a.B) return;
    const RowP prm = row_params(a, r);
    const int k = fast_k(a, prm);
    if (k == 0) return;
    fast_stream_part<T>(a, sm, r, p, prm, k);
    stores_complete();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&a.row_counter[r], 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        sm.last = (prev == (uint32_t)(a.S - 1)) ? 1u : 0u;
    }
    __syncthreads();
    if (!sm.last) return;
    if (threadIdx.x == 0) publish_u32(&a.row_counter[r], 0u);
    fast_finish_row<T>(a, sm, r, prm, k);
}

template __global__ void fast_kernel<float>(KArgs);
template __global__ void fast_kernel<uint16_t>(KArgs);
template __global__ void fast_kernel<_Float16>(KArgs);

}  // namespace vws
