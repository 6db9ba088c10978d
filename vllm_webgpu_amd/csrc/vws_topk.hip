// vws_topk.hip -- the top-k operation (vws_topk): the exact k <= 256 largest values of each row
// and their ids, ordered (value desc, id asc), split over several workgroups per row.
//
// Grid: B' x S workgroups of 256 threads (B' = B rounded up to 8).  Workgroup b serves row r,
// part p: xcd = b % 8, slot = b / 8, p = slot % S, r = (slot / S) * 8 + xcd, so the parts of a
// row are dispatched to one XCD.  Each part streams its slice of the row once in 16-byte loads
// (8 in flight per lane) and keeps every element at or above a threshold in per-wave LDS
// candidate buffers.  The threshold starts from the first iteration's values (a 2-level
// histogram estimate of the slice's 4k-th largest) and rises when a buffer fills (exact radix
// select).  The part then publishes its exact top-k, all ties included, to the workspace.  The
// last part of a row to arrive (atomic counter) merges the S lists and writes the row's top k.
// Rows it cannot finish (a list past its capacity: ties) are handed to general_kernel, which
// selects them exactly with the multi-pass path's radix select.
#include "vws_cand.h"
#include "vws_general.h"
#include "vws_internal.h"
#include "vws_row.h"

namespace vws {

constexpr int kSpec = 64;  // list entries per part read speculatively with the metas

struct FastSmem {
    uint32_t ckey[kFastWaves][kCapW];  // candidate keys (also: seed histograms, merged keys)
    int32_t cidx[kFastWaves][kCapW];   // candidate indices (also: merged indices)
    uint32_t hist[kFastWaves][256];    // per-wave radix-select scratch
    uint32_t tau;
    uint32_t status;
    uint32_t outcnt;
    uint32_t kth_part;
    uint32_t last;
    int cnt[kFastWaves];
    uint32_t pcnt[kMaxParts];
    uint32_t poff[kMaxParts + 1];
    uint32_t bcast[8];
};

// Cross-workgroup hand-off of the part lists: agent-scope atomic stores and loads (ag_*); the
// arrival counter is incremented only after every store of the workgroup has completed, so the
// last arriver, which reads after seeing the final count, observes all lists.

template <typename T>
__device__ __forceinline__ int body_index(const Slice<T>& sl, int vi) {
    return sl.a + vi * Elem<T>::kVec;
}

// ---- the part: stream a slice, publish its top-k list -----------------------------------

template <typename T>
__device__ __forceinline__ void fast_stream_part(const KArgs& a, FastSmem& sm, int r, int p, int k) {
    constexpr int NT = kFastThreads;
    constexpr int VEC = Elem<T>::kVec;
    constexpr int U = 32 / VEC;  // 16-byte loads in flight per lane per iteration
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const T* row = reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride;
    const int lo = p * a.part_len;
    const int hi = min(a.V, lo + a.part_len);

    // 1. the first two iterations of logits
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
    if (tid == 0) { sm.tau = 0; sm.status = 0; sm.outcnt = 0; sm.bcast[7] = 0; }
    uint32_t* bins = &sm.ckey[0][0];  // seed histograms (2048 + 256 bins)
    for (int b = tid; b < 2048 + 256; b += NT) bins[b] = 0u;
    __syncthreads();

    // 3. seed threshold: lower edge of the key range (11 + 8 bits) holding the `want`-th largest
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

    for (int b = tid; b < 2048 + 256; b += NT) bins[b] = 0u;  // the buffers reuse this LDS
    __syncthreads();

    CandBuf cb;
    // candidate test of one element (wave-uniform call)
    auto slot = [&](float v, int idx, bool valid) __attribute__((always_inline)) {
        const bool c = valid && v >= cb.tauf;
        if (wave_ballot(c) == 0ull) return;
        cb.append(c, key_of(v), idx);
    };
    auto run_stream = [&](uint32_t seed_tau) __attribute__((always_inline)) {
        cb.init(sm.ckey[wave], sm.cidx[wave], sm.hist[wave], &sm.tau, kCapW, k);
        cb.set_tau(seed_tau);
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
                    ag_store64(reinterpret_cast<uint64_t*>(out + pos), e);
                }
            }
        }
        __syncthreads();
        if (tid == 0) {
            const uint32_t n = sm.outcnt;
            ag_store32(&a.part_meta[pm + 0], n);
            ag_store32(&a.part_meta[pm + 1], excl);
            ag_store32(&a.part_meta[pm + 2], (n > (uint32_t)kPartCap) ? 1u : 0u);
        }
    } else if (tid == 0) {
        ag_store32(&a.part_meta[pm + 0], 0u);
        ag_store32(&a.part_meta[pm + 1], 0u);
        ag_store32(&a.part_meta[pm + 2], 1u);
    }
}

// ---- the last part: merge the lists and write the row's top k ----------------------------

__device__ __forceinline__ void fast_hand_to_general(const KArgs& a, int r) {
    if (threadIdx.x == 0) a.row_state[r] = kRowNeedsGeneral;
}

// Returns the positions of the row's top k written from the lists (k, or every candidate when
// the row has fewer than k that are not NaN), or -1 when the row was handed over.
__device__ __forceinline__ int fast_topk_merge(const KArgs& a, FastSmem& sm, int r, int k) {
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
        spec[s] = pp < S ? ag_load64(reinterpret_cast<const uint64_t*>(
                               a.part_list + ((size_t)r * kMaxParts + pp) * kPartCap + i))
                         : 0ull;
    }
    if (tid == 0) sm.status = 0;
    __syncthreads();
    if (tid < S) {
        const size_t pm = ((size_t)r * kMaxParts + tid) * 4;
        sm.pcnt[tid] = ag_load32(&a.part_meta[pm + 0]);
        if (ag_load32(&a.part_meta[pm + 2])) atomicOr(&sm.status, 4u);
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t off = 0;
        for (int pp = 0; pp < S; ++pp) { sm.poff[pp] = off; off += sm.pcnt[pp]; }
        sm.poff[S] = off;
        if (off > (uint32_t)kMergeCap) sm.status |= 8u;
    }
    __syncthreads();
    if (sm.status) { fast_hand_to_general(a, r); return -1; }
    const int N = (int)sm.poff[S];
#pragma unroll
    for (int s = 0; s < NSPEC; ++s) {
        const int e = s * NT + tid, pp = e / kSpec, i = e % kSpec;
        if (pp < S && i < (int)sm.pcnt[pp]) {
            const int o = (int)sm.poff[pp] + i;
            mk[o] = (uint32_t)spec[s];
            mi[o] = (int32_t)(uint32_t)(spec[s] >> 32);
        }
    }
    for (int pp = 0; pp < S; ++pp) {  // lists longer than the speculative window
        const int n = (int)sm.pcnt[pp];
        if (n <= kSpec) continue;
        const uint2* src = a.part_list + ((size_t)r * kMaxParts + pp) * kPartCap;
        for (int i = kSpec + tid; i < n; i += NT) {
            const uint64_t e = ag_load64(reinterpret_cast<const uint64_t*>(src + i));
            const int o = (int)sm.poff[pp] + i;
            mk[o] = (uint32_t)e;
            mi[o] = (int32_t)(uint32_t)(e >> 32);
        }
    }
    __syncthreads();

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
    if (kth != 0u) return k;
    // fewer than k candidates that are not NaN: every one of them was written
    if (wave == 0) {
        uint64_t c = 0;
        for (int j = lane; j < N; j += kWave) c += mk[j] != 0u ? 1u : 0u;
        c = wave_sum_u64(c);
        if (lane == 0) sm.bcast[1] = (uint32_t)c;
    }
    __syncthreads();
    return (int)sm.bcast[1];
}

template <typename T>
__global__ __launch_bounds__(kFastThreads) void fast_kernel(KArgs a) {
    __shared__ FastSmem sm;
    const int b = blockIdx.x;
    const int xcd = b & 7, slot = b >> 3;
    const int p = slot % a.S;
    const int r = (slot / a.S) * 8 + xcd;
    if (r >= a.B) return;
    const int k = a.topk_k;
    fast_stream_part<T>(a, sm, r, p, k);
    stores_complete();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = ag_add32(&a.row_counter[r], 1u);
        sm.last = (prev == (uint32_t)(a.S - 1)) ? 1u : 0u;
    }
    __syncthreads();
    if (!sm.last) return;
    if (threadIdx.x == 0) ag_store32(&a.row_counter[r], 0u);
    const int nv = fast_topk_merge(a, sm, r, k);
    if (nv >= 0 && nv < k && threadIdx.x < kWave)
        topk_fill_nan<T>(reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride, a.V, nv, k,
                         a.topk_vals + (size_t)r * k, a.topk_ids + (size_t)r * k);
}

// The rows fast_kernel handed over (row_state), selected exactly by the multi-pass path's radix
// select; one 1024-thread workgroup per row.
template <typename T>
__global__ __launch_bounds__(kGenThreads) void general_kernel(KArgs a) {
    __shared__ GenSmem sm;
    const int r = blockIdx.x;
    if (r >= a.B || a.row_state[r] == 0u) return;
    __syncthreads();
    if (threadIdx.x == 0) a.row_state[r] = 0u;
    general_topk_row<T>(a, sm, r);
}

template __global__ void fast_kernel<float>(KArgs);
template __global__ void fast_kernel<uint16_t>(KArgs);
template __global__ void fast_kernel<_Float16>(KArgs);
template __global__ void general_kernel<float>(KArgs);
template __global__ void general_kernel<uint16_t>(KArgs);
template __global__ void general_kernel<_Float16>(KArgs);

}  // namespace vws
