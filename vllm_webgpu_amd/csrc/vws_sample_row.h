// vws_sample_row.h -- the sampling kernel: one workgroup of 1024 threads per row.  Instantiated
// per logits type in vws_row_f32.hip, vws_row_bf16.hip and vws_row_f16.hip (each a code object
// of its own, compiled in parallel), with and without raw logprobs.
//
// Greedy rows and top-k rows (k <= 256) are finished in one streaming pass over the row:
//   1. the history ids are loaded, then the first two iterations of logits (8 x 16-byte loads
//      per lane each) are put in flight;
//   2. the history goes into an LDS hash (count, prompt flag);
//   3. a threshold is seeded from the first iteration: the lane maxima of its 32 values are
//      sorted per wave, the 16 largest of every wave are pooled and the m-th largest of the
//      pool (m = 3k x the sampled fraction of the row) becomes the starting threshold;
//   4. the row is streamed once, double-buffered, with buffer loads; an element at or above
//      the threshold goes to its wave's LDS candidate buffer by its raw value.  Penalties are
//      applied to the buffered candidates (when a buffer is compacted and once after the
//      stream): penalties that never raise a logit keep raw >= penalised, so nothing is missed;
//      otherwise the penalised history values are added up front and the stream entries of
//      history tokens dropped.  A full buffer is cut to its exact top-k by a radix select,
//      which raises the threshold for every wave;
//   5. the k-th largest candidate is selected.  It is exact when every element at or above it
//      was kept, i.e. when it is not below any threshold used (a seed above the k-th value
//      fails this check and sends the row to the general path);
//   6. survivors of temperature, top-k and min-p get their exact integer masses and race keys
//      (each wave fetches its candidates' uniforms as soon as its stream ends); top-p is
//      cut on the exact prefix sums and the race is reduced across the survivors.
// Every other row (top-k off or k > 256, logprobs requested, candidate or hash overflow, a
// seed above the k-th value, degenerate maxima, temperature ties across a threshold) runs the
// multi-pass path of vws_general.h in the same workgroup, so one launch serves the whole batch.
#pragma once

#include "vws_general.h"
#include "vws_topp.h"

namespace vws {

constexpr int kRowThreads = kGenThreads;     // 1024
constexpr int kRowWaves = kGenWaves;         // 16
constexpr int kRowCap = 512;                 // candidate slots per wave
constexpr int kRowHash = 2048;               // history hash slots
constexpr int kRowHashFill = 1536;           // unique history tokens served in LDS
constexpr int kRowHashBits = 1 << 17;        // presence bits of hashed tokens (token mod 2^17)
constexpr int kRowKeep = 256;                // survivors finished here
constexpr int kRowPack = kRowThreads;        // candidates finished here (more: general path)
constexpr int kSeedPerWave = 16;             // lane maxima each wave contributes to the seed pool
constexpr int kLoadNT = 2;                   // buffer-load cache policy: non-temporal

struct RowSmem {
    uint32_t ckey[kRowWaves][kRowCap];
    int32_t cidx[kRowWaves][kRowCap];
    // all candidates of the row, packed in any order: key(y) and index (k > 64), or one 64-bit
    // key per candidate (k <= 64)
    union alignas(16) {
        struct {
            uint32_t pkey[kRowPack];
            int32_t pidx[kRowPack];
        };
        uint64_t pk64[kRowPack];
    };
    float pu[kRowPack];                      // their uniforms (sampled rows)
    uint32_t crank[kRowPack];                // rank of each packed candidate (partial sums)
    uint64_t sC[kRowKeep];                   // survivors' cumulative masses (partial sums)
    uint64_t sW;                             // total mass of the survivors
    uint32_t rhist[kRowWaves][256];          // per-wave radix-select scratch
    uint32_t hkey[kRowHash];                 // history / processor token + 1 (0 = empty)
    uint32_t hval[kRowHash];                 // output count | kHBias | kHBan | kHPrompt
    float hpen[kRowHash];                    // processed value (gather mode)
    float hadj[kRowHash];                    // logit bias (kHBias)
    alignas(16) uint32_t hbits[kRowHashBits / 32];  // bit (t mod 2^17) set for every hashed token t
    alignas(16) uint64_t sck[kRowKeep];      // survivors: key(y) << 32 | index
    alignas(16) uint64_t sw[kRowKeep];       // exact mass
    float se[kRowKeep];                      // exp(y - max)
    uint32_t spos[kRowKeep];                 // packed position (for the uniform)
    alignas(16) uint64_t tk[kWave + 1];      // k <= 64: the 65 largest 64-bit keys, descending
    float tu[kWave];                         // and the uniforms of the first 64
    uint32_t npack;                          // candidates packed so far
    uint32_t seedk[kRowWaves * kSeedPerWave];
    uint64_t red[kRowWaves][8];
    uint32_t tauw[kRowWaves];
    uint32_t tau, status, nhash, nkeep;
    uint32_t ymax, tmaxk;                    // largest packed y key; largest threshold used
    uint32_t adjraise;                       // a positive logit bias was inserted
    uint32_t bc[8];
    // penalty context of the row for the out-of-line fix-up: mode 0 none, 1 penalise, 2 drop;
    // whether the hash holds tokens, and the row's token-state words (0 without a table)
    uint32_t pmode, phash;
    float prep, pinv, ppres, pfreq;
    uint64_t ptab;
    // raw logprobs (launches that ask for them): each wave's sum of 2^(x log2 e - lpA) over its share
    // of the row; the tail's token, packing layout, greedy flag and largest threshold; then
    // the sampled token's raw key, candidates at or above the threshold, the largest raw key
    // and the rank (row_logprobs_entry)
    uint32_t plp;
    double lpS[kRowWaves];
    float lpA[kRowWaves];
    uint32_t lpk[8];
    float lplog;
};

union RowShared {
    GenSmem g;
    RowSmem f;
    TopPSmem t;
};

__device__ __forceinline__ uint32_t rhash_slot(int t) {
    return ((uint32_t)t * 2654435761u) >> (32 - 11);  // kRowHash = 2048
}

// inc: 1 counts an output occurrence; otherwise kHPrompt, kHBan or kHBias (with its bias) is set
__device__ __forceinline__ void rhash_insert(RowSmem& sm, int t, uint32_t inc, float bias = 0.0f) {
    atomicOr(&sm.hbits[((uint32_t)t >> 5) & (kRowHashBits / 32 - 1)], 1u << (t & 31));
    uint32_t s = rhash_slot(t);
    for (int probe = 0; probe < kRowHash; ++probe) {
        const uint32_t prev = atomicCAS(&sm.hkey[s], 0u, (uint32_t)t + 1u);
        if (prev == 0u && atomicAdd(&sm.nhash, 1u) >= (uint32_t)kRowHashFill) atomicOr(&sm.status, 1u);
        if (prev == 0u || prev == (uint32_t)t + 1u) {
            if (inc == 1u) {
                atomicAdd(&sm.hval[s], 1u);
            } else {
                if (inc & kHBias) sm.hadj[s] = bias;  // one finite entry per token and row
                atomicOr(&sm.hval[s], inc);
            }
            return;
        }
        s = (s + 1u) & (kRowHash - 1);
    }
    atomicOr(&sm.status, 1u);
}

// whether token t may be in the row's hash (exact for vocabularies up to 2^17)
__device__ __forceinline__ bool rhash_maybe(const RowSmem& sm, int t) {
    return (sm.hbits[((uint32_t)t >> 5) & (kRowHashBits / 32 - 1)] >> (t & 31)) & 1u;
}

// slot of token t in the row's hash, -1 when absent
__device__ __forceinline__ int rhash_find(const RowSmem& sm, int t) {
    uint32_t s = rhash_slot(t);
    for (int probe = 0; probe < kRowHash; ++probe) {
        const uint32_t k = sm.hkey[s];
        if (k == (uint32_t)t + 1u) return (int)s;
        if (k == 0u) return -1;
        s = (s + 1u) & (kRowHash - 1);
    }
    return -1;
}

// LDS of the row kernel: the single-pass state, the top-p stream's and the general path's
// share it.
__shared__ RowShared g_row_sh;

__device__ __noinline__ TpDrop topp_compact_entry(int w, int cnt, float aw, float c, int want_raw) {
    return topp_compact(g_row_sh.t, w, cnt, aw, c, want_raw != 0);
}

__device__ __noinline__ void topp_rank_members_entry(uint32_t ng, float m) {
    topp_rank_members(g_row_sh.t, tp_u(ng), tp_uf(m));
}

// lane l's value of v, in every lane (wave-uniform l)
__device__ __forceinline__ uint64_t lane_bcast64(uint64_t v, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}

#if defined(__HIP_DEVICE_COMPILE__)  // the kernarg segment exists only in the device pass
// The launch arguments of an out-of-line function, read from the kernel's kernarg segment (the
// kernel hands over its address; a callee has no register of its own for it) into scalar
// registers.
__device__ __forceinline__ KArgs kargs_at(uint64_t kernarg) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)kernarg);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(kernarg >> 32));
    using KArgsConst = const KArgs __attribute__((address_space(4)));
    return *(KArgsConst*)(((uint64_t)hi << 32) | lo);
}
#endif

// A history row's buffers after its stream (topp_hist_prepare), out of line: rows without a
// history keep the finish's registers.
template <typename T>
__device__ __noinline__ int topp_hist_entry(int r, uint64_t kernarg, uint32_t tauk, float xmaxr) {
#if defined(__HIP_DEVICE_COMPILE__)
    const KArgs a = kargs_at(kernarg);
    r = __builtin_amdgcn_readfirstlane(r);
    const RowP prm = row_params(a, r);
    return topp_hist_prepare<T>(a, g_row_sh.t, r, prm, tp_u(tauk), tp_uf(xmaxr));
#else
    (void)r; (void)kernarg; (void)tauk; (void)xmaxr;
    return 0;
#endif
}

// The pass sm.pd over row r's body vectors [v0, v1) (and the edges): without, and with the
// penalties from the token-state table (separate functions, so that the plain pass keeps its
// registers).
template <typename T, bool PEN, int XF>
__device__ __forceinline__ void topp_range_body(int r, uint64_t kernarg, int v0, int v1, int edges) {
#if defined(__HIP_DEVICE_COMPILE__)
    const KArgs a = kargs_at(kernarg);
    r = __builtin_amdgcn_readfirstlane(r);
    v0 = __builtin_amdgcn_readfirstlane(v0);
    v1 = __builtin_amdgcn_readfirstlane(v1);
    edges = __builtin_amdgcn_readfirstlane(edges);
    TopPSmem& sm = g_row_sh.t;
    TpPassDesc d;
    d.kind = (int)tp_u((uint32_t)sm.pd.kind);
    d.key = tp_u(sm.pd.key);
    d.bstar = (int)tp_u((uint32_t)sm.pd.bstar);
    d.Tt = tp_uf(sm.pd.Tt);
    d.m = tp_uf(sm.pd.m);
    d.lp_min = tp_uf(sm.pd.lp_min);
    d.ksv = tp_u(sm.pd.ksv);
    d.kkeep = tp_u(sm.pd.kkeep);
    d.kmem = tp_u(sm.pd.kmem);
    TpPassAcc acc;
    tp_pass_range<T, PEN, XF>(a, sm, r, d, v0, v1, edges != 0, acc);
    tp_pass_reduce(sm, d.kind, acc);
#else
    (void)r; (void)kernarg; (void)v0; (void)v1; (void)edges;
#endif
}

// A range of a pass over row r (PEN: with the row's penalties; XF: what each logit goes through
// as it loads, the launch's mask or soft cap); one out-of-line function per combination, so
// that plain launches keep their registers.
template <typename T, bool PEN, int XF>
__device__ __noinline__ void topp_range_entry(int r, uint64_t kernarg, int v0, int v1, int edges) {
    topp_range_body<T, PEN, XF>(r, kernarg, v0, v1, edges);
}

template <typename T, int XF>
__device__ __forceinline__ void topp_range_any(bool pen, int r, uint64_t kernarg, int v0, int v1,
                                               int edges) {
    if (pen) topp_range_entry<T, true, XF>(r, kernarg, v0, v1, edges);
    else topp_range_entry<T, false, XF>(r, kernarg, v0, v1, edges);
}

template <typename T, bool PEN, int XF>
__device__ __noinline__ void topp_pass_entry(int kind, int r, uint64_t kernarg, float Tt, float m,
                                             float lp_min, uint32_t key, int bstar) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int NT = kGenThreads;
    // every argument is uniform: into scalar registers (the buffer descriptors need them there)
    const KArgs a = kargs_at(kernarg);
    kind = __builtin_amdgcn_readfirstlane(kind);
    r = __builtin_amdgcn_readfirstlane(r);
    bstar = __builtin_amdgcn_readfirstlane(bstar);
    const int tid = threadIdx.x, lane = tid & 63;
    TopPSmem& sm = g_row_sh.t;
    TpPassDesc d;
    d.kind = kind;
    d.key = tp_u(key);
    d.bstar = bstar;
    d.Tt = tp_uf(Tt);
    d.m = tp_uf(m);
    d.lp_min = tp_uf(lp_min);
    d.ksv = d.kkeep = d.kmem = 0u;
    if (kind == kTpPassWideRace) {
        tp_wide_keys(d, &sm.cp[8]);
        __syncthreads();
        const uint32_t ksv = tp_u(sm.cp[8]);
        const uint32_t kkeep = tp_u(sm.cp[9]), kmem = tp_u(sm.cp[10]);
        d.ksv = ksv;
        d.kkeep = kkeep > ksv ? kkeep : ksv;
        d.kmem = kmem > ksv ? kmem : ksv;
    }
    Slice<T> sl;
    sl.init(reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride, 0, a.V);
    const int nbody = __builtin_amdgcn_readfirstlane(sl.nbody);
    // chunks of kCoopChunkVecs vectors (a multiple of it for rows of more than
    // kCoopMaxChunks chunks)
    const int cmul = (nbody + kCoopMaxChunks * kCoopChunkVecs - 1) / (kCoopMaxChunks * kCoopChunkVecs);
    const int cvecs = (cmul > 0 ? cmul : 1) * kCoopChunkVecs;
    const int nch = (nbody + cvecs - 1) / cvecs;
    CoopState* st = a.coop;
    const bool coop = st != nullptr && nch >= kCoopMinChunks && nch <= kCoopMaxChunks;
    if (tid == 0) {
        sm.pd = d;  // what topp_range_entry runs
        sm.cp[4] = kCoopNone;
    }
    if (coop && tid < kWave) {
        // wave 0: a free slot for the row
        const uint32_t own = lane < kCoopSlots ? ag_load32(&st->slot[lane].owner) : 1u;
        uint64_t fr = wave_ballot(own == 0u);
        if (lane == 0) {
            while (fr) {
                const int s = __builtin_ctzll(fr);
                fr &= fr - 1ull;
                uint32_t expect = 0u;
                if (__hip_atomic_compare_exchange_strong(&st->slot[s].owner, &expect, (uint32_t)r + 1u,
                                                         __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT)) {
                    sm.cp[4] = (uint32_t)s;
                    break;
                }
            }
        }
    }
    __syncthreads();
    const uint32_t slot = tp_u(sm.cp[4]);
    const bool pen = PEN && tp_pass_pen(a, r, kind);
    if (slot == kCoopNone) {
        topp_range_any<T, XF>(pen, r, kernarg, 0, nbody, 1);
        return;
    }
    CoopSlot& S = st->slot[slot];
    // describe the pass and clear the totals it adds to, then open its chunks
    if (kind == kTpPassExact)
        for (int b = tid; b < kCoopBuckets; b += NT) ag_store64(&S.hmass[b], 0ull);
    if (kind == kTpPassWideRace && tid < kCoopMaxChunks) {
        ag_store64(&S.race[tid][0], 0ull);
        ag_store64(&S.race[tid][1], 0ull);
        ag_store64(&S.race[tid][2], 0ull);
    }
    if (tid == 0) {
        ag_store64(&S.sw, 0ull);
        ag_store64(&S.n, 0ull);
        ag_store64(&S.nrem, 0ull);
        ag_store32(&S.ngather, 0u);
        ag_store32(&S.done, 0u);
        ag_store32(reinterpret_cast<uint32_t*>(&S.kind), (uint32_t)kind);
        ag_store32(reinterpret_cast<uint32_t*>(&S.r), (uint32_t)r);
        ag_store32(reinterpret_cast<uint32_t*>(&S.bstar), (uint32_t)bstar);
        ag_store32(&S.key, d.key);
        ag_store32(&S.ksv, d.ksv);
        ag_store32(&S.kkeep, d.kkeep);
        ag_store32(&S.kmem, d.kmem);
        ag_store32(reinterpret_cast<uint32_t*>(&S.Tt), f2u(d.Tt));
        ag_store32(reinterpret_cast<uint32_t*>(&S.m), f2u(d.m));
        ag_store32(reinterpret_cast<uint32_t*>(&S.lp_min), f2u(d.lp_min));
        ag_store32(reinterpret_cast<uint32_t*>(&S.cvecs), (uint32_t)cvecs);
    }
    stores_complete();
    __syncthreads();
    uint32_t gen = 0u;
    if (tid == 0) {
        gen = (uint32_t)(ag_load64(&S.claim) >> 40) + 1u;
        if (!sm.coop_hold) {
            ag_add64(&st->wgs, kCoopActive);  // the row holds a slot until it is done
            sm.coop_hold = 1u;
        }
        ag_store64(&S.claim, coop_claim_word(gen, (uint32_t)nch));
        sm.cp[5] = coop_chunk_of(ag_add64(&S.claim, 1ull));
    }
    __syncthreads();
    // the chunks the row claims itself, one at a time; thread 0 keeps the totals
    RowRace tr;
    uint64_t t0 = 0ull, t1 = 0ull, t3 = 0ull;
    uint32_t own = 0u;
    uint32_t c = tp_u(sm.cp[5]);
    for (int k = 0; c != kCoopNone; ++k) {
        const int v0 = (int)c * cvecs;
        const int v1 = nbody < v0 + cvecs ? nbody : v0 + cvecs;
        topp_range_any<T, XF>(pen, r, kernarg, v0, v1, c == 0u ? 1 : 0);
        __syncthreads();
        if (tid == 0) {
            ++own;
            if (kind == kTpPassWideRace) {
                RowRace o;
                o.best = sm.bc64[10];
                o.second = (uint32_t)sm.bc64[11];
                o.nkept = (uint32_t)sm.bc64[12];
                o.last = sm.bc64[14];
                tr.merge(o);
                t3 += sm.bc64[13];
            } else {
                t0 += sm.bc64[10];
                t1 += sm.bc64[11];
            }
            // the next chunk, claimed once this one has run (helpers take the others meanwhile)
            sm.cp[6 + (k & 1)] = coop_chunk_of(ag_add64(&S.claim, 1ull));
        }
        __syncthreads();
        c = tp_u(sm.cp[6 + (k & 1)]);
    }
    // the chunks other workgroups claimed: every one is running, so the wait ends; it is bounded
    // all the same (a.coop_wait_polls; 0, a test setting, gives every pass up here).  Giving up
    // hands the slot to whoever completes it: the owner adds kCoopAbandon - others to the done
    // count, and the completion that brings the count to exactly kCoopAbandon frees the slot --
    // the owner itself when every chunk was done meanwhile (with a non-zero bound the pass then
    // counts as completed), else the last helper's increment (coop_help_entry).  No chunk is
    // open at this point (the owner's own claims ran out), so a freed slot has no late chunk
    // left to add into it.
    if (tid == 0) {
        const uint32_t others = (uint32_t)nch - own;
        const int polls = a.coop_wait_polls;
        uint32_t done = ag_load32(&S.done);
        for (int poll = 0; done < others && poll < polls; ++poll) {
            __builtin_amdgcn_s_sleep(1);
            done = ag_load32(&S.done);
        }
        uint32_t ok = done >= others ? 1u : 0u;
        if (!ok || polls == 0) {
            const uint32_t prev = ag_add32(&S.done, kCoopAbandon - others);
            ok = (prev == others && polls != 0) ? 1u : 0u;
            if (prev == others && polls == 0) {
                ag_store64(&S.claim, coop_claim_word(gen, 0u));
                ag_store32(&S.owner, 0u);
            }
        }
        sm.cp[4] = ok;
    }
    __syncthreads();
    if (!tp_u(sm.cp[4])) {
        // abandoned: the slot is the late helpers' to free; the row takes the multi-pass path
        if (tid == 0) sm.coop_fail = 1u;
        return;
    }
    // their totals
    RowRace hr;
    if (kind == kTpPassWideRace && tid < nch) {
        hr.best = ag_load64(&S.race[tid][0]);
        const uint64_t x = ag_load64(&S.race[tid][1]);
        hr.second = (uint32_t)(x >> 32);
        hr.nkept = (uint32_t)x;
        hr.last = ag_load64(&S.race[tid][2]);
    }
    if (kind == kTpPassWideRace && tid < kWave) {
        hr.shfl_merge(32); hr.shfl_merge(16); hr.shfl_merge(8);
        hr.shfl_merge(4); hr.shfl_merge(2); hr.shfl_merge(1);
    }
    if (kind == kTpPassExact) {
        for (int b = tid; b < kCoopBuckets; b += NT) {
            const uint64_t v = ag_load64(&S.hmass[b]);
            if (v) sm.h.hmass[b] += v;
        }
    }
    uint32_t base = 0u, ngh = 0u;
    if (kind == kTpPassWideRace) {
        // the boundary members the others gathered, after the row's own
        ngh = ag_load32(&S.ngather);
        base = tp_u(sm.bc[4]);
        const uint32_t nld = ngh < (uint32_t)kCoopGather ? ngh : (uint32_t)kCoopGather;
        for (uint32_t i = (uint32_t)tid; i < nld; i += NT)
            if (base + i < (uint32_t)kTpGather) sm.g.key[base + i] = ag_load64(&S.gkey[i]);
    }
    // the totals sw, n, nrem, one per lane of wave 0, in one round trip (thread 0 uses them)
    uint64_t hsw = 0ull, hn = 0ull, hrem = 0ull;
    if (tid < kWave) {
        const uint64_t v = tid < 3 ? ag_load64(&S.sw + tid) : 0ull;
        hsw = lane_bcast64(v, 0);
        hn = lane_bcast64(v, 1);
        hrem = lane_bcast64(v, 2);
    }
    __syncthreads();
    if (tid == 0) {
        if (kind == kTpPassExact) {
            sm.bc64[10] = t0 + hsw;
            sm.bc64[11] = t1 + hn;
        } else if (kind == kTpPassWideRace) {
            tr.merge(hr);
            sm.bc64[10] = tr.best;
            sm.bc64[11] = tr.second;
            sm.bc64[12] = tr.nkept;
            sm.bc64[13] = t3 + hrem;
            sm.bc64[14] = tr.last;
            sm.bc[4] = base + ngh;
        } else {
            sm.bc64[10] = t0 + hn;
        }
        // free the slot: nothing open, no owner
        ag_store64(&S.claim, coop_claim_word(gen, 0u));
        ag_store32(&S.owner, 0u);
    }
#else
    (void)kind; (void)r; (void)kernarg; (void)Tt; (void)m; (void)lp_min; (void)key; (void)bstar;
#endif
}

// A workgroup without a row (or between two rows) runs chunks of the passes other rows opened,
// adding its totals into their slots.  spin: poll again while rows hold slots (no row of the
// launch is left to start, so no row waits for this workgroup's CU); otherwise return once no
// chunk is open.  PEN: the launch has penalties from a token-state table with its bitmap (some
// chunks are of penalised passes; without, the function calls only the plain range function).
template <typename T, bool PEN, int XF>
__device__ __noinline__ void coop_help_entry(uint64_t kernarg, int spin) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int NT = kGenThreads;
    const KArgs a = kargs_at(kernarg);
    spin = __builtin_amdgcn_readfirstlane(spin);
    CoopState* st = a.coop;
    TopPSmem& sm = g_row_sh.t;
    const int tid = threadIdx.x, lane = tid & 63;
    // the slot whose description sm.pd holds, its generation, and a chunk claimed there
    uint32_t got = kCoopNone, gen = 0u, c = kCoopNone;
    for (int poll = 0; poll < kCoopHelpPolls; ++poll) {
        if (c == kCoopNone) {
            // wave 0: the slots with chunks open, a claim on one of them, its description
            if (tid < kWave) {
                const uint64_t cl = lane < kCoopSlots ? ag_load64(&st->slot[lane].claim) : 0ull;
                uint64_t open = wave_ballot(lane < kCoopSlots && coop_chunk_of(cl) != kCoopNone);
                uint32_t g = kCoopNone, cc = kCoopNone, gn = 0u;
                if (lane == 0) {
                    while (open) {
                        const int s = __builtin_ctzll(open);
                        open &= open - 1ull;
                        // acquire: the pass description is read after the claim
                        const uint64_t x = __hip_atomic_fetch_add(&st->slot[s].claim, 1ull, __ATOMIC_ACQUIRE,
                                                                  __HIP_MEMORY_SCOPE_AGENT);
                        cc = coop_chunk_of(x);
                        if (cc != kCoopNone) {
                            g = (uint32_t)s;
                            gn = (uint32_t)(x >> 40);
                            break;
                        }
                    }
                }
                g = (uint32_t)__builtin_amdgcn_readfirstlane((int)g);
                uint32_t stop = 0u;
                if (g != kCoopNone) {
                    // the description's words (kind, r, bstar, key, ksv, kkeep, kmem, Tt, m,
                    // lp_min, cvecs), one per lane, in one round trip
                    const uint32_t* dw = reinterpret_cast<const uint32_t*>(&st->slot[g].kind);
                    const uint32_t w = lane < 11 ? ag_load32(dw + lane) : 0u;
                    if (lane < 11) sm.cp[8 + lane] = w;
                    if (lane == 0) {
                        sm.cp[2] = cc;
                        sm.cp[1] = gn;
                    }
                } else if (lane == 0) {
                    stop = (!spin || coop_pending(ag_load64(&st->wgs)) == 0u) ? 1u : 0u;
                }
                if (lane == 0) {
                    sm.cp[0] = g;
                    sm.cp[3] = stop;
                }
            }
            __syncthreads();
            got = tp_u(sm.cp[0]);
            if (got == kCoopNone) {
                const bool stop = tp_u(sm.cp[3]) != 0u;
                __syncthreads();  // every wave has read the broadcast before wave 0 writes it again
                if (stop) break;
                __builtin_amdgcn_s_sleep(8);
                continue;
            }
            c = tp_u(sm.cp[2]);
            gen = tp_u(sm.cp[1]);
            if (tid == 0) {
                // the description as topp_range_entry reads it
                sm.pd.kind = (int)sm.cp[8];
                sm.pd.bstar = (int)sm.cp[10];
                sm.pd.key = sm.cp[11];
                sm.pd.ksv = sm.cp[12];
                sm.pd.kkeep = sm.cp[13];
                sm.pd.kmem = sm.cp[14];
                sm.pd.Tt = u2f(sm.cp[15]);
                sm.pd.m = u2f(sm.cp[16]);
                sm.pd.lp_min = u2f(sm.cp[17]);
            }
        }
        const int r = (int)tp_u(sm.cp[9]);
        const int kind = (int)tp_u(sm.cp[8]);
        const int cvecs = (int)tp_u(sm.cp[18]);
        CoopSlot& S = st->slot[got];
        // an owner only ever describes a row of this launch and a pass it knows
        if (r < 0 || r >= a.B || kind < kTpPassExact || kind > kTpPassRank || c >= (uint32_t)kCoopMaxChunks ||
            cvecs <= 0) {
            __syncthreads();
            c = kCoopNone;
            continue;
        }
        // the chunk's totals start from zero here
        if (kind == kTpPassExact)
            for (int b = tid; b < kTpBuckets; b += NT) sm.h.hmass[b] = 0ull;
        if (tid == 0) sm.bc[4] = 0u;
        __syncthreads();
        Slice<T> sl;
        sl.init(reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride, 0, a.V);
        const int nbody = __builtin_amdgcn_readfirstlane(sl.nbody);
        const int v0 = (int)c * cvecs;
        const int v1 = nbody < v0 + cvecs ? nbody : v0 + cvecs;
        topp_range_any<T, XF>(PEN && tp_pass_pen(a, r, kind), r, kernarg, v0, v1, c == 0u ? 1 : 0);
        __syncthreads();
        // the next chunk, claimed while this one's totals go out (before this one counts as
        // done, so the pass cannot have been replaced meanwhile)
        uint64_t nx = 0ull;
        if (tid == 0)
            nx = __hip_atomic_fetch_add(&S.claim, 1ull, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
        // added into the slot
        if (kind == kTpPassExact) {
            for (int b = tid; b < kTpBuckets; b += NT) {
                const uint64_t v = sm.h.hmass[b];
                if (v) ag_add64(&S.hmass[b], v);
            }
            if (tid == 0) {
                ag_add64(&S.sw, sm.bc64[10]);
                ag_add64(&S.n, sm.bc64[11]);
            }
        } else if (kind == kTpPassWideRace) {
            const uint32_t ng = sm.bc[4];
            if (tid == 0) {
                ag_store64(&S.race[c][0], sm.bc64[10]);
                ag_store64(&S.race[c][1], (sm.bc64[11] << 32) | (uint32_t)sm.bc64[12]);
                ag_store64(&S.race[c][2], sm.bc64[14]);
                ag_add64(&S.nrem, sm.bc64[13]);
                sm.cp[4] = ng ? ag_add32(&S.ngather, ng) : 0u;
            }
            __syncthreads();
            const uint32_t base = tp_u(sm.cp[4]);
            const uint32_t nst = ng < (uint32_t)kTpGather ? ng : (uint32_t)kTpGather;
            for (uint32_t i = (uint32_t)tid; i < nst; i += NT)
                if (base + i < (uint32_t)kCoopGather) ag_store64(&S.gkey[base + i], sm.g.key[i]);
        } else if (tid == 0) {
            ag_add64(&S.n, sm.bc64[10]);
        }
        stores_complete();
        __syncthreads();
        if (tid == 0) {
            // the last chunk of a pass its owner gave up on: free the slot (no chunk of it is
            // open or running any more)
            if (ag_add32(&S.done, 1u) + 1u == kCoopAbandon) {
                ag_store64(&S.claim, coop_claim_word(gen, 0u));
                ag_store32(&S.owner, 0u);
            }
            // the claimed next chunk: of this pass (same generation) it runs with the same
            // description; of a later pass the description is read again (a claimed chunk always
            // runs); none: look again
            const uint32_t cn = coop_chunk_of(nx);
            const bool same = ((uint32_t)(nx >> 40) & 0xFFFFFFu) == (gen & 0xFFFFFFu);
            sm.cp[5] = cn;
            sm.cp[6] = (cn != kCoopNone && !same) ? 1u : 0u;
            sm.cp[7] = (uint32_t)(nx >> 40);
        }
        __syncthreads();
        c = tp_u(sm.cp[5]);
        if (c != kCoopNone && tp_u(sm.cp[6])) {
            // a later pass in the same slot: its description
            if (tid < kWave) {
                const uint32_t* dw = reinterpret_cast<const uint32_t*>(&S.kind);
                const uint32_t w = lane < 11 ? ag_load32(dw + lane) : 0u;
                if (lane < 11) sm.cp[8 + lane] = w;
            }
            __syncthreads();
            gen = tp_u(sm.cp[7]);
            if (tid == 0) {
                sm.pd.kind = (int)sm.cp[8];
                sm.pd.bstar = (int)sm.cp[10];
                sm.pd.key = sm.cp[11];
                sm.pd.ksv = sm.cp[12];
                sm.pd.kkeep = sm.cp[13];
                sm.pd.kmem = sm.cp[14];
                sm.pd.Tt = u2f(sm.cp[15]);
                sm.pd.m = u2f(sm.cp[16]);
                sm.pd.lp_min = u2f(sm.cp[17]);
            }
        }
        __syncthreads();
    }
#else
    (void)kernarg; (void)spin;
#endif
}

// Applies the logits processors and penalties to wave w's candidates [from, cnt), in place, and
// returns the new count.  Candidates enter the buffer by their raw value; when nothing can raise
// a logit (mode 1: bans, non-positive biases, penalties with r >= 1, f >= 0, p >= 0) the raw
// value bounds the processed one from above, so nothing is missed and the key is corrected
// here.  In mode 2 (something may raise a logit) the processed values of the hashed tokens were
// added up front with bit 31 of the index set; stream entries of hashed tokens are dropped.
// Penalties from a token-state table (whose tokens are never hashed) are monotone here: the
// table's words are read at the candidates, in both modes.
__device__ __noinline__ int row_fixup(int w, int from, int cnt) {
    RowSmem& sm = g_row_sh.f;
    const uint32_t mode = sm.pmode;
    if (mode == 0u || from >= cnt) return cnt;
    uint32_t* ck = sm.ckey[w];
    int32_t* ci = sm.cidx[w];
    const bool hashed = sm.phash != 0u;
    const uint32_t* tab = reinterpret_cast<const uint32_t*>(sm.ptab);
    const int lane = lane_id();
    int out = from;
    for (int base = from; base < cnt; base += kWave) {
        const int i = base + lane;
        bool keep = false;
        uint32_t kk = 0;
        int32_t ii = 0;
        if (i < cnt) {
            kk = ck[i];
            ii = ci[i];
            keep = true;
            if (ii < 0) {
                ii &= 0x7FFFFFFF;  // added up front, already penalised
            } else {
                const int hs = hashed ? rhash_find(sm, ii) : -1;
                if (hs >= 0 && mode == 2u) {
                    keep = false;
                } else {
                    uint32_t hv = hs >= 0 ? sm.hval[hs] : 0u;
                    if (tab) hv |= tab[ii] & kStateMask;
                    if (hs >= 0 || hv != 0u)
                        kk = key_of(apply_hashed(val_of(kk), hv, hs >= 0 ? sm.hadj[hs] : 0.0f, sm.prep,
                                                 sm.pinv, sm.pfreq, sm.ppres));
                }
            }
        }
        const uint64_t bal = wave_ballot(keep);
        if (keep) { const int pos = out + lane_prefix(bal); ck[pos] = kk; ci[pos] = ii; }
        out += __popcll(bal);
        wave_sync();
    }
    return out;
}

// Penalises wave w's unfixed candidates [nfix, cnt), then cuts the buffer to its exact top-k,
// all ties included, in place, and raises the shared threshold to the k-th key.  Returns
// (k-th key << 32) | new count (k-th key 0 when fewer than k candidates remain).  Compaction is
// rare, so it lives out of line and the unrolled streaming loop stays small.
__device__ __noinline__ uint64_t row_compact(int w, int nfix, int cnt, int k) {
    // raw logprobs need the candidates' raw keys, which a fix-up replaces (and a cut by
    // processed values may drop an element of the raw top L): the row takes the multi-pass path
    if (g_row_sh.f.plp && g_row_sh.f.pmode != 0u) atomicOr(&g_row_sh.f.status, 8u);
    cnt = row_fixup(w, nfix, cnt);
    if (cnt <= k) return (uint64_t)(uint32_t)cnt;
    RowSmem& sm = g_row_sh.f;
    uint32_t* ck = sm.ckey[w];
    int32_t* ci = sm.cidx[w];
    const int lane = lane_id();
    const uint32_t kth = wave_kth_largest(ck, cnt, k, sm.rhist[w]);
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
    if (lane == 0) atomicMax(&sm.tau, kth);
    wave_sync();
    return ((uint64_t)kth << 32) | (uint32_t)out;
}

// Per-wave candidate buffer of the row kernel: every element of the wave's share at or above
// the wave's threshold; the threshold only rises (own compactions, other waves' via sm.tau).
struct RowCand {
    int w, k, cnt;        // wave-uniform
    int nfix;             // entries [0, nfix) carry penalised keys
    uint32_t tau;         // threshold key
    float tauf;           // its value form (-inf when every non-NaN value passes)
    bool ovf;             // ties overflowed the buffer
    bool compact_ok;      // a full buffer may be cut to its top k (not with the soft cap)
    __device__ __forceinline__ void init(int w_, int k_, bool compact_ok_) {
        w = w_; k = k_; cnt = 0; nfix = 0; tau = 0u; tauf = -__builtin_inff(); ovf = false;
        compact_ok = compact_ok_;
    }
    __device__ __forceinline__ void set_tau(uint32_t t) {
        if (t > tau) {
            tau = t;
            tauf = (tau > 0x007FFFFFu) ? val_of(tau) : -__builtin_inff();
        }
    }
    __device__ __forceinline__ void refresh() {
        set_tau(__builtin_amdgcn_readfirstlane(
            __hip_atomic_load(&g_row_sh.f.tau, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)));
    }
    // Appends all VEC elements of the lanes in hm (raw keys; elements below the threshold and
    // NaNs included, dropped by filter()); wave-uniform call.
    template <int VEC>
    __device__ __forceinline__ void append_vec(const float* v, int i0, uint64_t hm) {
        if (ovf) return;
        int n = __popcll(hm) * VEC;
        if (cnt + n > kRowCap) {
            if (!compact_ok) { ovf = true; return; }
            const uint64_t rc = row_compact(w, nfix, cnt, k);
            cnt = __builtin_amdgcn_readfirstlane((uint32_t)rc);
            nfix = cnt;
            set_tau(__builtin_amdgcn_readfirstlane((uint32_t)(rc >> 32)));
            if (cnt + n > kRowCap) { ovf = true; return; }
        }
        if ((hm >> lane_id()) & 1ull) {
            const int pos = cnt + lane_prefix(hm) * VEC;
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                g_row_sh.f.ckey[w][pos + j] = key_of(v[j]);
                g_row_sh.f.cidx[w][pos + j] = i0 + j;
            }
        }
        cnt += n;
        wave_sync();
    }
    // Drops the entries below the threshold (and NaNs) in place, keeping the order.
    __device__ __forceinline__ void filter() {
        uint32_t* ck = g_row_sh.f.ckey[w];
        int32_t* ci = g_row_sh.f.cidx[w];
        const int lane = lane_id();
        int out = 0, outfix = 0;
        for (int base = 0; base < cnt; base += kWave) {
            const int i = base + lane;
            uint32_t kk = 0u;
            int32_t ii = 0;
            if (i < cnt) { kk = ck[i]; ii = ci[i]; }
            const bool keep = i < cnt && kk != 0u && kk >= tau;
            const uint64_t bal = wave_ballot(keep);
            if (keep) { const int pos = out + lane_prefix(bal); ck[pos] = kk; ci[pos] = ii; }
            out += __popcll(bal);
            outfix += __popcll(wave_ballot(keep && i < nfix));
            wave_sync();
        }
        cnt = out;
        nfix = outfix;
    }
    // Appends (kk, idx) from the lanes where c holds; wave-uniform call.
    __device__ __forceinline__ void append(bool c, uint32_t kk, int32_t idx) {
        uint64_t bal = wave_ballot(c);
        if (!bal || ovf) return;
        int n = __popcll(bal);
        if (cnt + n > kRowCap) {
            if (!compact_ok) { ovf = true; return; }
            const uint64_t rc = row_compact(w, nfix, cnt, k);
            cnt = __builtin_amdgcn_readfirstlane((uint32_t)rc);
            nfix = cnt;
            set_tau(__builtin_amdgcn_readfirstlane((uint32_t)(rc >> 32)));
            c = c && kk >= tau;
            bal = wave_ballot(c);
            n = __popcll(bal);
            if (cnt + n > kRowCap) { ovf = true; return; }
        }
        if (c) {
            const int pos = cnt + lane_prefix(bal);
            g_row_sh.f.ckey[w][pos] = kk;
            g_row_sh.f.cidx[w][pos] = idx;
        }
        cnt += n;
        wave_sync();
    }
    // penalised keys for every candidate (once, after the stream)
    __device__ __forceinline__ void finish() {
        if (nfix < cnt) cnt = __builtin_amdgcn_readfirstlane((uint32_t)row_fixup(w, nfix, cnt));
        nfix = cnt;
    }
};

// Defaults read in place of a missing per-row parameter array, so every parameter is one
// unconditional scalar load: T, top_p, min_p, repetition, presence, frequency.  The arrays are
// never written; they are not const so that they live in the global address space, like the
// arrays they stand in for, and the pointer select between the two stays global.
static __device__ float kRowDefaultsF[8] = {0.0f, 1.0f, 0.0f, 1.0f, 0.0f, 0.0f, 0.0f, 0.0f};
// top_k (0 = off), a length that clamps to the history width (absent lengths = full width), and
// a token-state row (replaced by the row itself when the table has no row map)
static __device__ int32_t kRowDefaultsI[4] = {0, 0x7FFFFFFF, 0, 0};

// Per-row parameters, all issued as scalar loads before the first one is used.  Scalar loads
// complete on their own counter, so waiting for them never waits for the logits in flight.
__device__ __forceinline__ RowP row_params_scalar(const KArgs& a, int r) {
    const float* pT = a.temperature ? a.temperature + r : &kRowDefaultsF[0];
    const float* pP = a.top_p ? a.top_p + r : &kRowDefaultsF[1];
    const float* pM = a.min_p ? a.min_p + r : &kRowDefaultsF[2];
    const float* pR = a.rep ? a.rep + r : &kRowDefaultsF[3];
    const float* pS = a.pres ? a.pres + r : &kRowDefaultsF[4];
    const float* pF = a.freq ? a.freq + r : &kRowDefaultsF[5];
    const int32_t* pK = a.top_k ? a.top_k + r : &kRowDefaultsI[0];
    const int32_t* pPL = a.plens ? a.plens + r : &kRowDefaultsI[1];
    const int32_t* pOL = a.olens ? a.olens + r : &kRowDefaultsI[1];
    const int32_t* pAL = a.adjlens ? a.adjlens + r : &kRowDefaultsI[1];
    const int32_t* pTR = a.trows ? a.trows + r : &kRowDefaultsI[2];
    RowP p;
    int pl, ol, al, tr;
    // scalar loads on the scalar counter; the compiler would otherwise issue vector loads, and
    // waiting for those would also wait for every logits load issued before them
    asm volatile(
        "s_load_dword %0, %11, 0x0\n\t"
        "s_load_dword %1, %12, 0x0\n\t"
        "s_load_dword %2, %13, 0x0\n\t"
        "s_load_dword %3, %14, 0x0\n\t"
        "s_load_dword %4, %15, 0x0\n\t"
        "s_load_dword %5, %16, 0x0\n\t"
        "s_load_dword %6, %17, 0x0\n\t"
        "s_load_dword %7, %18, 0x0\n\t"
        "s_load_dword %8, %19, 0x0\n\t"
        "s_load_dword %9, %20, 0x0\n\t"
        "s_load_dword %10, %21, 0x0\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(p.T), "=&s"(p.top_p), "=&s"(p.min_p), "=&s"(p.rep), "=&s"(p.pres), "=&s"(p.freq),
          "=&s"(p.k), "=&s"(pl), "=&s"(ol), "=&s"(al), "=&s"(tr)
        : "s"(pT), "s"(pP), "s"(pM), "s"(pR), "s"(pS), "s"(pF), "s"(pK), "s"(pPL), "s"(pOL), "s"(pAL),
          "s"(pTR)
        : "memory");
    p.greedy = is_greedy(p.T);
    p.inv_rep = 1.0f / p.rep;
    p.np = (a.prompt && p.rep != 1.0f) ? min(max(pl, 0), a.pwidth) : 0;  // see row_params
    p.no = a.output ? min(max(ol, 0), a.owidth) : 0;
    const bool identity = (p.rep == 1.0f && p.pres == 0.0f && p.freq == 0.0f);
    p.tab = a.tstate != nullptr && !identity;
    p.trow = a.trows ? tr : r;
    p.has_hist = p.tab || ((p.np > 0 || p.no > 0) && !identity);
    p.na = a.adj_ids ? min(max(al, 0), a.adjwidth) : 0;
    p.need_hash = (p.has_hist && !p.tab) || p.na > 0;
    return p;
}

// floor(a / b) for 0 <= a < 2^20 and 1 <= b <= 1024: (a + 1/2) / b lies at least 1 / (2b) from
// an integer, far beyond the error of the reciprocal, so the truncation is exact.
__device__ __forceinline__ int small_div(int a, int b) {
    return (int)(((float)a + 0.5f) * __builtin_amdgcn_rcpf((float)b));
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
    // the builtin returns int: widen each half as unsigned
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((uint32_t)v, l);
    return ((uint64_t)hi << 32) | lo;
}

// Tail of a row with k <= 64, after the candidates are packed as 64-bit keys (key(y) << 32 |
// index; the index reversed for greedy rows).  The number of keys above a candidate is its
// position in descending key order, so the 65 largest keys land in tk[] sorted; the rest of
// the row is finished by wave 0 from registers:
//   * top-k with ties: the candidates whose y is at least the y of tk[k - 1];
//   * min-p, then the exact masses; the sum of the masses at and after slot j is the
//     cumulative mass of that survivor in ascending (y, index) order, a suffix sum;
//   * top-p removes the survivors whose cumulative mass is at most floor((1 - p) W), the
//     maximum never; the kept ones are a prefix of the slots;
//   * the race: the largest e / (-ln u) among the kept survivors, the lowest index on ties.
// Exact when the k-th key is strictly above the largest y a dropped element can have (ylim).
// Returns false (uniformly over the workgroup) when the row must take the general path.
__device__ __forceinline__ bool row_tail_small(const KArgs& a, RowSmem& sm, int r, const RowP& prm,
                                               int k, int total, uint32_t seed, bool sampling,
                                               bool short_ok) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool mine = tid < total;
    const uint64_t myk = mine ? sm.pk64[tid] : 0ull;
    // every candidate's uniform is loaded now, so that the latency overlaps the rank count; the
    // 64 largest candidates store theirs once ranked
    float u_mine = 0.5f;
    if (sampling && mine) u_mine = row_uniform(a, r, (int)(uint32_t)myk);
    {
        // Waves split the count as (group of 64 candidates, range of keys) pairs, 8 keys per
        // step with 128-bit LDS reads, and add their partial counts into LDS.  Unpacked slots
        // hold key 0 and never count.
        const int ngrp = (total + kWave - 1) >> 6;
        const int nspl = ngrp > 0 ? small_div(kRowWaves, ngrp) : 0;
        if (wave < ngrp * nspl) {
            const int sp = small_div(wave, ngrp), g = wave - sp * ngrp;
            const int c = g * kWave + lane;
            const uint64_t kc = sm.pk64[c];
            const int chunk = (small_div(total + nspl - 1, nspl) + 7) & ~7;
            const int j0 = sp * chunk, j1 = min(j0 + chunk, (total + 7) & ~7);
            const uint4* p4 = reinterpret_cast<const uint4*>(sm.pk64);
            uint32_t cnt = 0;
            for (int j = j0; j < j1; j += 8) {
                const uint4 a0 = p4[j / 2], a1 = p4[j / 2 + 1], a2 = p4[j / 2 + 2], a3 = p4[j / 2 + 3];
                const uint64_t v[8] = {((uint64_t)a0.y << 32) | a0.x, ((uint64_t)a0.w << 32) | a0.z,
                                       ((uint64_t)a1.y << 32) | a1.x, ((uint64_t)a1.w << 32) | a1.z,
                                       ((uint64_t)a2.y << 32) | a2.x, ((uint64_t)a2.w << 32) | a2.z,
                                       ((uint64_t)a3.y << 32) | a3.x, ((uint64_t)a3.w << 32) | a3.z};
#pragma unroll
                for (int i = 0; i < 8; ++i) cnt += v[i] > kc;
            }
            if (c < total && cnt) atomicAdd(&sm.crank[c], cnt);
        }
    }
    // every threshold used (raw keys), and the largest y an element below them can have (-inf
    // when only NaNs were dropped; with the soft cap, a bound on it)
    const uint32_t tmax = seed > sm.tmaxk ? seed : sm.tmaxk;
    float vlim = val_of(tmax - 1u);
    if (a.softcap > 0.0f) {
        vlim = softcap_bound(vlim, a.inv_softcap, a.softcap);
        if (a.softcap_f16) vlim = round_f16(vlim);  // the rounding is monotone: still a bound
    }
    const float ylim = tmax > 0x007FFFFFu ? (sampling ? vlim / prm.T : vlim) : -__builtin_inff();
    __syncthreads();
    // the uniforms of the 64 largest candidates are stored into their slots once wave 0 is
    // about to race
    const uint32_t mpos = mine ? sm.crank[tid] : 0xFFFFFFFFu;
    if (mine) {
        const uint32_t pos = mpos;
        if (pos <= (uint32_t)kWave) sm.tk[pos] = myk;
        const uint32_t yk = (uint32_t)(myk >> 32);
        // the k-th key must lie strictly above every dropped element (ties included)
        if (pos == (uint32_t)(k - 1) && yk != 0u && !(val_of(yk) > ylim)) atomicOr(&sm.status, 4u);
    }
    __syncthreads();
    // tie or hash overflow, a k-th key not above a dropped element, or fewer than k candidates
    // with a threshold used
    if (sm.status != 0u || (tmax != 0u && total < k && !(short_ok && tmax == 0x00800000u))) return false;
    const uint64_t top = total > 0 ? sm.tk[0] : 0ull;
    if (!sampling) {
        // greedy: the lowest index at the maximum of the processed logits (0 without candidates)
        if (tid == 0) {
            const int32_t tok = (top >> 32) != 0ull ? (int32_t)(0x7FFFFFFFu - (uint32_t)top) : 0;
            a.sampled[r] = tok;
            if (a.flags) a.flags[r] = VWS_FLAG_GREEDY;
            if (a.nkept) a.nkept[r] = 1;
            // for row_logprobs_entry: the token, 64-bit packing, greedy, the largest threshold
            sm.lpk[0] = (uint32_t)tok; sm.lpk[1] = 1u; sm.lpk[2] = 1u; sm.lpk[3] = tmax;
        }
        return true;
    }
    const uint32_t y0k = (uint32_t)(top >> 32);
    const float m = y0k ? val_of(y0k) : __builtin_nanf("");
    if (!(m > -__builtin_inff() && m < __builtin_inff())) return false;  // degenerate row
    // fewer candidates than k (no threshold used): every candidate is in the top k
    const uint32_t ykth = total >= k ? (uint32_t)(sm.tk[k - 1] >> 32) : 0u;
    if (total > kWave && (uint32_t)(sm.tk[kWave] >> 32) >= ykth) return false;  // > 64 tied members
    auto store_u = [&]() __attribute__((always_inline)) {
        if (sampling && mpos < (uint32_t)kWave) sm.tu[mpos] = u_mine;
    };
    if (wave != 0) {
        store_u();
        __syncthreads();
        return true;
    }

    const bool have = lane < total;
    const uint64_t key = have ? sm.tk[lane] : 0ull;
    const uint32_t yk = (uint32_t)(key >> 32);
    const float y = val_of(yk);
    const float lp_min = (prm.min_p > 0.0f) ? log_det(prm.min_p < 1.0f ? prm.min_p : 1.0f)
                                            : -__builtin_inff();
    const bool keep = have && yk >= ykth && (y - m) >= lp_min;
    const float e = keep ? exp_det(y - m) : 0.0f;
    const uint64_t w = keep ? mass_of(e) : 0ull;
    uint64_t C = w, W = w;
#pragma unroll
    for (int s = 1; s < kWave; s <<= 1) {
        const uint64_t t = lane_xor64(W, s);
        if (!(lane & s)) C += t;
        W += t;
    }
    const float q32 = 1.0f - prm.top_p;
    const bool topp = q32 > 0.0f;
    const bool abl = topp && !(q32 < 1.0f);  // top_p <= 0: only the maximum is kept
    const uint64_t thr = (topp && !abl) ? scale_floor(q32, W) : 0ull;
    const bool removed = keep && topp && (abl ? (C != W) : (C <= thr && C != W));
    const bool kept = keep && !removed;
    store_u();
    __syncthreads();
    const float uu = have ? sm.tu[lane] : 0.5f;
    // race: key bits + 1 (0 = no valid key) reduced as 32-bit maxima; the lowest index wins
    // among equal keys, and the best key of the other lanes is the runner-up
    const float rkey = e / (0.0f - log_det(uu));
    const uint32_t kb = (kept && rkey >= 0.0f) ? f2u(rkey) + 1u : 0u;
    const uint32_t kmax = wave_max_u32(kb);
    const uint64_t at = wave_ballot(kb == kmax && kmax != 0u);
    int win = -1;
    uint32_t widx = 0u;
    if (at) {
        win = (int)__builtin_ctzll(at);
        widx = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, win);
        if (at & (at - 1ull)) {  // equal keys: the lowest index
            widx = wave_min_u32(((at >> lane) & 1ull) ? (uint32_t)key : 0xFFFFFFFFu);
            win = (int)__builtin_ctzll(wave_ballot(((at >> lane) & 1ull) && (uint32_t)key == widx));
        }
    }
    const uint32_t second = wave_max_u32(lane != win ? kb : 0u);
    const int nkept = __popcll(wave_ballot(kept));
    const int nrem = __popcll(wave_ballot(removed));
    const uint64_t cat = readlane64(C, nkept - 1);              // smallest kept cumulative mass
    const uint64_t cprev = nrem ? readlane64(C, nkept) : 0ull;  // largest removed one
    if (lane == 0) {
        int32_t tok;
        uint32_t fl = 0;
        if (kmax) {
            tok = (int32_t)widx;
            const float bk = u2f(kmax - 1u);
            if (second) {
                const float sk = u2f(second - 1u);
                if ((double)sk >= (double)bk * (1.0 - 1e-6)) fl |= VWS_FLAG_RACE_NEAR_TIE;
            }
        } else {
            tok = (int32_t)(uint32_t)top;  // no valid race key: the largest (y, index) kept
        }
        if (topp && !abl) {
            const uint64_t tol = (uint64_t)((double)W * 1e-6);
            if ((nrem > 0 && thr - cprev <= tol) || (cat > thr && cat - thr <= tol))
                fl |= VWS_FLAG_TOPP_NEAR_TIE;
        }
        a.sampled[r] = tok;
        if (a.flags) a.flags[r] = fl;
        if (a.nkept) a.nkept[r] = nkept;
        sm.lpk[0] = (uint32_t)tok; sm.lpk[1] = 1u; sm.lpk[2] = 0u; sm.lpk[3] = tmax;
    }
    return true;
}

// Serves greedy and top-k rows; returns false when the row must take the general path (nothing
// has been written for it then); *topp_row tells whether the single-pass top-p path may serve
// the row instead.  LP (launches with raw logprobs): the stream also sums exp(x - a) over every
// element (a the wave's largest value of its first iteration), the candidates keep their raw
// keys, and the threshold keeps at least max(k, L) candidates, so that row_logprobs_entry can
// finish the logprobs from the candidates.  MASK (launches with an allowed-token mask) without
// LP (SM): every element outside the row's mask becomes -inf as it is loaded, before the seed
// and the threshold see it.  One mask word per lane and iteration covers the wave's whole
// iteration (U vectors of 64 lanes x VEC elements = 64 words; row starts 16-byte aligned), and
// each lane takes its vector's bits from the lane that loaded them (ds_bpermute).  MASK with LP
// (CM): the stream keeps raw values (the logprobs are of the raw logits), and each candidate is
// masked at its pack.
template <typename T, bool LP, bool MASK>
__device__ __forceinline__ bool row_fast(const KArgs& a, RowSmem& sm, int r, const void* logits,
                                         int64_t lstride, int V, bool* topp_row) {
    constexpr int NT = kRowThreads;
    constexpr int VEC = Elem<T>::kVec;
    constexpr int U = 32 / VEC;  // 16-byte loads in flight per lane per iteration
    constexpr bool SM = MASK && !LP, CM = MASK && LP;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const T* row = reinterpret_cast<const T*>(logits) + (size_t)r * lstride;
    // position of this lane in the workgroup, recomputed where the streaming loop needs it
    auto tid_now = [&]() __attribute__((always_inline)) { return wave * kWave + lane_now(); };

    // 1. loads, none behind a branch (a load that only some paths issue makes the wait for
    //    everything before it conservative): the first iteration of logits (it needs only the
    //    preloaded arguments), the history ids and processor lists (zero-sized buffers when
    //    absent), the second iteration, then the parameters as scalar loads.
    //    Buffer loads: loads past the end of the row read zeros (range-checked vector offsets),
    //    so nothing is clamped.
    //    The row addresses are computed without branches (an absent list gets a zero-sized
    //    buffer, whatever its address), so that the kernel arguments are read in one batch.
    // LP: the row's parameters first.  Launches with logprobs also hold rows the single pass does
    // not serve (top-p without top-k: most of such a batch); those must not issue the first two
    // iterations (256 KB of fp32 logits) only to stream the row again on the top-p path.
    // Without logprobs the first loads wait for no argument read.
    if (LP) {
        const RowP p0 = row_params_scalar(a, r);
        if (fast_k<CM>(a, p0) == 0) {
            *topp_row = topp_eligible(a, p0);
            return false;
        }
    }
    Slice<T> sl;
    sl.init(row, 0, V);
    const int nbody = sl.nbody;
    const int nit = (nbody + NT * U - 1) / (NT * U);
    const __amdgpu_buffer_rsrc_t lrs = make_rsrc(row + sl.a, 16u * (uint32_t)nbody);
    float A[U][VEC], Bq[U][VEC];
    // Vectors past the body read zeros; consumers skip them (vi >= nbody).  The whole byte
    // offset is the vector offset (the scalar offset is 0): a raw buffer access is out of range,
    // returns zeros and fetches nothing when its vector offset plus instruction offset is at or
    // past the resource's num_records, so the prefetches past the row's end never leave the row.
    // The loads are non-temporal (nt): the row is read once, and streaming it with the default
    // policy evicts the kernel's own code and small operands from L2 and the infinity cache.
    auto load_part = [&](float (&buf)[U][VEC], int it, auto keep, int q0, int q1) __attribute__((always_inline)) {
#pragma unroll
        for (int q = q0; q < q1; ++q) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(
                lrs, 16u * (uint32_t)(tid_now() + (it * U + q) * NT), 0u, decltype(keep)::value ? 0 : kLoadNT);
            Elem<T>::from_words((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3], buf[q]);
        }
    };
    auto load_iter = [&](float (&buf)[U][VEC], int it, auto keep) __attribute__((always_inline)) {
        load_part(buf, it, keep, 0, U);
    };
    // the first half of the first iteration depends only on the preloaded arguments: issued
    // before anything waits for the rest of the kernel arguments; the history ids follow it
    // and the rest of the iteration follows them, so the history hash is built while that
    // rest is still arriving (a wait for a load waits for every load issued before it)
    load_part(A, 0, BoolC<true>{}, 0, U / 2);
    __builtin_amdgcn_sched_barrier(0);
    const bool has_p = a.prompt && a.pwidth > 0, has_o = a.output && a.owidth > 0;
    const bool has_a = a.adj_ids && a.adjwidth > 0;
    const uint64_t ru = (uint64_t)r;
    const int32_t* aidrow = reinterpret_cast<const int32_t*>((uint64_t)a.adj_ids + 4u * ru * (uint64_t)a.adjstride);
    const float* avrow = reinterpret_cast<const float*>((uint64_t)a.adj_vals + 4u * ru * (uint64_t)a.adjstride);
    const int32_t* prow = reinterpret_cast<const int32_t*>((uint64_t)a.prompt + 4u * ru * (uint64_t)a.pstride);
    const int32_t* orow = reinterpret_cast<const int32_t*>((uint64_t)a.output + 4u * ru * (uint64_t)a.ostride);
    const __amdgpu_buffer_rsrc_t prs = make_rsrc(prow, has_p ? 4u * (uint32_t)a.pwidth : 0u);
    const __amdgpu_buffer_rsrc_t ors = make_rsrc(orow, has_o ? 4u * (uint32_t)a.owidth : 0u);
    const int hp_raw = __builtin_amdgcn_raw_buffer_load_b32(prs, 4u * (uint32_t)tid, 0u, 0);
    const int ho_raw = __builtin_amdgcn_raw_buffer_load_b32(ors, 4u * (uint32_t)tid, 0u, 0);
    const __amdgpu_buffer_rsrc_t ais = make_rsrc(aidrow, has_a ? 4u * (uint32_t)a.adjwidth : 0u);
    const __amdgpu_buffer_rsrc_t avs = make_rsrc(avrow, has_a ? 4u * (uint32_t)a.adjwidth : 0u);
    const int ha_id = __builtin_amdgcn_raw_buffer_load_b32(ais, 4u * (uint32_t)tid, 0u, 0);
    const float ha_val = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(avs, 4u * (uint32_t)tid, 0u, 0));
    __builtin_amdgcn_sched_barrier(0);
    load_part(A, 0, BoolC<true>{}, U / 2, U);
    // SM: the row's allowed-token words; lane l loads word l of the wave's share of an
    // iteration (vector l / (2 VEC), word l % (2 VEC) of it); words past the mask read 0
    const uint32_t* mrow = SM ? a.allowed + (size_t)r * (size_t)a.astride : nullptr;
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(mrow, SM ? 4u * (uint32_t)((V + 31) >> 5) : 0u);
    auto load_mask = [&](uint32_t& mw, int it) __attribute__((always_inline)) {
        if (SM) {
            const int ln = lane_now();
            const uint32_t wi = (uint32_t)((((it * U + ln / (2 * VEC)) * NT + wave * kWave) * VEC) >> 5) +
                                (uint32_t)(ln % (2 * VEC));
            mw = __builtin_amdgcn_raw_buffer_load_b32(mrs, 4u * wi, 0u, 0);
        }
    };
    // elements of buf outside the mask become -inf (mw: this lane's word of the iteration)
    auto mask_iter = [&](float (&buf)[U][VEC], uint32_t mw) __attribute__((always_inline)) {
        if (SM) {
            const int ln = lane_now();
#pragma unroll
            for (int q = 0; q < U; ++q) {
                const int src = q * 2 * VEC + ((ln * VEC) >> 5);
                const uint32_t w = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)mw);
                const uint32_t bits = w >> ((ln * VEC) & 31);
#pragma unroll
                for (int j = 0; j < VEC; ++j) buf[q][j] = ((bits >> j) & 1u) ? buf[q][j] : -__builtin_inff();
            }
        }
    };
    uint32_t MA = 0u, MB = 0u;
    load_mask(MA, 0);
    load_iter(Bq, 1, BoolC<false>{});
    load_mask(MB, 1);
    const RowP prm = row_params_scalar(a, r);
    const int k = fast_k<CM>(a, prm);
    VWS_TRACE_MARK_AFTER(a, VWS_TRACE_PARAMS, k);
    if (k == 0) {
        // SM: the top-p stream masks by whole words only for rows that start 16-byte aligned
        *topp_row = topp_eligible(a, prm) && !(SM && sl.a != 0);
        return false;
    }
    // raw logprobs are of the capped logits, which this stream does not compute (the top-p
    // path's does: greedy rows with logprobs go there)
    if (LP && a.softcap > 0.0f) {
        *topp_row = topp_eligible(a, prm);
        return false;
    }
    // SM: the mask words line up with the vectors only when the row starts 16-byte aligned
    if (SM && sl.a != 0) return false;
    // the threshold keeps at least kc candidates: the top-L raw logits must be among them
    const int kc = LP ? max(k, a.L) : k;
    const bool hh = prm.has_hist;     // penalties
    const bool hx = prm.need_hash;    // penalties or logits processors
    // processors and penalties that never raise a logit let hashed candidates be found by their
    // raw value (a positive logit bias is only seen once the hash is built)
    const bool mono = !hh || (prm.rep >= 1.0f && prm.pres >= 0.0f && prm.freq >= 0.0f);
    // penalties that may raise a logit need every penalised token up front, which a token-state
    // table cannot list: the multi-pass path serves such rows
    if (prm.tab && !mono) return false;
    // the row's token-state words (read at the candidates only)
    const uint32_t* tabrow = prm.tab ? a.tstate + (size_t)prm.trow * (size_t)a.tstride : nullptr;
    const int32_t* pr = hh && prm.np > 0 ? prow : nullptr;
    const int32_t* ou = hh && prm.no > 0 ? orow : nullptr;

    // 2. LDS state and the history hash
    if (tid == 0) {
        sm.tau = 0u; sm.status = 0u; sm.nhash = 0u; sm.nkeep = 0u; sm.npack = 0u; sm.bc[4] = 0u;
        sm.ymax = 0u; sm.tmaxk = 0u;
        sm.pmode = (hx || prm.tab) ? 1u : 0u;
        sm.phash = hx ? 1u : 0u;
        sm.ptab = (uint64_t)tabrow;
        sm.adjraise = 0u;
        sm.prep = prm.rep; sm.pinv = prm.inv_rep; sm.ppres = prm.pres; sm.pfreq = prm.freq;
        sm.plp = LP ? 1u : 0u;
        if (LP)
            for (int i = 0; i < 8; ++i) sm.lpk[i] = 0u;
    }
    if (hx) {
        for (int s = tid; s < kRowHash; s += NT) { sm.hkey[s] = 0u; sm.hval[s] = 0u; }
        for (int s = tid; s < kRowHashBits / 128; s += NT)
            reinterpret_cast<uint4*>(sm.hbits)[s] = make_uint4(0u, 0u, 0u, 0u);
    }
    sm.pk64[tid] = 0ull;  // unpacked slots keep key 0, which ranks below every candidate
    sm.crank[tid] = 0u;
    if (tid < kRowKeep) sm.sC[tid] = 0ull;
    if (tid == 0) sm.sW = 0ull;
    __syncthreads();
    if (hh) {
        if (tid < prm.np && hp_raw >= 0 && hp_raw < V) rhash_insert(sm, hp_raw, 0x80000000u);
        if (tid < prm.no && ho_raw >= 0 && ho_raw < V) rhash_insert(sm, ho_raw, 1u);
        if (pr) {
            for (int i = NT + tid; i < prm.np; i += NT) {
                const int t = pr[i];
                if (t >= 0 && t < V) rhash_insert(sm, t, 0x80000000u);
            }
        }
        if (ou) {
            for (int i = NT + tid; i < prm.no; i += NT) {
                const int t = ou[i];
                if (t >= 0 && t < V) rhash_insert(sm, t, 1u);
            }
        }
    }
    if (prm.na > 0) {
        auto add = [&](int t, float bv) {
            if (t < 0 || t >= V) return;
            if (bv == -__builtin_inff()) {
                rhash_insert(sm, t, kHBan);
                // a ban turns a NaN logit into -inf, an element that the candidates (chosen by
                // raw value) never hold: such a row leaves for the multi-pass path (bit 1, as a
                // hash overflow), which bans every listed element whatever its value
                if (key_of(Elem<T>::load1(row + t)) == 0u) atomicOr(&sm.status, 1u);
            } else {
                rhash_insert(sm, t, kHBias, bv);
                if (bv > 0.0f) sm.adjraise = 1u;
            }
        };
        if (tid < prm.na) add(ha_id, ha_val);
        for (int i = NT + tid; i < prm.na; i += NT) add(aidrow[i], avrow[i]);
    }

    // 3. seed threshold from the first iteration: the m-th largest lane maximum of the sample.
    //    The sample holds lambda = (k - 1) * sample / V elements above the row's k-th value on
    //    average (about Poisson); m = ceil(lambda + 5 sqrt(lambda) + 3) puts the seed above
    //    the k-th value (the row then takes the general path) with probability at most 1.2e-6
    //    for any lambda, and keeps about m * V / sample candidates (k = 1: the sample's
    //    maximum, never above the k-th).  m = k is never above the k-th value: at least k lane
    //    maxima, so at least k elements, lie at or above the m-th largest lane maximum (and the
    //    pool's m-th largest is at most that).  So m is capped at k, which the rule exceeds when
    //    the sample is most of the row (short rows: fewer candidates, and no 256-entry pool).
    const int sample = nbody > 0 ? min(NT * U, nbody) * VEC : 0;
    const float lam = (float)(kc - 1) * (float)sample / (float)V;
    const int m_seed = sample > 0 ? min(kc, (int)__builtin_ceilf(lam + 5.0f * __builtin_sqrtf(lam) + 3.0f)) : 0;
    const bool seeded = sample > 0 && m_seed <= kRowWaves * kSeedPerWave;
    // m <= 64: the pool is every wave's 4 largest lane maxima, otherwise the 16 largest of every
    // wave, whose m-th largest wave 0 selects
    const bool small_pool = m_seed <= kRowWaves * 4;
    // LP: the wave's anchor, its largest value over the first iteration (0 when it has none
    // that is finite), so that its sum of exp(x - anchor) starts near 1 and cannot overflow
    // unless a later value lies ~88 above it (the row then takes the multi-pass path)
    mask_iter(A, MA);
    float aw = 0.0f;
    if (LP) {
        float lm = __builtin_nanf("");
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const bool ok = q * NT + tid < nbody;
#pragma unroll
            for (int j = 0; j < VEC; ++j) lm = ok ? fmaxf(lm, A[q][j]) : lm;
        }
        const uint32_t km = wave_max_u32(key_of(lm));
        aw = (km > 0x007FFFFFu && km < 0xFF800000u) ? val_of(km) : 0.0f;
    }
    if (seeded) {
        float mx = __builtin_nanf("");  // fmaxf ignores NaN; clamped duplicate loads are skipped
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const bool ok = q * NT + tid < nbody;
#pragma unroll
            for (int j = 0; j < VEC; ++j) mx = ok ? fmaxf(mx, A[q][j]) : mx;
        }
        if (small_pool) {
            const uint32_t t4 = wave_top4(key_of(mx));
            if (lane < 4) sm.seedk[wave * 4 + lane] = t4;
            VWS_TRACE_MARK_AFTER(a, VWS_TRACE_FIRST, t4);
        } else {
            const uint32_t sk = wave_sort_desc64(key_of(mx));
            if (lane < kSeedPerWave) sm.seedk[wave * kSeedPerWave + lane] = sk;
            VWS_TRACE_MARK_AFTER(a, VWS_TRACE_FIRST, sk);
        }
    }
    __syncthreads();  // also publishes the hash
    VWS_TRACE_MARK(a, VWS_TRACE_SEED);
    // the hash is complete here; a row whose history overflowed it takes the general path
    if (sm.status & 1u) return false;
    // Rows whose stream waits for later iterations: every wave selects a small pool's seed for
    // itself while those land.  Rows held in the first two iterations wait for nothing else:
    // wave 0 selects and the others read it after a barrier (16 waves selecting at once cost
    // their CU's issue slots, ~1.5 us).
    const bool sel0 = !small_pool || nit <= 2;
    uint32_t seed = 0u;
    if (seeded && !sel0) {
        seed = wave_mth_largest64(sm.seedk[lane], m_seed);
    } else if (seeded && small_pool && wave == 0) {
        const uint32_t t0 = wave_mth_largest64_count(sm.seedk[lane], m_seed);
        if (lane == 0) sm.bc[0] = t0;
    } else if (seeded && wave == 0) {
        const uint32_t t0 = wave_kth_largest_256(sm.seedk[4 * lane], sm.seedk[4 * lane + 1],
                                                 sm.seedk[4 * lane + 2], sm.seedk[4 * lane + 3], m_seed);
        if (lane == 0) sm.bc[0] = t0;
    }
    const bool gather = hx && (!mono || sm.adjraise != 0u);
    // something may raise a logit and the logits are capped: the general path serves the row
    if (gather && a.softcap > 0.0f) return false;
    // LP: the up-front processed values would leave the candidates without their raw keys
    if (LP && gather) return false;
    if (gather) {
        if (lane == 0) sm.pmode = 2u;  // every wave writes the same value before its stream
        for (int s = tid; s < kRowHash; s += NT) {
            const uint32_t kk = sm.hkey[s];
            if (kk) {
                const uint32_t hv = sm.hval[s] | (tabrow ? tabrow[kk - 1u] & kStateMask : 0u);
                float xr = Elem<T>::load1(row + (kk - 1u));
                if (SM && !((mrow[(kk - 1u) >> 5] >> ((kk - 1u) & 31u)) & 1u)) xr = -__builtin_inff();
                sm.hpen[s] = apply_hashed(xr, hv, sm.hadj[s], prm.rep, prm.inv_rep, prm.freq, prm.pres);
            }
        }
    }
    if (gather || (seeded && sel0)) {
        __syncthreads();
        if (seeded && sel0) seed = sm.bc[0];
    }

    // 4. stream; 5. the k-th largest candidate, checked against every threshold used.  A seeded
    //    pass whose k-th candidate lies below a threshold is streamed again without the seed.
    RowCand cb;
    auto slot = [&](float v, int idx, bool valid) __attribute__((always_inline)) {
        const bool c = valid && v >= cb.tauf;
        if (wave_ballot(c) == 0ull) return;
        cb.append(c, key_of(v), idx);  // raw value; penalties are applied by RowCand::finish
    };
    // LP: this lane's sum of exp(x - aw) = 2^(x log2 e - aw log2 e) (one fma and the hardware
    // exp2; the product aw log2 e rounded once for the whole wave, which scales every term of
    // the wave alike and is undone exactly by the rescale in row_logprobs_entry; each
    // iteration's float partial sum added in double)
    const float awc = aw * kLog2e;
    double lacc = 0.0;
    // One vector (VEC elements per lane) at a time: the lane maximum against the threshold
    // decides for the whole wave whether any element of the vector is examined one by one.
    // SM: the first iteration was masked whole (the seed needs it); later ones are masked
    // only where a vector passes the threshold by its raw values (a masked value is at most
    // its raw one), which on rows the mask leaves mostly open is a few vectors per iteration
    auto examine = [&](float (&buf)[U][VEC], uint32_t mw, int it) __attribute__((always_inline)) {
        cb.refresh();
        const int t = tid_now();
        float lit = 0.0f;
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const int vi = (it * U + q) * NT + t;
            const bool ok = vi < nbody;
            if (LP) {
                float tq = 0.0f;
#pragma unroll
                for (int j = 0; j < VEC; ++j) tq += __builtin_amdgcn_exp2f(__builtin_fmaf(buf[q][j], kLog2e, -awc));
                lit += ok ? tq : 0.0f;
            }
            float mq = buf[q][0];
#pragma unroll
            for (int j = 1; j < VEC; ++j) mq = fmaxf(mq, buf[q][j]);
            uint64_t hm = wave_ballot(ok && mq >= cb.tauf);
            if (__builtin_expect(hm == 0ull, 1)) continue;
            if (SM && it > 0) {
                const int ln = lane_now();
                const int src = q * 2 * VEC + ((ln * VEC) >> 5);
                const uint32_t w = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)mw);
                const uint32_t bits = w >> ((ln * VEC) & 31);
#pragma unroll
                for (int j = 0; j < VEC; ++j) buf[q][j] = ((bits >> j) & 1u) ? buf[q][j] : -__builtin_inff();
                mq = buf[q][0];
#pragma unroll
                for (int j = 1; j < VEC; ++j) mq = fmaxf(mq, buf[q][j]);
                hm = wave_ballot(ok && mq >= cb.tauf);
                if (hm == 0ull) continue;
            }
            cb.template append_vec<VEC>(buf[q], sl.a + vi * VEC, hm);
        }
        if (LP) lacc += (double)lit;
    };
    // The same examination, after which each vector's registers take vector q of iteration nxt
    // at once (run: examine iteration it at all), so the next loads leave as soon as their
    // registers are free.  Used by the masked kernel and the 16-bit kernels without logprobs:
    // measured faster there (C3 with one masked row 36.5 -> 34.0 us, C4 164.2 -> 161.0 us) and
    // slower in the fp32 plain and logprob kernels (C3 +0.8 us, C3 + 20 logprobs +2.7 us).
    constexpr bool REFILL = SM || (!LP && VEC == 8);
    auto examine_pv = [&](float (&buf)[U][VEC], uint32_t mw, int it, int nxt, bool run) __attribute__((always_inline)) {
        if (run) cb.refresh();
        const int t = tid_now();
#pragma unroll
        for (int q = 0; q < U; ++q) {
            // (a continue leaves the do-while: the vector has nothing at or above the threshold)
            if (run) do {
                const int vi = (it * U + q) * NT + t;
                const bool ok = vi < nbody;
                float mq = buf[q][0];
#pragma unroll
                for (int j = 1; j < VEC; ++j) mq = fmaxf(mq, buf[q][j]);
                uint64_t hm = wave_ballot(ok && mq >= cb.tauf);
                if (__builtin_expect(hm == 0ull, 1)) continue;
                if (SM && it > 0) {
                    const int ln = lane_now();
                    const int src = q * 2 * VEC + ((ln * VEC) >> 5);
                    const uint32_t w = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)mw);
                    const uint32_t bits = w >> ((ln * VEC) & 31);
#pragma unroll
                    for (int j = 0; j < VEC; ++j) buf[q][j] = ((bits >> j) & 1u) ? buf[q][j] : -__builtin_inff();
                    mq = buf[q][0];
#pragma unroll
                    for (int j = 1; j < VEC; ++j) mq = fmaxf(mq, buf[q][j]);
                    hm = wave_ballot(ok && mq >= cb.tauf);
                    if (hm == 0ull) continue;
                }
                cb.template append_vec<VEC>(buf[q], sl.a + vi * VEC, hm);
            } while (0);
            load_part(buf, nxt, BoolC<false>{}, q, q + 1);
        }
    };
    const bool sampling = !prm.greedy;
    // With the soft cap the buffer keeps raw values throughout (the cap is applied at the pack),
    // so it is never cut by processed values: a full buffer sends the row to the general path.
    const bool capped = a.softcap > 0.0f;
    // The check after the stream bounds the capped value of everything below the threshold by
    // the capped threshold plus a margin (softcap_bound); a seed at an element's own value
    // would leave that element, often the k-th, inside the margin.  The seed is lowered below
    // it by twice the margin in capped units.
    if (capped && seed > 0x007FFFFFu)
        seed = key_of(softcap_lower(val_of(seed), a.inv_softcap, a.softcap));
    // SM: the elements outside the mask are -inf; the threshold admits finite values only
    // (the smallest key above -inf), so that they never become candidates
    if (SM && seed < 0x00800000u) seed = 0x00800000u;
    // Fewer candidates than k are exact when no threshold was used.  With the finite-only
    // threshold alone (SM), every finite value is a candidate and the top k also holds every
    // -inf element (y = -inf >= the k-th value): those have zero mass, fail min-p, are removed
    // by top-p when it is on (their cumulative mass 0 is at most the cut; the near-tie term they
    // would add needs 1 - p within 2e-6 of 0, which is left to the multi-pass path), and lose
    // every race, so they change nothing when min-p or top-p is on.
    const bool short_ok = SM && seed == 0x00800000u &&
                          (prm.min_p > 0.0f || (1.0f - prm.top_p) > 2e-6f);
    cb.init(wave, kc, !capped);
    cb.set_tau(seed);
    if (gather) {
        constexpr int per = kRowHash / kRowWaves;
        for (int s0 = wave * per; s0 < (wave + 1) * per; s0 += kWave) {
            const int s = s0 + lane;
            const uint32_t kk = sm.hkey[s];
            const uint32_t pk = kk ? key_of(sm.hpen[s]) : 0u;
            cb.append(pk != 0u && pk >= cb.tau, pk, (int32_t)((kk - 1u) | 0x80000000u));
        }
    }
    if (REFILL) {
        for (int it = 0; it < nit && !cb.ovf; it += 2) {
            examine_pv(A, MA, it, it + 2, true);
            load_mask(MA, it + 2);
            examine_pv(Bq, MB, it + 1, it + 3, it + 1 < nit && !cb.ovf);
            load_mask(MB, it + 3);
        }
    } else {
        for (int it = 0; it < nit && !cb.ovf; it += 2) {
            examine(A, MA, it);
            load_iter(A, it + 2, BoolC<false>{});
            load_mask(MA, it + 2);
            if (it + 1 < nit && !cb.ovf) examine(Bq, MB, it + 1);
            load_iter(Bq, it + 3, BoolC<false>{});
            load_mask(MB, it + 3);
        }
    }
    VWS_TRACE_MARK_AFTER(a, VWS_TRACE_WAVE_LOOP, cb.cnt);
    if (wave == 0) {
        // unaligned head (thread 0) and tail (thread 1), fewer than 2 vectors in total; handled
        // last, and by wave 0 alone, so no other wave waits for its loads
        float v[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[j] = __builtin_nanf("");
        int i0 = 0;
        if (tid <= 1) i0 = sl.load_edge(tid, v);
        const int end = tid == 0 ? sl.a : V;
        if (SM && tid <= 1) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const int t = i0 + j;
                if (t < end && !((mrow[t >> 5] >> (t & 31)) & 1u)) v[j] = -__builtin_inff();
            }
        }
#pragma unroll
        for (int j = 0; j < VEC; ++j) slot(v[j], i0 + j, tid <= 1 && i0 + j < end);
        if (LP) {
#pragma unroll
            for (int j = 0; j < VEC; ++j)
                if (tid <= 1 && i0 + j < end) lacc += (double)__builtin_amdgcn_exp2f(__builtin_fmaf(v[j], kLog2e, -awc));
        }
    }
    if (LP) {
        // the wave's sum (a NaN or an overflow sends the row to the multi-pass path)
        double sw = lacc;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) sw += __shfl_xor(sw, o, kWave);
        if (lane == 0) {
            sm.lpS[wave] = sw;
            sm.lpA[wave] = awc;  // the wave's terms are 2^(x log2 e - awc)
            if (!(sw < 1e300)) atomicOr(&sm.status, 16u);
        }
    }
    // each wave packs its candidates into the row's arrays as soon as its own stream ends, while
    // other waves are still streaming: the key of y (the processed logit over T; the processed
    // logit itself for greedy rows) and the index.  Rows with k <= 64 pack one 64-bit key per
    // candidate, (key(y) << 32) | index, with the index reversed for greedy rows so that the
    // largest key is the lowest index at the maximum; their uniforms are loaded for the 64
    // largest keys only, once ranked.  Larger k load the uniform of every candidate here (that
    // of each lane's first candidate is stored once the ranks are counted, so that its latency
    // overlaps the count).
    const float Tt = prm.T;
    const bool small = k <= kWave;
    float u_first = 0.0f;
    int u_slot = -1;
    if (!cb.ovf) {
        // Mode 2 (something may raise a logit) drops the stream entries of hashed tokens, which
        // compacts the buffer: done out of line.  In mode 1 the processed value of each hashed
        // candidate not yet fixed by a compaction replaces its raw value here, found through
        // the presence bits with one LDS read per candidate.
        const uint32_t pmode = sm.pmode;
        uint32_t ymx = 0u;
        // CM: the row's mask lowers each masked candidate to -inf at its pack.  A mask only
        // lowers values, so every element below the thresholds stays below them; a masked
        // candidate that reaches the top k fails the exactness check (multi-pass path).
        const uint32_t* cmrow = CM ? a.allowed + (size_t)r * (size_t)a.astride : nullptr;
        // one candidate: its processed value (cap, then the hashed processors and penalties
        // unless a compaction has applied them) and its packed entry at slot pos
        auto pack_one = [&](int pos, uint32_t kx, int32_t ii, bool fixed, bool first)
            __attribute__((always_inline)) {
            // LP: the raw key of every packed candidate (the soft cap and up-front processed
            // values never occur with LP; a compaction that processed keys set status bit 8)
            if (LP) reinterpret_cast<uint32_t*>(sm.hpen)[pos] = kx;
            if (capped) kx = key_of(softcap_out(val_of(kx), a.inv_softcap, a.softcap, a.softcap_f16 != 0));
            if (CM && !((cmrow[(uint32_t)ii >> 5] >> (ii & 31)) & 1u)) kx = key_of(-__builtin_inff());
            if (!fixed) {
                const int hs = (hx && rhash_maybe(sm, ii)) ? rhash_find(sm, ii) : -1;
                uint32_t hv = hs >= 0 ? sm.hval[hs] : 0u;
                if (tabrow) hv |= tabrow[ii] & kStateMask;
                if (hs >= 0 || hv != 0u)
                    kx = key_of(apply_hashed(val_of(kx), hv, hs >= 0 ? sm.hadj[hs] : 0.0f, sm.prep,
                                             sm.pinv, sm.pfreq, sm.ppres));
            }
            const uint32_t ky = sampling ? key_of(val_of(kx) / Tt) : kx;
            if (small) {
                sm.pk64[pos] = ((uint64_t)ky << 32) | (uint32_t)(sampling ? ii : 0x7FFFFFFF - ii);
            } else {
                ymx = ky > ymx ? ky : ymx;
                sm.pkey[pos] = ky;
                sm.pidx[pos] = ii;
                if (sampling) {
                    if (first) {
                        u_slot = pos;  // loaded below, stored once the ranks are counted
                    } else {
                        sm.pu[pos] = row_uniform(a, r, ii);
                    }
                }
            }
        };
        if (pmode != 2u && cb.cnt <= kWave) {
            // at most one entry per lane: dropped below the threshold and packed from registers
            const bool have = lane < cb.cnt;
            const uint32_t kx = have ? sm.ckey[wave][lane] : 0u;
            const int32_t ii = have ? sm.cidx[wave][lane] : 0;
            const bool keep = kx != 0u && kx >= cb.tau;
            const uint64_t bal = wave_ballot(keep);
            uint32_t b = 0;
            if (lane == 0) b = atomicAdd(&sm.npack, (uint32_t)__popcll(bal));
            const int pbase = __builtin_amdgcn_readlane(b, 0);
            if (keep && pbase + __popcll(bal) <= kRowPack) {
                pack_one(pbase + lane_prefix(bal), kx, ii, pmode == 0u || lane < cb.nfix, true);
                if (sampling && !small) u_first = row_uniform(a, r, ii);
            }
        } else {
            cb.filter();
            const int nfix = pmode == 1u ? cb.nfix : cb.cnt;
            if (pmode == 2u) cb.finish();
            uint32_t b = 0;
            if (lane == 0) b = atomicAdd(&sm.npack, (uint32_t)cb.cnt);
            const int pbase = __builtin_amdgcn_readlane(b, 0);
            if (pbase + cb.cnt <= kRowPack) {
                // e = lane first (its uniform stays in flight), then any further candidates
                for (int e = lane; e < cb.cnt; e += kWave)
                    pack_one(pbase + e, sm.ckey[wave][e], sm.cidx[wave][e], e < nfix, e == lane);
                // the first candidate's uniform, loaded outside the loop so that nothing waits
                // for it before it is stored
                if (sampling && !small && u_slot >= 0)
                    u_first = row_uniform(a, r, sm.cidx[wave][lane]);
            }
        }
        if (!small) {
            ymx = wave_max_u32(ymx);
            if (lane == 0 && ymx) atomicMax(&sm.ymax, ymx);
        }
    }
    if (lane == 0) {
        atomicMax(&sm.tmaxk, cb.tau);
        if (cb.ovf) atomicOr(&sm.status, 2u);
    }
    VWS_TRACE_MARK(a, VWS_TRACE_WAVE_PACK);
    __syncthreads();
    VWS_TRACE_MARK(a, VWS_TRACE_STREAM);
    const int total = (int)sm.npack;
    if (total > kRowPack) return false;  // too many candidates
    // the single-wave finish checks the status and the thresholds once its count is running
    if (small) return row_tail_small(a, sm, r, prm, k, total, seed, sampling, short_ok);
    if (sm.status != 0u) return false;  // tie or hash overflow
    const uint32_t tmax = seed > sm.tmaxk ? seed : sm.tmaxk;  // every threshold used (raw keys)
    // fewer than k candidates can only be exact when no threshold was used
    if (tmax != 0u && total < k && !(short_ok && tmax == 0x00800000u)) return false;
    // the largest y an element below the thresholds can have (with the soft cap, a bound on
    // it); -inf when only NaNs were dropped
    float vlim = val_of(tmax - 1u);
    if (capped) {
        vlim = softcap_bound(vlim, a.inv_softcap, a.softcap);
        if (a.softcap_f16) vlim = round_f16(vlim);  // the rounding is monotone: still a bound
    }
    const float ylim = tmax > 0x007FFFFFu ? (sampling ? vlim / Tt : vlim) : -__builtin_inff();
    const bool mine = tid < total;

    // 5. ranks in y: candidate c's rank is the number of candidate keys above its own, so the
    //    top k (ties included) are exactly the candidates of rank < k.  Waves split the count
    //    as (group of 64 candidates, range of keys) pairs, 16 keys per step with 128-bit LDS
    //    reads, and add their partial ranks into LDS.  Slots past the packed candidates hold
    //    key 0 and never count.
    const uint32_t mk = sm.ymax;                              // largest y
    const uint32_t myk = mine ? sm.pkey[tid] : 0u;
    if (tid == 0) sm.nkeep = 0u;
    {
        const int ngrp = (total + kWave - 1) >> 6;
        const int nspl = ngrp > 0 ? small_div(kRowWaves, ngrp) : 0;
        if (wave < ngrp * nspl) {
            const int sp = small_div(wave, ngrp), g = wave - sp * ngrp;
            const int c = g * kWave + lane;
            const uint32_t kc = sm.pkey[c];
            const int chunk = (small_div(total + nspl - 1, nspl) + 15) & ~15;
            const int j0 = sp * chunk, j1 = min(j0 + chunk, (total + 15) & ~15);
            const uint4* p4 = reinterpret_cast<const uint4*>(sm.pkey);
            uint32_t cnt = 0;
            for (int j = j0; j < j1; j += 16) {
                const uint4 a0 = p4[j / 4], a1 = p4[j / 4 + 1], a2 = p4[j / 4 + 2], a3 = p4[j / 4 + 3];
                const uint32_t v[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                                        a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
#pragma unroll
                for (int i = 0; i < 16; ++i) cnt += v[i] > kc;
            }
            if (c < total && cnt) atomicAdd(&sm.crank[c], cnt);
        }
    }
    __syncthreads();
    // Exact when no element left out of the candidates can reach the top k: fewer than k
    // candidates only without any threshold, and every top-k candidate strictly above the
    // largest y an element below the thresholds can have (a seed above the k-th value, or a
    // tie created by the division by T, sends the row to the general path).  NaN keys (0) are
    // candidates only when no threshold was used.
    const uint32_t rk = mine ? sm.crank[tid] : 0xFFFFFFFFu;
    const bool topk = rk < (uint32_t)k;
    if (topk && myk != 0u && !(val_of(myk) > ylim)) atomicOr(&sm.status, 4u);

    // 6. survivors of temperature + top-k + min-p: exact masses, compacted into the survivor
    //    arrays (any order)
    const float m = mk ? val_of(mk) : __builtin_nanf("");
    if (!(m > -__builtin_inff() && m < __builtin_inff())) return false;  // degenerate row
    const float lp_min = (prm.min_p > 0.0f) ? log_det(prm.min_p < 1.0f ? prm.min_p : 1.0f)
                                            : -__builtin_inff();
    if (wave * kWave < total) {
        const float y = val_of(myk);
        const bool keep = topk && (y - m) >= lp_min;
        const uint64_t bal = wave_ballot(keep);
        uint32_t off = 0;
        if (lane == 0 && bal) off = atomicAdd(&sm.nkeep, (uint32_t)__popcll(bal));
        off = __builtin_amdgcn_readlane(off, 0);
        uint64_t mw = 0ull;
        if (keep) {
            const uint32_t pos = off + (uint32_t)lane_prefix(bal);
            if (pos < (uint32_t)kRowKeep) {
                const float e = exp_det(y - m);
                mw = mass_of(e);
                sm.sck[pos] = ((uint64_t)myk << 32) | (uint32_t)sm.pidx[tid];
                sm.sw[pos] = mw;
                sm.se[pos] = e;
                sm.spos[pos] = (uint32_t)tid;
            }
        }
        mw = wave_sum_u64(mw);
        if (lane == 0 && mw) atomicAdd(&sm.sW, mw);
    }
    if (u_slot >= 0) sm.pu[u_slot] = u_first;
    __syncthreads();
    if (sm.status != 0u) return false;  // a top-k candidate at or below the largest dropped y
    const int n = (int)sm.nkeep;
    if (n == 0 || n > kRowKeep) return false;

    // 7. top-p over exact masses: the cumulative mass of every survivor, then the race among
    //    the kept survivors, reduced across the wave and the waves
    const float q32 = 1.0f - prm.top_p;
    const bool topp = q32 > 0.0f;
    const bool abl = topp && !(q32 < 1.0f);  // top_p <= 0: only the last survivor is kept
    const int nws = (n + kWave - 1) / kWave;
    {
        // C_j = sum of w_i over the survivors i <= j in (y, index) order.  Waves split the sums
        // as (group of 64 survivors, range of survivors) pairs and add them into LDS.
        const int nsp = min(kRowWaves / nws, (n + 15) / 16);
        if (wave < nws * nsp) {
            const int g = wave % nws, sp = wave / nws;
            const int j = g * kWave + lane;
            const uint64_t ckj = j < n ? sm.sck[j] : 0ull;
            const int chunk = (n + nsp - 1) / nsp;
            const int i0 = sp * chunk, i1 = min(n, i0 + chunk);
            uint64_t part = 0ull;
#pragma unroll 4
            for (int i = i0; i < i1; ++i) part += sm.sck[i] <= ckj ? sm.sw[i] : 0ull;
            if (j < n && part) atomicAdd(&sm.sC[j], part);
        }
    }
    __syncthreads();
    if (wave >= nws) return true;
    const bool mys = tid < n;
    const uint64_t myck = mys ? sm.sck[tid] : ~0ull;
    const uint64_t C = mys ? sm.sC[tid] : 0ull;
    const uint64_t W = sm.sW;
    const uint64_t thr = (topp && !abl) ? scale_floor(q32, W) : 0ull;
    RowRace rs;
    if (mys) {
        const bool removed = topp && (abl ? (C != W) : (C <= thr && C != W));
        if (removed) {
            rs.cprev = C;
            rs.nrem = 1;
        } else {
            rs.cat = C;
            rs.nkept = 1;
            rs.last = myck;
            rs.add_key(sm.se[tid] / (0.0f - log_det(sm.pu[sm.spos[tid]])), (int)(uint32_t)myck);
        }
    }
    rs.shfl_merge(32); rs.shfl_merge(16); rs.shfl_merge(8);
    rs.shfl_merge(4); rs.shfl_merge(2); rs.shfl_merge(1);
    if (nws > 1) {
        if (lane == 0) {
            sm.red[wave][0] = rs.best; sm.red[wave][1] = rs.last; sm.red[wave][2] = rs.cprev;
            sm.red[wave][3] = rs.cat; sm.red[wave][4] = rs.second;
            sm.red[wave][5] = ((uint64_t)rs.nrem << 32) | rs.nkept;
        }
        // only the waves that hold survivors are still here (the others have left, so no
        // workgroup barrier): each of them counts itself in, and wave 0 waits for all of them.
        // Every one of these waves reaches the increment; the wait is bounded all the same.
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (lane == 0) {
            __hip_atomic_fetch_add(&sm.bc[4], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (wave == 0) {
                for (int spin = 0; spin < (1 << 22); ++spin) {
                    if (__hip_atomic_load(&sm.bc[4], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >=
                        (uint32_t)nws) break;
                    __builtin_amdgcn_s_sleep(1);
                }
            }
        }
        if (wave != 0) return true;
        wave_sync();
        if (lane == 0) {
            for (int w = 1; w < nws; ++w) {
                RowRace o;
                o.best = sm.red[w][0]; o.last = sm.red[w][1]; o.cprev = sm.red[w][2]; o.cat = sm.red[w][3];
                o.second = (uint32_t)sm.red[w][4]; o.nkept = (uint32_t)sm.red[w][5];
                o.nrem = (uint32_t)(sm.red[w][5] >> 32);
                rs.merge(o);
            }
        }
    } else if (wave != 0) {
        return true;
    }
    if (lane == 0) {
        int32_t tok;
        uint32_t fl = 0;
        if (rs.best) {
            tok = (int32_t)(0x7FFFFFFF - (uint32_t)(rs.best & 0xFFFFFFFFu));
            const float bk = u2f((uint32_t)(rs.best >> 32));
            if (rs.second) {
                const float sk = u2f(rs.second - 1u);
                if ((double)sk >= (double)bk * (1.0 - 1e-6)) fl |= VWS_FLAG_RACE_NEAR_TIE;
            }
        } else {
            tok = (int32_t)(uint32_t)(rs.last & 0xFFFFFFFFu);
        }
        if (topp && !abl) {
            const uint64_t tol = (uint64_t)((double)W * 1e-6);
            if ((rs.nrem > 0u && thr - rs.cprev <= tol) || (rs.cat > thr && rs.cat - thr <= tol))
                fl |= VWS_FLAG_TOPP_NEAR_TIE;
        }
        a.sampled[r] = tok;
        if (a.flags) a.flags[r] = fl;
        if (a.nkept) a.nkept[r] = (int32_t)rs.nkept;
        sm.lpk[0] = (uint32_t)tok; sm.lpk[1] = 0u; sm.lpk[2] = 0u; sm.lpk[3] = tmax;
    }
    return true;
}

// Raw logprobs of a row the single pass has sampled (launches that ask for them; every thread
// calls it after row_fast succeeded).  The packed candidates are every element of the row at
// or above its wave's final threshold, with their raw keys (sm.hpen) and indices (packed
// keys); every element left out lies below the largest threshold any wave used (tmax).  So the
// L largest raw logits (value desc, index asc) are the L largest candidates as long as at
// least L candidates lie at or above tmax, and the sampled token's rank (#{j : x_j >= x_s})
// is counted among the candidates as long as x_s >= tmax.  The log-normaliser is the stream's
// per-wave sums of exp(x - a_w), rescaled to the row maximum in double.  Returns 0 (nothing of
// the logprobs written; the row's token is written again by the multi-pass path) when a
// condition fails.
__device__ __noinline__ int row_logprobs_entry(int r, uint64_t kernarg) {
#if defined(__HIP_DEVICE_COMPILE__)
    const KArgs a = kargs_at(kernarg);
    r = __builtin_amdgcn_readfirstlane(r);
    RowSmem& sm = g_row_sh.f;
    const int tid = threadIdx.x, lane = tid & 63;
    __syncthreads();  // the tail's hand-off (sm.lpk[0..3])
    const int total = (int)sm.npack;
    const bool small = sm.lpk[1] != 0u, greedy = sm.lpk[2] != 0u;
    const uint32_t tok = sm.lpk[0], tmax = sm.lpk[3];
    const uint32_t* rawk = reinterpret_cast<const uint32_t*>(sm.hpen);
    const bool mine = tid < total;
    const uint32_t rk = mine ? rawk[tid] : 0u;
    uint32_t ix = 0u;
    if (mine) {
        const uint32_t lo = small ? (uint32_t)sm.pk64[tid] : (uint32_t)sm.pidx[tid];
        ix = (small && greedy) ? 0x7FFFFFFFu - lo : lo;
    }
    if (mine && ix == tok) sm.lpk[4] = rk;
    const uint32_t nge = (uint32_t)__popcll(wave_ballot(mine && rk >= tmax));
    const uint32_t mxk = wave_max_u32(rk);
    if (lane == 0) {
        if (nge) atomicAdd(&sm.lpk[5], nge);
        atomicMax(&sm.lpk[6], mxk);
    }
    __syncthreads();
    const uint32_t ks = sm.lpk[4], ngeq = sm.lpk[5], km = sm.lpk[6];
    const int L = a.L;
    if (!(ks != 0u && ks >= tmax && (int)ngeq >= L && km > 0x007FFFFFu && km < 0xFF800000u)) return 0;
    // the rank, and each candidate's position in (raw desc, index asc) order, counted over a
    // 64-bit copy of the candidates in the (now free) candidate buffers
    const uint32_t nrk = (uint32_t)__popcll(wave_ballot(mine && rk >= ks));
    if (lane == 0 && nrk) atomicAdd(&sm.lpk[7], nrk);
    uint64_t* keys = reinterpret_cast<uint64_t*>(&sm.ckey[0][0]);
    const uint64_t me = ((uint64_t)rk << 32) | (0x7FFFFFFFu - ix);
    if (mine) keys[tid] = me;
    const float A = val_of(km);  // the row maximum: the largest candidate
    if (tid < kWave) {
        // the waves' sums rescaled to the row maximum, one lane per wave (double exp2 and log
        // in parallel rather than one after another in one thread), summed by a butterfly
        double t = 0.0;
        if (lane < kRowWaves && sm.lpS[lane] > 0.0)
            t = sm.lpS[lane] * exp2((double)sm.lpA[lane] - (double)A * (double)kLog2e);
#pragma unroll
        for (int o = 1; o < kRowWaves; o <<= 1)
            t += __builtin_bit_cast(double, lane_xor64(__builtin_bit_cast(uint64_t, t), o));
        if (lane == 0) sm.lplog = (float)log(t);
    }
    __syncthreads();
    uint32_t pos = 0u;
    if (mine && rk >= tmax) {
        // (eight independent LDS reads in flight per step)
#pragma unroll 8
        for (int j = 0; j < total; ++j) pos += keys[j] > me ? 1u : 0u;
    }
    const float logS = sm.lplog;
    const int stride = L + 1;
    if (tid == 0) {
        a.lp_ids[(size_t)r * stride] = (int32_t)tok;
        a.lp_vals[(size_t)r * stride] = (val_of(ks) - A) - logS;
        a.lp_ranks[r] = (int32_t)sm.lpk[7];
    }
    if (mine && rk >= tmax && pos < (uint32_t)L) {
        a.lp_ids[(size_t)r * stride + 1 + pos] = (int32_t)ix;
        a.lp_vals[(size_t)r * stride + 1 + pos] = (val_of(rk) - A) - logS;
    }
    return 1;
#else
    (void)r;
    (void)kernarg;
    return 0;
#endif
}

// The general path runs in a function of its own so that its register allocation (it needs
// more than the 128 VGPRs a 1024-thread workgroup allows and spills) stays out of the
// single-pass loop.  The kernel hands it the address of its kernarg segment (a callee has no
// register of its own for it); the launch arguments are read from there into scalar registers.
template <typename T>
__device__ __noinline__ void row_general(int r, uint64_t kernarg) {
#if defined(__HIP_DEVICE_COMPILE__)
    const KArgs a = kargs_at(kernarg);
    const RowP prm = row_params(a, r);
    general_row<T>(a, g_row_sh.g, r, prm);
#else
    (void)r;
    (void)kernarg;
#endif
}

// One row: the single pass, the single-pass top-p path or the multi-pass path.  Returns whether
// The single-pass top-p path of a row in a launch with an allowed mask or the soft cap (stream
// and finish, XF); returns 0 or the reason the row takes the multi-pass path.
template <typename T, int XF>
__device__ __noinline__ int topp_row_xf_entry(int r, uint64_t kernarg) {
#if defined(__HIP_DEVICE_COMPILE__)
    const KArgs a = kargs_at(kernarg);
    r = __builtin_amdgcn_readfirstlane(r);
    const RowP prm = row_params(a, r);
    if (prm.has_hist) {
        const float fill = tp_uf(topp_hist_begin(a, g_row_sh.t, prm));
        topp_stream<T, XF>(a, g_row_sh.t, r, prm, fill);
    } else {
        topp_stream<T, XF>(a, g_row_sh.t, r, prm, kTpFill * (float)kTpCapW);
    }
    return topp_finish<T, XF>(a, g_row_sh.t, r, prm, kernarg);
#else
    (void)r;
    (void)kernarg;
    return 0;
#endif
}

// the row took one of the longer paths (top-p or multi-pass), whose workgroup then looks for
// chunks of other rows' passes.
template <typename T, bool LP, int XF>
__device__ __forceinline__ bool row_one(const KArgs& a, int r, const void* logits, int64_t lstride,
                                        int V, uint64_t kernarg) {
    bool topp = false;
    if (a.nofast) {
        topp = topp_eligible(a, row_params(a, r));
    } else if (row_fast<T, LP, XF == kXfMask>(a, g_row_sh.f, r, logits, lstride, V, &topp)) {
        if (!LP || row_logprobs_entry(r, kernarg)) return false;
    }
    int why = 0;
    if (topp) {
        // the single-pass top-p path, inline: it starts after the single-pass function has
        // returned (no live range crosses that function's stream) and issues its own loads
        __syncthreads();
        // a top-p row in progress may open a cooperative pass
        if (threadIdx.x == 0 && a.coop) ag_add64(&a.coop->wgs, kCoopPending);
        if (XF != kXfNone) {
            // launches with an allowed mask or the soft cap: out of line, so that the kernel's
            // single pass keeps the registers it has without these top-p paths
            why = topp_row_xf_entry<T, XF>(r, kernarg);
        } else {
            const RowP prm = row_params(a, r);
            if (prm.has_hist) {
                // history rows: their bitmap into LDS first (a copy of the stream of its own)
                const float fill = tp_uf(topp_hist_begin(a, g_row_sh.t, prm));
                topp_stream<T, kXfNone>(a, g_row_sh.t, r, prm, fill);
            } else {
                topp_stream<T, kXfNone>(a, g_row_sh.t, r, prm, kTpFill * (float)kTpCapW);
            }
            why = topp_finish<T, kXfNone>(a, g_row_sh.t, r, prm, kernarg);
        }
        // done with it: no longer pending, and no longer holding slots (thread 0 set the mark)
        if (threadIdx.x == 0 && a.coop)
            ag_add64(&a.coop->wgs, 0ull - kCoopPending - (g_row_sh.t.coop_hold ? kCoopActive : 0ull));
        if (why == 0) return true;
    }
    __syncthreads();
    row_general<T>(r, kernarg);
    // diagnostic: why the single-pass top-p path handed the row over (thread 0 wrote the flags)
    if (why && threadIdx.x == 0 && a.flags) a.flags[r] |= (uint32_t)why << 16;
    return true;
}

// After the workgroup's row: look for chunks of the passes other rows opened.  Every row has a
// workgroup: those of the longer paths poll while top-p rows are in progress (the device runs
// nothing else of the launch meanwhile).  More rows than the device holds at once: every
// workgroup counts itself finished; once every workgroup has started it polls while top-p rows
// are in progress, before that it only runs chunks already open (so that it keeps no row from
// starting).  Out of line: nothing but the kernarg address stays live across the row.
template <typename T, int XF>
__device__ __noinline__ void row_kernel_rest(uint64_t kernarg, int long_row) {
#if defined(__HIP_DEVICE_COMPILE__)
    const KArgs a = kargs_at(kernarg);
    long_row = __builtin_amdgcn_readfirstlane(long_row);
    if (!a.coop) return;
    // chunks of other rows' passes, run as the launch loads its logits (mask, soft cap or as
    // they are) and with penalties from the token-state table where the launch has them
    auto help = [&](int spin) __attribute__((always_inline)) {
        if (a.tbits) coop_help_entry<T, true, XF>(kernarg, spin);
        else coop_help_entry<T, false, XF>(kernarg, spin);
    };
    if (!a.coop_count) {
        if (long_row) {
            __syncthreads();
            help(1);
        }
        return;
    }
    TopPSmem& sm = g_row_sh.t;
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint64_t x = ag_add64(&a.coop->wgs, kCoopFinished);
        const bool all_started = coop_started(x) == gridDim.x;
        // the last workgroup to finish: every one has started and finished, no row is pending
        if (coop_finished(x) + 1u == gridDim.x) ag_store64(&a.coop->wgs, 0ull);
        sm.cp[6] = (all_started && coop_pending(x) != 0u) ? 2u : (coop_active(x) != 0u ? 1u : 0u);
    }
    __syncthreads();
    const uint32_t how = tp_u(sm.cp[6]);
    if (how) {
        __syncthreads();
        help(how == 2u ? 1 : 0);
    }
#else
    (void)kernarg;
    (void)long_row;
#endif
}

// The row workgroup b serves when the launch counts its workgroups (more rows than the device
// holds at once): the sampled rows whose survivors top-p alone cuts (top-k off, 0 < top_p < 1:
// the longer paths) first, then the others, each group in index order, so that long rows do
// not start last.  Every thread calls it; two passes over the rows' top-k, top-p and
// temperature.
__device__ __noinline__ int row_order_entry(uint64_t kernarg, int b) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int NT = kGenThreads;
    const KArgs a = kargs_at(kernarg);
    b = __builtin_amdgcn_readfirstlane(b);
    TopPSmem& sm = g_row_sh.t;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int B = a.B;
    auto is_long = [&](int i) __attribute__((always_inline)) {
        const int k = a.top_k ? a.top_k[i] : 0;
        const float p = a.top_p ? a.top_p[i] : 1.0f;
        const float t = a.temperature ? a.temperature[i] : 0.0f;
        return !is_greedy(t) && (k <= 0 || k >= a.V) && p > 0.0f && p < 1.0f;
    };
    // pass 1: the number of long rows
    uint32_t nl = 0u;
    for (int base = 0; base < B; base += NT) {
        const int i = base + tid;
        nl += (uint32_t)__popcll(wave_ballot(i < B && is_long(i)));
    }
    if (lane == 0) sm.cp[8 + wave] = nl;
    if (tid == 0) sm.cp[0] = (uint32_t)b;  // fallback: the identity
    __syncthreads();
    uint32_t F = 0u;
#pragma unroll
    for (int w = 0; w < kGenWaves; ++w) F += sm.cp[8 + w];
    F = tp_u(F);
    __syncthreads();
    // pass 2: the b-th row of the order (ranks among the long rows, or among the others)
    uint32_t before = 0u;  // long rows before this chunk
    for (int base = 0; base < B; base += NT) {
        const int i = base + tid;
        const bool l = i < B && is_long(i);
        const uint64_t bal = wave_ballot(l);
        if (lane == 0) sm.cp[8 + wave] = (uint32_t)__popcll(bal);
        __syncthreads();
        uint32_t below = before;  // long rows before this thread's row
        for (int w = 0; w < wave; ++w) below += sm.cp[8 + w];
        below += (uint32_t)lane_prefix(bal);
        if (i < B) {
            if (l && below == (uint32_t)b) sm.cp[0] = (uint32_t)i;
            if (!l && (uint32_t)i - below == (uint32_t)b - F && (uint32_t)b >= F) sm.cp[0] = (uint32_t)i;
        }
        uint32_t chunk = 0u;
#pragma unroll
        for (int w = 0; w < kGenWaves; ++w) chunk += sm.cp[8 + w];
        before += chunk;
        __syncthreads();
    }
    return (int)tp_u(sm.cp[0]);
#else
    (void)kernarg;
    return b;
#endif
}

// One workgroup per row (the grid is exactly B workgroups).  `coop` (preloaded with the row's
// address, stride and V, so that testing it costs no argument read): bit 0, the cooperative
// region is present; bit 1, the workgroups are counted (KArgs::coop_count); bit 2, the rows are
// served longest first (row_order_entry: every workgroup scans the batch's parameters, so the
// launcher asks for it only up to kRowOrderMaxBatch rows).
template <typename T, bool LP, int XF>
__global__ __launch_bounds__(kRowThreads) void row_kernel(const void* logits, int64_t lstride, int V,
                                                          int coop, KArgs a) {
#ifdef VWS_TRACE
    // stored once the row is done: a store this early turns the row parameters' scalar loads
    // into vector ones
    uint64_t tr_entry = 0;
    if (__builtin_amdgcn_readfirstlane(threadIdx.x) == blockDim.x - 64u) tr_entry = trace_clock();
#endif
    const uint64_t kernarg = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr() + 24u;
    int r = blockIdx.x;
    if (coop & 2) {
        if (threadIdx.x == 0) ag_add64(&a.coop->wgs, kCoopStarted);
        if (coop & 4) r = __builtin_amdgcn_readfirstlane(row_order_entry(kernarg, r));
    }
    const bool long_row = row_one<T, LP, XF>(a, r, logits, lstride, V, kernarg);
    VWS_TRACE_MARK(a, VWS_TRACE_ROW);
#ifdef VWS_TRACE
    trace_put(a, VWS_TRACE_ENTRY, tr_entry);
    trace_put(a, VWS_TRACE_XCC, trace_xcc());
    trace_put(a, VWS_TRACE_ROWID, (uint64_t)r);
#endif
    if ((coop & 2) || ((coop & 1) && long_row)) row_kernel_rest<T, XF>(kernarg, long_row ? 1 : 0);
    VWS_TRACE_MARK(a, VWS_TRACE_EXIT);
}

}  // namespace vws
