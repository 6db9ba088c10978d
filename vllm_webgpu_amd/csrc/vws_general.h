// vws_general.h -- multi-pass sampler for the rows the single-pass kernel does not
// finish: top-k off (top-p / min-p over the full vocabulary), k > 256, rows handed over after
// a candidate overflow, degenerate rows, and every row when logprobs are requested.
//
// One workgroup of 1024 threads owns one row and streams it from HBM several times (the row
// stays hot in L2/MALL between passes):
//   A  max of the penalised logits (+ lowest/highest index at the max), raw max and top-L raw
//      candidates for logprobs, level-1 radix histogram when top-k must be found exactly;
//   K  (top-k only) two more radix levels -> exact k-th largest value;
//   B  integer masses w = floor(exp_det(y - m) * 2^44) of the survivors of top-k and min-p,
//      summed into 4096 buckets of d = m - y (width 1/128) -> total W and the bucket b* that
//      holds the top-p boundary;
//   C  exponential race over every survivor strictly above b*, b*'s members gathered to LDS,
//      sorted by (y, index), prefix-summed and cut exactly, then raced;
//   R  (only when b* holds more than 2048 members) key-range refinement passes and, for a
//      single huge tie group, an index radix select, so the cut stays exact;
//   D  (logprobs) log-sum-exp of the raw logits and the rank of the sampled token.
// Penalised values come from a per-row hash of the history in the workspace, found through a
// per-row LDS bitmap of history positions, so the logits are never written.
#pragma once

#include "vws_cand.h"
#include "vws_internal.h"
#include "vws_row.h"

namespace vws {

constexpr int kBitmapWords = VWS_MAX_VOCAB / 32 + 2;

struct GenSmem {
    uint32_t bitmap[kBitmapWords];
    union {
        uint64_t hmass[kBuckets];
        uint32_t whist[kGenWaves][256];  // pass A: per-wave radix-select scratch
    };
    uint32_t hcnt[kBuckets];
    union {
        struct {
            uint32_t key[kGenWaves][kLpCapW];
            int32_t idx[kGenWaves][kLpCapW];
        } lp;
        uint64_t gather[kGatherCap];
    } u;
    uint64_t red[kGenWaves];
    uint32_t lp_sel_key[128];
    int32_t lp_sel_idx[128];
    int lp_cnt[kGenWaves];
    uint32_t lp_tau;
    uint32_t gcount;
    uint32_t nsel;
    uint32_t bc32[8];
    uint64_t bc64[8];
};

// ---- workspace hash of the history (open addressing, token + 1 as key) -----------------

__device__ __forceinline__ uint32_t ghash_slot(int t, int hs) {
    return ((uint32_t)t * 2654435761u) & (uint32_t)(hs - 1);
}

// inc: 1 counts an output occurrence; otherwise kHPrompt, kHBan or kHBias (with its bias) is set
__device__ __forceinline__ void ghash_insert(uint32_t* hkey, uint32_t* hval, uint32_t* hadj, int hs,
                                             int t, uint32_t inc, float bias = 0.0f) {
    uint32_t s = ghash_slot(t, hs);
    for (int probe = 0; probe < hs; ++probe) {
        const uint32_t prev = atomicCAS(&hkey[s], 0u, (uint32_t)t + 1u);
        if (prev == 0u || prev == (uint32_t)t + 1u) {
            if (inc == 1u) {
                atomicAdd(&hval[s], 1u);
            } else {
                if (inc & kHBias) __hip_atomic_store(&hadj[s], f2u(bias), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                atomicOr(&hval[s], inc);
            }
            return;
        }
        s = (s + 1u) & (uint32_t)(hs - 1);
    }
}

// The processed value of hashed token t into *out; false when t is not in the hash.
__device__ __forceinline__ bool ghash_pen(const uint32_t* hkey, const uint32_t* hpen, int hs, int t, float* out) {
    uint32_t s = ghash_slot(t, hs);
    for (int probe = 0; probe < hs; ++probe) {
        const uint32_t k = __hip_atomic_load(&hkey[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (k == (uint32_t)t + 1u) {
            *out = u2f(__hip_atomic_load(&hpen[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            return true;
        }
        if (k == 0u) break;
        s = (s + 1u) & (uint32_t)(hs - 1);
    }
    return false;
}

// ---- block helpers for 1024 threads ---------------------------------------------------------

__device__ __forceinline__ uint64_t gblock_sum(uint64_t v, GenSmem& sm) {
    v = wave_sum_u64(v);
    __syncthreads();
    if (lane_id() == 0) sm.red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < kGenWaves; ++i) t += sm.red[i];
    return t;
}

__device__ __forceinline__ uint64_t gblock_max(uint64_t v, GenSmem& sm) {
    v = wave_max_u64(v);
    __syncthreads();
    if (lane_id() == 0) sm.red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int i = 0; i < kGenWaves; ++i) t = t > sm.red[i] ? t : sm.red[i];
    return t;
}

__device__ __forceinline__ uint64_t gblock_min(uint64_t v, GenSmem& sm) {
    v = wave_min_u64(v);
    __syncthreads();
    if (lane_id() == 0) sm.red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = ~0ull;
#pragma unroll
    for (int i = 0; i < kGenWaves; ++i) t = t < sm.red[i] ? t : sm.red[i];
    return t;
}

__device__ __forceinline__ double gblock_sum_f64(double v, GenSmem& sm) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    __syncthreads();
    if (lane_id() == 0) sm.red[threadIdx.x >> 6] = (uint64_t)__double_as_longlong(v);
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < kGenWaves; ++i) t += __longlong_as_double((long long)sm.red[i]);
    return t;
}

// Exclusive prefix over threads in descending thread order: sum of v over threads > tid.
__device__ __forceinline__ uint64_t gblock_suffix_excl(uint64_t v, GenSmem& sm) {
    const int lane = lane_id(), w = threadIdx.x >> 6;
    // inclusive suffix within the wave
    uint64_t s = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint64_t t = __shfl_down(s, o, kWave);
        if (lane + o < kWave) s += t;
    }
    __syncthreads();
    if (lane == 0) sm.red[w] = s;  // wave total
    __syncthreads();
    uint64_t above = 0;
    for (int i = w + 1; i < kGenWaves; ++i) above += sm.red[i];
    return above + (s - v);
}

// Scans bins from index nb-1 down to 0 and returns the first bin b whose inclusive cumulative
// count (sum over bins >= b) reaches `target`; *above gets the sum over bins > b.  Requires the
// total to reach target.  4 bins per thread (nb = 4096) or 1 (nb <= 1024).
template <typename C>
__device__ __forceinline__ int gfind_from_top(const C* bins, int nb, uint64_t target, uint64_t* above, GenSmem& sm) {
    const int per = nb / kGenThreads > 0 ? nb / kGenThreads : 1;
    const int t = threadIdx.x;
    uint64_t loc[4] = {0, 0, 0, 0};
    uint64_t tot = 0;
    if (t * per < nb) {
        for (int i = 0; i < per; ++i) { loc[i] = (uint64_t)bins[t * per + i]; tot += loc[i]; }
    }
    const uint64_t ab = gblock_suffix_excl(tot, sm);  // bins above this thread's range
    if (threadIdx.x == 0) { sm.bc32[0] = 0xFFFFFFFFu; sm.bc64[0] = 0ull; }
    __syncthreads();
    if (t * per < nb) {
        uint64_t run = ab;
        for (int i = per - 1; i >= 0; --i) {
            const uint64_t before = run;
            run += loc[i];
            if (before < target && run >= target) {
                sm.bc32[0] = (uint32_t)(t * per + i);
                sm.bc64[0] = before;
            }
        }
    }
    __syncthreads();
    *above = sm.bc64[0];
    const uint32_t b = sm.bc32[0];
    return b < (uint32_t)nb ? (int)b : 0;  // not found only if the caller's invariant is broken
}

// ---- the row ------------------------------------------------------------------------------

template <typename T>
__device__ __forceinline__ uint32_t general_topk_select(const KArgs& a, GenSmem& sm, int r, int k);

struct RaceAcc {
    uint64_t best = 0;     // (key bits << 32) | (0x7FFFFFFF - index), 0 = none
    uint32_t second = 0;   // key bits + 1 of the best non-winning key, 0 = none
    uint64_t last = 0;     // max (key(y) << 32 | index) over kept tokens
    uint32_t nkept = 0;
    __device__ __forceinline__ void add(float e, uint32_t ky, int idx, float uu) {
        nkept++;
        const uint64_t lk = ((uint64_t)ky << 32) | (uint32_t)idx;
        last = last > lk ? last : lk;
        const float key = e / (0.0f - log_det(uu));
        if (!(key >= 0.0f)) return;
        const uint64_t pk = ((uint64_t)f2u(key) << 32) | (uint32_t)(0x7FFFFFFF - idx);
        if (pk > best) {
            if (best) { const uint32_t o = (uint32_t)(best >> 32) + 1u; second = second > o ? second : o; }
            best = pk;
        } else {
            const uint32_t o = f2u(key) + 1u;
            second = second > o ? second : o;
        }
    }
};

template <typename T>
__device__ __forceinline__ void general_row(const KArgs& a, GenSmem& sm, int r, const RowP& prm) {
    constexpr int NT = kGenThreads;
    constexpr int VEC = Elem<T>::kVec;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int V = a.V;
    const T* row = reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride;
    const float* urow = a.u ? a.u + (size_t)r * a.ustride : nullptr;
    Slice<T> sl;
    sl.init(row, 0, V);
    const int nch = sl.nchunks();
    const int nit = (nch + 2 * NT - 1) / (2 * NT);
    const bool hh = prm.need_hash;
    // penalties from the token-state table: the tokens with a non-zero word are marked in the
    // bitmap (one scan of the row's words) and penalised from their word where they are read
    const bool tb = prm.tab;
    const uint32_t* tabrow = tb ? a.tstate + (size_t)prm.trow * (size_t)a.tstride : nullptr;
    const int hs = a.hs_row;
    uint32_t* hkey = a.hist_hash + (size_t)r * (size_t)hs * 4;
    uint32_t* hval = hkey + hs;
    uint32_t* hpen = hval + hs;
    uint32_t* hadj = hpen + hs;
    const uint32_t* mrow = a.allowed ? a.allowed + (size_t)r * a.astride : nullptr;
    const int nmw = (V + 31) / 32;
    const int L = a.L;

    // ---- history: hash in the workspace + bitmap of positions in LDS
    if (hh || tb) {
        const int nw = (V + 31) / 32 + 2;
        for (int i = tid; i < nw; i += NT) sm.bitmap[i] = 0u;
        if (hh)
            for (int i = tid; i < hs; i += NT) { hkey[i] = 0u; hval[i] = 0u; hpen[i] = 0u; }
        __threadfence();
        __syncthreads();
        if (tb) {
            // each wave marks 64 consecutive tokens per step (two bitmap words)
            for (int i0 = wave * kWave; i0 < V; i0 += NT) {
                const int i = i0 + lane;
                const uint64_t nz = wave_ballot(i < V && (tabrow[i] & kStateMask) != 0u);
                if (lane == 0 && nz) {
                    atomicOr(&sm.bitmap[i0 >> 5], (uint32_t)nz);
                    atomicOr(&sm.bitmap[(i0 >> 5) + 1], (uint32_t)(nz >> 32));
                }
            }
        }
        if (prm.has_hist && prm.np > 0) {
            const int32_t* pr = a.prompt + (size_t)r * a.pstride;
            for (int i = tid; i < prm.np; i += NT) {
                const int t = pr[i];
                if (t >= 0 && t < V) {
                    ghash_insert(hkey, hval, hadj, hs, t, kHPrompt);
                    atomicOr(&sm.bitmap[t >> 5], 1u << (t & 31));
                }
            }
        }
        if (prm.has_hist && prm.no > 0) {
            const int32_t* ou = a.output + (size_t)r * a.ostride;
            for (int i = tid; i < prm.no; i += NT) {
                const int t = ou[i];
                if (t >= 0 && t < V) {
                    ghash_insert(hkey, hval, hadj, hs, t, 1u);
                    atomicOr(&sm.bitmap[t >> 5], 1u << (t & 31));
                }
            }
        }
        if (prm.na > 0) {
            const int32_t* ai = a.adj_ids + (size_t)r * a.adjstride;
            const float* av = a.adj_vals + (size_t)r * a.adjstride;
            for (int i = tid; i < prm.na; i += NT) {
                const int t = ai[i];
                if (t >= 0 && t < V) {
                    const float bv = av[i];
                    ghash_insert(hkey, hval, hadj, hs, t, bv == -__builtin_inff() ? kHBan : kHBias, bv);
                    atomicOr(&sm.bitmap[t >> 5], 1u << (t & 31));
                }
            }
        }
        __threadfence();
        __syncthreads();
        for (int s = tid; s < hs; s += NT) {
            const uint32_t kk = __hip_atomic_load(&hkey[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (kk) {
                uint32_t v = __hip_atomic_load(&hval[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (tb) v |= tabrow[kk - 1u] & kStateMask;
                float raw = Elem<T>::load1(row + (kk - 1u));
                if (a.softcap > 0.0f) raw = softcap_out(raw, a.inv_softcap, a.softcap, a.softcap_f16 != 0);
                const float bias = u2f(__hip_atomic_load(&hadj[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                const float pen = apply_hashed(raw, v, bias, prm.rep, prm.inv_rep, prm.freq, prm.pres);
                __hip_atomic_store(&hpen[s], f2u(pen), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __threadfence();
        __syncthreads();
    }
    // Elements of the chunk being visited that belong to the row: the first cur_nv (a body
    // vector all VEC; the unaligned head and tail fewer, their other slots NaN padding whose
    // indices are other elements'; chunks past the tail none).  Only those are processed, so
    // padding never turns into a masked or penalised copy of another element.
    int cur_nv = VEC;
    auto chunk_nv = [&](int c) -> int {
        if (c >= 1 && c <= sl.nbody) return VEC;
        if (c == 0) return sl.a - sl.lo;
        if (c == sl.nbody + 1) return sl.hi - sl.body_end();
        return 0;
    };
    // processed values of a chunk: hashed tokens (processors, then penalties), then the
    // allowed-token mask (masked tokens are -inf whatever the hash did to them)
    auto finalize = [&](float* v, int i0) {
        if (hh || tb) {
            const uint32_t w = (uint32_t)i0 >> 5, sh = (uint32_t)i0 & 31u;
            const uint64_t win = (uint64_t)sm.bitmap[w] | ((uint64_t)sm.bitmap[w + 1] << 32);
            const uint32_t bits = (uint32_t)(win >> sh) & ((1u << cur_nv) - 1u);
            if (bits) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    if (!((bits >> j) & 1u)) continue;
                    // processor tokens are hashed (their word folded in); others are table tokens
                    if (hh && ghash_pen(hkey, hpen, hs, i0 + j, &v[j])) continue;
                    if (tb)
                        v[j] = apply_hashed(v[j], tabrow[i0 + j] & kStateMask, 0.0f, prm.rep,
                                            prm.inv_rep, prm.freq, prm.pres);
                }
            }
        }
        if (mrow) {
            const int w = i0 >> 5, sh = i0 & 31;
            const uint64_t win = (uint64_t)mrow[w < nmw ? w : nmw - 1] |
                                 ((uint64_t)(w + 1 < nmw ? mrow[w + 1] : 0u) << 32);
            const uint32_t bits = (uint32_t)(win >> sh);
#pragma unroll
            for (int j = 0; j < VEC; ++j)
                if (!((bits >> j) & 1u) && j < cur_nv) v[j] = -__builtin_inff();
        }
    };
    // every pass visits the same chunks in the same order: 2 chunks per thread per iteration
    auto for_rows = [&](auto&& f) {
        for (int it = 0; it < nit; ++it) {
            float v0[VEC], v1[VEC];
            const int c0 = it * 2 * NT + tid;
            const int i0 = sl.load(c0, v0);
            const int i1 = sl.load(c0 + NT, v1);
            if (a.softcap > 0.0f) {  // the model's output is the capped logit
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    v0[j] = softcap_out(v0[j], a.inv_softcap, a.softcap, a.softcap_f16 != 0);
                    v1[j] = softcap_out(v1[j], a.inv_softcap, a.softcap, a.softcap_f16 != 0);
                }
            }
            cur_nv = chunk_nv(c0);
            f(v0, i0);
            cur_nv = chunk_nv(c0 + NT);
            f(v1, i1);
        }
    };
    // the same visit for the race passes, with the chunks' uniforms loaded together with their
    // logits (a race pass otherwise waits for one uniform load per racing survivor)
    auto for_rows_u = [&](auto&& f) {
        for (int it = 0; it < nit; ++it) {
            float v0[VEC], v1[VEC], u0[VEC], u1[VEC];
            const int c0 = it * 2 * NT + tid;
            const int i0 = sl.load(c0, v0);
            const int i1 = sl.load(c0 + NT, v1);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                u0[j] = (urow && i0 + j < V) ? urow[i0 + j] : 0.5f;
                u1[j] = (urow && i1 + j < V) ? urow[i1 + j] : 0.5f;
            }
            if (a.softcap > 0.0f) {  // the model's output is the capped logit
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    v0[j] = softcap_out(v0[j], a.inv_softcap, a.softcap, a.softcap_f16 != 0);
                    v1[j] = softcap_out(v1[j], a.inv_softcap, a.softcap, a.softcap_f16 != 0);
                }
            }
            cur_nv = chunk_nv(c0);
            f(v0, i0, u0);
            cur_nv = chunk_nv(c0 + NT);
            f(v1, i1, u1);
        }
    };

    const bool sampling = !prm.greedy;
    const int k = prm.k;
    const bool topk_try = sampling && k > 0 && k < V;
    const float Tt = prm.T;

    // ---- pass A
    uint32_t mk = 0, m0k = 0, nvalid = 0;
    int mi = 0x7FFFFFFF, mxi = -1;
    if (tid == 0) { sm.lp_tau = 0u; sm.bc64[4] = 0ull; }
    if (topk_try) for (int i = tid; i < kBuckets; i += NT) sm.hcnt[i] = 0u;
    __syncthreads();
    CandBuf lpb;
    uint32_t* whist = sm.whist[wave];
    lpb.init(sm.u.lp.key[wave], sm.u.lp.idx[wave], whist, &sm.lp_tau, kLpCapW, L > 0 ? L : 1);
    for_rows([&](float* v, int i0) {
        if (L > 0) {
            lpb.refresh();
#pragma unroll
            for (int j = 0; j < VEC; ++j) lpb.append(v[j] >= lpb.tauf, key_of(v[j]), i0 + j);
        }
        if (L >= 0) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) { const uint32_t kk = key_of(v[j]); m0k = m0k > kk ? m0k : kk; }
        }
        finalize(v, i0);
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const uint32_t kk = key_of(v[j]);
            if (kk) {
                nvalid++;
                if (topk_try) agg_count(sm.hcnt, kk >> 20);
            }
            if (kk > mk) { mk = kk; mi = i0 + j; mxi = i0 + j; }
            else if (kk == mk && kk != 0u) { mi = min(mi, i0 + j); mxi = max(mxi, i0 + j); }
        }
    });
    if (L > 0 && !lpb.ovf) lpb.compact();
    if (L > 0 && lane == 0) sm.lp_cnt[wave] = lpb.ovf ? -1 : lpb.cnt;
    const uint64_t top_lo = gblock_max(((uint64_t)mk << 32) | (uint32_t)(0x7FFFFFFF - (mk ? mi : 0)), sm);
    const uint64_t top_hi = gblock_max(((uint64_t)mk << 32) | (uint32_t)(mk ? mxi + 1 : 0), sm);
    const uint32_t maxkey = (uint32_t)(top_lo >> 32);
    const int argmax_lo = (int)(0x7FFFFFFF - (uint32_t)(top_lo & 0xFFFFFFFFu));
    const int argmax_hi = (int)(uint32_t)(top_hi & 0xFFFFFFFFu) - 1;
    const uint32_t nval = (uint32_t)gblock_sum(nvalid, sm);
    const uint32_t m0key = (uint32_t)gblock_max(m0k, sm);

    // top-L raw candidates -> lp_sel (value desc, index asc), before LDS is reused
    if (L > 0) {
        __syncthreads();
        if (wave == 0) {
            int cnts[kGenWaves];
            int total = 0;
            bool bad = false;
            for (int w = 0; w < kGenWaves; ++w) { cnts[w] = sm.lp_cnt[w]; bad |= cnts[w] < 0; total += cnts[w] < 0 ? 0 : cnts[w]; }
            uint32_t kth = 0;
            if (!bad && total >= L) kth = wave_kth_largest_multi(&sm.u.lp.key[0][0], kLpCapW, cnts, kGenWaves, L, whist);
            if (lane == 0) { sm.bc32[1] = kth; sm.nsel = 0; sm.bc32[2] = bad ? 1u : 0u; }
        }
        __syncthreads();
        const uint32_t kth = sm.bc32[1];
        if (sm.bc32[2] == 0u) {
            const int n = sm.lp_cnt[wave];
            for (int i = lane; i < n; i += 64) {
                const uint32_t kk = sm.u.lp.key[wave][i];
                if (kk >= kth && kk != 0u) {
                    const uint32_t pos = agg_reserve(&sm.nsel);
                    if (pos < 128u) { sm.lp_sel_key[pos] = kk; sm.lp_sel_idx[pos] = sm.u.lp.idx[wave][i]; }
                }
            }
        }
        __syncthreads();
    }

    int32_t token = 0;
    uint32_t flags = VWS_FLAG_GENERAL_PATH;
    int32_t nkept_out = 1;

    if (prm.greedy) {
        token = maxkey ? argmax_lo : 0;
        flags |= VWS_FLAG_GREEDY;
        goto logprobs;
    }
    {
        const float m = maxkey ? val_of(maxkey) / Tt : __builtin_nanf("");
        if (!(m > -__builtin_inff() && m < __builtin_inff())) {
            // degenerate: first index of the largest key(x / Tt)
            const uint32_t km = key_of(m);
            int first = 0x7FFFFFFF;
            for_rows([&](float* v, int i0) {
                finalize(v, i0);
#pragma unroll
                for (int j = 0; j < VEC; ++j)
                    if (i0 + j < V && key_of(v[j] / Tt) == km) first = min(first, i0 + j);
            });
            const uint64_t f = gblock_max((uint64_t)(0x7FFFFFFF - first), sm);
            token = (int32_t)(0x7FFFFFFF - (uint32_t)f);
            if (token >= V) token = 0;
            flags |= VWS_FLAG_DEGENERATE;
            goto logprobs;
        }

        // ---- exact k-th largest penalised value (top-k), 3 radix levels over 32-bit keys
        float kth_y = -__builtin_inff();
        if (topk_try && (uint32_t)k <= nval) {
            uint64_t ab;
            const int b1 = gfind_from_top(sm.hcnt, kBuckets, (uint64_t)k, &ab, sm);
            uint64_t rem = (uint64_t)k - ab;
            __syncthreads();
            for (int i = tid; i < kBuckets; i += NT) sm.hcnt[i] = 0u;
            __syncthreads();
            for_rows([&](float* v, int i0) {
                finalize(v, i0);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    const uint32_t kk = key_of(v[j]);
                    if (kk && (kk >> 20) == (uint32_t)b1) agg_count(sm.hcnt, (kk >> 8) & 0xFFFu);
                }
            });
            __syncthreads();
            const int b2 = gfind_from_top(sm.hcnt, kBuckets, rem, &ab, sm);
            rem -= ab;
            const uint32_t pre = ((uint32_t)b1 << 12) | (uint32_t)b2;
            __syncthreads();
            for (int i = tid; i < 256; i += NT) sm.hcnt[i] = 0u;
            __syncthreads();
            for_rows([&](float* v, int i0) {
                finalize(v, i0);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    const uint32_t kk = key_of(v[j]);
                    if (kk && (kk >> 8) == pre) agg_count(sm.hcnt, kk & 0xFFu);
                }
            });
            __syncthreads();
            const int b3 = gfind_from_top(sm.hcnt, 256, rem, &ab, sm);
            const uint32_t kth = (pre << 8) | (uint32_t)b3;
            kth_y = val_of(kth) / Tt;
        }
        const float lp_min = (prm.min_p > 0.0f) ? log_det(prm.min_p < 1.0f ? prm.min_p : 1.0f)
                                                : -__builtin_inff();
        const float q32 = 1.0f - prm.top_p;
        const bool topp = q32 > 0.0f;
        const bool abl = topp && !(q32 < 1.0f);
        // (raw logprobs are of the unmasked, unpenalised logits: the sampling sum serves them
        // only when nothing changes a logit)
        const bool share_lse = (L >= 0) && !hh && !tb && !mrow && Tt == 1.0f && kth_y == -__builtin_inff() &&
                               lp_min == -__builtin_inff();
        auto survivor = [&](float x, float& y, float& d) -> bool {
            y = (Tt == 1.0f) ? x : x / Tt;
            d = y - m;
            return key_of(y) != 0u && y >= kth_y && d >= lp_min;
        };
        auto bucket_of = [&](float d) -> int {
            const float dd = -d;  // = fl(m - y) >= 0
            return dd < 32.0f ? (int)(dd * 128.0f) : kBuckets - 1;
        };

        RaceAcc race;
        uint64_t W = 0, thr = 0, nk_all = 0;
        double s0_shared = 0.0;
        if (abl) {
            // top_p <= 0: only the last token of the ascending order survives
            if (tid == 0) {
                const int idx = argmax_hi;
                const float y = val_of(maxkey) / Tt;
                race.add(1.0f, key_of(y), idx, row_uniform(a, r, idx));
            }
            if (share_lse) {
                for_rows([&](float* v, int i0) {
#pragma unroll
                    for (int j = 0; j < VEC; ++j) if (v[j] == v[j]) s0_shared += (double)exp_det(v[j] - m);
                });
            }
        } else if (!topp) {
            // no top-p: every survivor of top-k and min-p races
            for_rows_u([&](float* v, int i0, const float* uc) {
                finalize(v, i0);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    float y, d;
                    if (survivor(v[j], y, d)) {
                        const float e = exp_det(d);
                        if (share_lse) s0_shared += (double)e;
                        race.add(e, key_of(y), i0 + j, urow ? uc[j] : row_uniform(a, r, i0 + j));
                    } else if (share_lse && v[j] == v[j]) {
                        s0_shared += (double)exp_det(d);
                    }
                }
            });
        } else {
            // ---- pass B: masses per bucket
            for (int i = tid; i < kBuckets; i += NT) sm.hmass[i] = 0ull;
            __syncthreads();
            uint64_t wl = 0, nkl = 0;
            for_rows([&](float* v, int i0) {
                finalize(v, i0);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    float y, d;
                    if (survivor(v[j], y, d)) {
                        const float e = exp_det(d);
                        if (share_lse) s0_shared += (double)e;
                        const uint64_t w = mass_of(e);
                        wl += w;
                        nkl++;
                        if (w) agg_add64(sm.hmass, (uint32_t)bucket_of(d), w);
                    } else if (share_lse && v[j] == v[j]) {
                        s0_shared += (double)exp_det(d);
                    }
                }
            });
            W = gblock_sum(wl, sm);
            nk_all = gblock_sum(nkl, sm);
            thr = scale_floor(q32, W);
            uint64_t cbelow;
            const int bstar = gfind_from_top(sm.hmass, kBuckets, thr + 1, &cbelow, sm);

            // ---- pass C: race above b*, gather b*
            if (tid == 0) sm.gcount = 0u;
            __syncthreads();
            uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
            for_rows_u([&](float* v, int i0, const float* uc) {
                finalize(v, i0);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    float y, d;
                    if (!survivor(v[j], y, d)) continue;
                    const int b = bucket_of(d);
                    if (b < bstar) {
                        race.add(exp_det(d), key_of(y), i0 + j, urow ? uc[j] : row_uniform(a, r, i0 + j));
                    } else if (b == bstar) {
                        const uint32_t ky = key_of(y);
                        kmin = min(kmin, ky);
                        kmax = max(kmax, ky);
                        const uint32_t pos = agg_reserve(&sm.gcount);
                        if (pos < (uint32_t)kGatherCap) sm.u.gather[pos] = ((uint64_t)ky << 32) | (uint32_t)(i0 + j);
                    }
                }
            });
            const uint64_t kminb = gblock_min(kmin, sm);
            const uint64_t kmaxb = gblock_max(kmax, sm);
            const uint32_t ng = sm.gcount;
            const uint64_t n_above_c = gblock_sum(race.nkept, sm);

            uint32_t klo = (uint32_t)kminb, khi = (uint32_t)kmaxb;
            uint64_t cb = cbelow;       // mass of survivors below [klo, khi] in the ascending order
            uint32_t nrange = ng;       // survivors in bucket b* with key in [klo, khi]
            uint64_t n_p_above = 0;     // survivors in bucket b* with key > khi (kept)
            bool gathered = ng <= (uint32_t)kGatherCap;
            uint32_t idx_thr = 0;
            uint64_t wt = 0, rrem = 0;
            bool tie_rule = false;
            auto in_bstar = [&](float x, float& y, float& d) -> bool {
                return survivor(x, y, d) && bucket_of(d) == bstar;
            };
            if (!gathered) {
                // ---- refinement: split [klo, khi] into 4096 key sub-ranges until the boundary
                // range fits in LDS or is a single key
                for (int iter = 0; iter < 8; ++iter) {
                    const uint64_t span = (uint64_t)khi - klo + 1ull;
                    for (int i = tid; i < kBuckets; i += NT) { sm.hmass[i] = 0ull; sm.hcnt[i] = 0u; }
                    __syncthreads();
                    for_rows([&](float* v, int i0) {
                        finalize(v, i0);
#pragma unroll
                        for (int j = 0; j < VEC; ++j) {
                            float y, d;
                            if (!in_bstar(v[j], y, d)) continue;
                            const uint32_t ky = key_of(y);
                            if (ky < klo || ky > khi) continue;
                            const int s = kBuckets - 1 - (int)(((uint64_t)(ky - klo) * kBuckets) / span);
                            const uint64_t w = mass_of(exp_det(d));
                            if (w) agg_add64(sm.hmass, (uint32_t)s, w);
                            agg_count(sm.hcnt, (uint32_t)s);
                        }
                    });
                    __syncthreads();
                    uint64_t below_in;
                    const int sp = gfind_from_top(sm.hmass, kBuckets, thr + 1 - cb, &below_in, sm);
                    const int s = kBuckets - 1 - sp;
                    // keys above the crossing sub-range (still inside [klo, khi]) are kept
                    uint64_t above_cnt = 0;
                    for (int i = tid; i < sp; i += NT) above_cnt += sm.hcnt[i];
                    above_cnt = gblock_sum(above_cnt, sm);
                    const uint32_t nlo = klo + (uint32_t)(((uint64_t)s * span + kBuckets - 1) / kBuckets);
                    const uint32_t nhi = klo + (uint32_t)((((uint64_t)(s + 1) * span + kBuckets - 1) / kBuckets) - 1);
                    n_p_above += above_cnt;
                    cb += below_in;
                    nrange = sm.hcnt[sp];
                    klo = nlo;
                    khi = nhi;
                    __syncthreads();
                    if (nrange <= (uint32_t)kGatherCap || klo == khi) break;
                }
                if (nrange > (uint32_t)kGatherCap) {
                    // a single tie group: every member has the same y, e and w; members are removed
                    // in index order, so the survivors are those at or after the (rrem+1)-th index
                    tie_rule = true;
                    wt = mass_of(exp_det(val_of(klo) - m));
                    rrem = (thr - cb) / wt;
                    uint64_t rank = rrem + 1;  // 1-based rank of the first kept member
                    for (int i = tid; i < 1024; i += NT) sm.hcnt[i] = 0u;
                    __syncthreads();
                    for_rows([&](float* v, int i0) {
                        finalize(v, i0);
#pragma unroll
                        for (int j = 0; j < VEC; ++j) {
                            float y, d;
                            if (in_bstar(v[j], y, d) && key_of(y) == klo)
                                agg_count(sm.hcnt, 1023u - (uint32_t)((i0 + j) >> 9));
                        }
                    });
                    __syncthreads();
                    uint64_t ab;
                    const int c1 = gfind_from_top(sm.hcnt, 1024, rank, &ab, sm);
                    rank -= ab;
                    const int hi_bits = 1023 - c1;
                    __syncthreads();
                    for (int i = tid; i < 1024; i += NT) sm.hcnt[i] = 0u;
                    __syncthreads();
                    for_rows([&](float* v, int i0) {
                        finalize(v, i0);
#pragma unroll
                        for (int j = 0; j < VEC; ++j) {
                            float y, d;
                            const int ix = i0 + j;
                            if ((ix >> 9) == hi_bits && in_bstar(v[j], y, d) && key_of(y) == klo)
                                agg_count(sm.hcnt, 1023u - (uint32_t)(ix & 511));
                        }
                    });
                    __syncthreads();
                    const int c2 = gfind_from_top(sm.hcnt, 1024, rank, &ab, sm);
                    idx_thr = ((uint32_t)hi_bits << 9) | (uint32_t)(1023 - c2);
                }
                // ---- final pass over b*: race above the range, gather the range (or apply the
                // tie rule)
                if (tid == 0) sm.gcount = 0u;
                __syncthreads();
                for_rows_u([&](float* v, int i0, const float* uc) {
                    finalize(v, i0);
#pragma unroll
                    for (int j = 0; j < VEC; ++j) {
                        float y, d;
                        if (!in_bstar(v[j], y, d)) continue;
                        const uint32_t ky = key_of(y);
                        const int ix = i0 + j;
                        if (ky > khi) {
                            race.add(exp_det(d), ky, ix, urow ? uc[j] : row_uniform(a, r, ix));
                        } else if (ky >= klo) {
                            if (tie_rule) {
                                if ((uint32_t)ix >= idx_thr) race.add(exp_det(d), ky, ix, urow ? uc[j] : row_uniform(a, r, ix));
                            } else {
                                const uint32_t pos = agg_reserve(&sm.gcount);
                                if (pos < (uint32_t)kGatherCap) sm.u.gather[pos] = ((uint64_t)ky << 32) | (uint32_t)ix;
                            }
                        }
                    }
                });
                __syncthreads();
                gathered = !tie_rule;
            }

            // ---- resolve the gathered boundary range exactly
            uint64_t cprev = 0, cat = ~0ull;
            bool any_removed;
            if (gathered) {
                const uint32_t n = sm.gcount;
                uint32_t P = 1;
                while (P < n) P <<= 1;
                for (uint32_t i = n + tid; i < P; i += NT) sm.u.gather[i] = ~0ull;
                __syncthreads();
                for (uint32_t size = 2; size <= P; size <<= 1) {
                    for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                        for (uint32_t t = tid; t < P / 2; t += NT) {
                            const uint32_t i = 2 * t - (t & (stride - 1));
                            const uint32_t j = i + stride;
                            const bool up = (i & size) == 0;
                            const uint64_t x = sm.u.gather[i], z = sm.u.gather[j];
                            if ((x > z) == up) { sm.u.gather[i] = z; sm.u.gather[j] = x; }
                        }
                        __syncthreads();
                    }
                }
                // inclusive prefix of masses in sorted order: 2 entries per thread
                uint64_t w0 = 0, w1 = 0;
                const uint32_t j0 = 2 * tid, j1 = 2 * tid + 1;
                if (j0 < n) w0 = mass_of(exp_det(val_of((uint32_t)(sm.u.gather[j0] >> 32)) - m));
                if (j1 < n) w1 = mass_of(exp_det(val_of((uint32_t)(sm.u.gather[j1] >> 32)) - m));
                // exclusive prefix over threads in ascending order = total - suffix_incl
                const uint64_t pair = w0 + w1;
                const uint64_t suf = gblock_suffix_excl(pair, sm);  // over threads > tid
                const uint64_t tot = gblock_sum(pair, sm);
                const uint64_t before = tot - suf - pair;
                uint32_t nrem_in = 0;
                for (int q = 0; q < 2; ++q) {
                    const uint32_t j = q ? j1 : j0;
                    if (j >= n) continue;
                    const uint64_t C = cb + before + w0 + (q ? w1 : 0ull);
                    const bool removed = (C <= thr && C != W);
                    const uint64_t g = sm.u.gather[j];
                    const uint32_t ky = (uint32_t)(g >> 32);
                    const int ix = (int)(uint32_t)g;
                    if (removed) { nrem_in++; cprev = cprev > C ? cprev : C; }
                    else {
                        cat = cat < C ? cat : C;
                        race.add(exp_det(val_of(ky) - m), ky, ix, row_uniform(a, r, ix));
                    }
                }
                const uint64_t nrem_b = gblock_sum(nrem_in, sm);
                const uint64_t kept_in = (uint64_t)n - nrem_b;
                const uint64_t removed_below = nk_all - n_above_c - n_p_above - kept_in - nrem_b;
                cprev = gblock_max(cprev, sm);
                if (nrem_b == 0 && removed_below > 0) cprev = cb;
                any_removed = (nrem_b + removed_below) > 0;
                cat = gblock_min(cat, sm);
            } else {
                // tie rule
                cat = cb + (rrem + 1) * wt;
                const uint64_t removed_below = nk_all - n_above_c - n_p_above - nrange;
                any_removed = rrem > 0 || removed_below > 0;
                cprev = rrem > 0 ? cb + rrem * wt : cb;
            }
            if (tid == 0) {
                const uint64_t tol = (uint64_t)((double)W * 1e-6);
                if ((any_removed && thr - cprev <= tol) || (cat > thr && cat - thr <= tol))
                    sm.bc32[3] = VWS_FLAG_TOPP_NEAR_TIE;
                else
                    sm.bc32[3] = 0u;
            }
            __syncthreads();
            flags |= sm.bc32[3];
        }

        // ---- combine the race over the workgroup
        const uint64_t best = gblock_max(race.best, sm);
        uint32_t second = race.second;
        {
            const uint32_t loser = (race.best && race.best != best) ? (uint32_t)(race.best >> 32) + 1u : 0u;
            second = second > loser ? second : loser;
        }
        const uint64_t sec = gblock_max(second, sm);
        const uint64_t lastk = gblock_max(race.last, sm);
        nkept_out = (int32_t)gblock_sum(race.nkept, sm);
        if (best) {
            token = (int32_t)(0x7FFFFFFF - (uint32_t)(best & 0xFFFFFFFFu));
            if (sec) {
                const float bk = u2f((uint32_t)(best >> 32));
                const float sk = u2f((uint32_t)sec - 1u);
                if ((double)sk >= (double)bk * (1.0 - 1e-6)) flags |= VWS_FLAG_RACE_NEAR_TIE;
            }
        } else {
            token = (int32_t)(uint32_t)(lastk & 0xFFFFFFFFu);
        }
        if (share_lse) {
            const double s0 = gblock_sum_f64(s0_shared, sm);
            if (tid == 0) sm.bc64[4] = (uint64_t)__double_as_longlong(s0);
            __syncthreads();
        } else if (tid == 0) {
            sm.bc64[4] = 0ull;
        }
    }

logprobs:
    if (tid == 0) {
        a.sampled[r] = token;
        if (a.flags) a.flags[r] = flags;
        if (a.nkept) a.nkept[r] = nkept_out;
    }
    if (L >= 0) {
        __syncthreads();
        const float m0 = m0key ? val_of(m0key) : 0.0f;
        float raw_s = Elem<T>::load1(row + token);
        if (a.softcap > 0.0f) raw_s = softcap_out(raw_s, a.inv_softcap, a.softcap, a.softcap_f16 != 0);
        const uint32_t ks = key_of(raw_s);
        double s0 = 0.0;
        const bool have_s0 = !prm.greedy && sm.bc64[4] != 0ull;
        uint32_t rank = 0;
        for_rows([&](float* v, int i0) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const uint32_t kk = key_of(v[j]);
                if (!kk) continue;
                rank += kk >= ks ? 1u : 0u;
                if (!have_s0) s0 += (double)exp_det(v[j] - m0);
            }
        });
        const uint32_t rk = (uint32_t)gblock_sum(rank, sm);
        const double S0 = have_s0 ? __longlong_as_double((long long)sm.bc64[4]) : gblock_sum_f64(s0, sm);
        const float logS = (float)log(S0);
        const int stride = L + 1;
        if (tid == 0) {
            a.lp_ids[(size_t)r * stride] = token;
            a.lp_vals[(size_t)r * stride] = (raw_s - m0) - logS;
            a.lp_ranks[r] = (int32_t)rk;
        }
        // Fewer than L elements that are not NaN: the rest of the top L are the row's NaN
        // elements in index order (a sort by key puts them last, lowest index first), found by
        // wave 0 a block of 64 at a time (it stops once it has them: such a row is short or
        // mostly NaN), then -1 / NaN past the row's end
        auto fill_rest = [&](int n) {
            if (n >= L || wave != 0) return;
            const int need = L - n;
            int found = 0;
            for (int base = 0; base < V && found < need; base += kWave) {
                const int i = base + lane;
                const float xi = i < V ? Elem<T>::load1(row + i) : 0.0f;
                const bool isn = i < V && !(xi == xi);
                const uint64_t bal = wave_ballot(isn);
                const int pos = found + lane_prefix(bal);
                if (isn && pos < need) {
                    a.lp_ids[(size_t)r * stride + 1 + n + pos] = i;
                    a.lp_vals[(size_t)r * stride + 1 + n + pos] = __builtin_nanf("");
                }
                found += __popcll(bal);
            }
            for (int j = n + min(found, need) + lane; j < L; j += kWave) {
                a.lp_ids[(size_t)r * stride + 1 + j] = -1;
                a.lp_vals[(size_t)r * stride + 1 + j] = __builtin_nanf("");
            }
        };
        // the buffered top-L candidates overflowed (ties) or their cut holds more than the 128
        // gathered: the exact selection over the row
        const bool exact_sel = L > 0 && (sm.bc32[2] != 0u || sm.nsel > 128u);
        if (exact_sel) {
            const uint32_t n = general_topk_select<T>(a, sm, r, L);
            for (uint32_t j = tid; j < n; j += NT) {
                const uint64_t g = sm.u.gather[j];
                a.lp_ids[(size_t)r * stride + 1 + j] = (int32_t)(uint32_t)g;
                a.lp_vals[(size_t)r * stride + 1 + j] = (val_of(~(uint32_t)(g >> 32)) - m0) - logS;
            }
            fill_rest((int)n);
        } else if (L > 0) {
            const uint32_t n = min(sm.nsel, 128u);
            for (uint32_t j = tid; j < n; j += NT) {
                const uint32_t kj = sm.lp_sel_key[j];
                const int32_t ij = sm.lp_sel_idx[j];
                int pos = 0;
                for (uint32_t i = 0; i < n; ++i) {
                    const uint32_t ki = sm.lp_sel_key[i];
                    pos += (ki > kj || (ki == kj && sm.lp_sel_idx[i] < ij)) ? 1 : 0;
                }
                if (pos < L) {
                    a.lp_ids[(size_t)r * stride + 1 + pos] = ij;
                    a.lp_vals[(size_t)r * stride + 1 + pos] = (val_of(kj) - m0) - logS;
                }
            }
            fill_rest((int)n);
        }
    }
    // the workspace is left as it was found (zeros): other operations that share it, such as
    // the top-k's part counters, overlap the hash region
    if (hh) {
        __syncthreads();
        for (int i = tid; i < hs; i += NT) { hkey[i] = 0u; hval[i] = 0u; hpen[i] = 0u; hadj[i] = 0u; }
    }
}

// Exact top-k of a row by raw value (after the soft cap, if any): the k-th largest key by a
// 3-level radix select, the tie group at that key cut by an index radix select (lowest indices
// first), then the winners sorted by (value desc, index asc) into sm.u.gather as
// (~key << 32) | index.  Returns the number of winners, min(k, non-NaN elements).
template <typename T>
__device__ __forceinline__ uint32_t general_topk_select(const KArgs& a, GenSmem& sm, int r, int k) {
    constexpr int NT = kGenThreads;
    constexpr int VEC = Elem<T>::kVec;
    const int tid = threadIdx.x;
    const int V = a.V;
    const T* row = reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride;
    Slice<T> sl;
    sl.init(row, 0, V);
    const int nit = (sl.nchunks() + 2 * NT - 1) / (2 * NT);
    auto for_rows = [&](auto&& f) {
        for (int it = 0; it < nit; ++it) {
            float v0[VEC], v1[VEC];
            const int c0 = it * 2 * NT + tid;
            const int i0 = sl.load(c0, v0);
            const int i1 = sl.load(c0 + NT, v1);
            if (a.softcap > 0.0f) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    v0[j] = softcap_out(v0[j], a.inv_softcap, a.softcap, a.softcap_f16 != 0);
                    v1[j] = softcap_out(v1[j], a.inv_softcap, a.softcap, a.softcap_f16 != 0);
                }
            }
            f(v0, i0);
            f(v1, i1);
        }
    };
    uint32_t nvalid = 0;
    __syncthreads();
    for (int i = tid; i < kBuckets; i += NT) sm.hcnt[i] = 0u;
    __syncthreads();
    for_rows([&](float* v, int i0) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const uint32_t kk = key_of(v[j]);
            if (kk) { nvalid++; agg_count(sm.hcnt, kk >> 20); }
        }
    });
    const uint32_t nval = (uint32_t)gblock_sum(nvalid, sm);
    const int kk_eff = (uint32_t)k < nval ? k : (int)nval;
    if (kk_eff == 0) return 0u;
    uint64_t ab;
    const int b1 = gfind_from_top(sm.hcnt, kBuckets, (uint64_t)kk_eff, &ab, sm);
    uint64_t rem = (uint64_t)kk_eff - ab;
    __syncthreads();
    for (int i = tid; i < kBuckets; i += NT) sm.hcnt[i] = 0u;
    __syncthreads();
    for_rows([&](float* v, int i0) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const uint32_t kk = key_of(v[j]);
            if (kk && (kk >> 20) == (uint32_t)b1) agg_count(sm.hcnt, (kk >> 8) & 0xFFFu);
        }
    });
    __syncthreads();
    const int b2 = gfind_from_top(sm.hcnt, kBuckets, rem, &ab, sm);
    rem -= ab;
    const uint32_t pre = ((uint32_t)b1 << 12) | (uint32_t)b2;
    __syncthreads();
    for (int i = tid; i < 256; i += NT) sm.hcnt[i] = 0u;
    __syncthreads();
    for_rows([&](float* v, int i0) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const uint32_t kk = key_of(v[j]);
            if (kk && (kk >> 8) == pre) agg_count(sm.hcnt, kk & 0xFFu);
        }
    });
    __syncthreads();
    const int b3 = gfind_from_top(sm.hcnt, 256, rem, &ab, sm);
    rem -= ab;  // members of the k-th key's tie group that make the cut (lowest indices)
    const uint32_t kth = (pre << 8) | (uint32_t)b3;
    // index of the rem-th smallest member of the tie group
    __syncthreads();
    for (int i = tid; i < 1024; i += NT) sm.hcnt[i] = 0u;
    __syncthreads();
    for_rows([&](float* v, int i0) {
#pragma unroll
        for (int j = 0; j < VEC; ++j)
            if (key_of(v[j]) == kth) agg_count(sm.hcnt, 1023u - (uint32_t)((i0 + j) >> 9));
    });
    __syncthreads();
    uint64_t rank = rem;
    const int c1 = gfind_from_top(sm.hcnt, 1024, rank, &ab, sm);
    rank -= ab;
    const int hi_bits = 1023 - c1;
    __syncthreads();
    for (int i = tid; i < 1024; i += NT) sm.hcnt[i] = 0u;
    __syncthreads();
    for_rows([&](float* v, int i0) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const int ix = i0 + j;
            if ((ix >> 9) == hi_bits && key_of(v[j]) == kth) agg_count(sm.hcnt, 1023u - (uint32_t)(ix & 511));
        }
    });
    __syncthreads();
    const int c2 = gfind_from_top(sm.hcnt, 1024, rank, &ab, sm);
    const uint32_t idx_last = ((uint32_t)hi_bits << 9) | (uint32_t)(1023 - c2);
    // gather the k winners, sort by (key desc, index asc): sort ascending on (~key, index)
    if (tid == 0) sm.gcount = 0u;
    __syncthreads();
    for_rows([&](float* v, int i0) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const uint32_t kk = key_of(v[j]);
            const int ix = i0 + j;
            if (kk > kth || (kk == kth && (uint32_t)ix <= idx_last)) {
                const uint32_t pos = agg_reserve(&sm.gcount);
                if (pos < (uint32_t)kGatherCap) sm.u.gather[pos] = ((uint64_t)(~kk) << 32) | (uint32_t)ix;
            }
        }
    });
    __syncthreads();
    const uint32_t n = min(sm.gcount, (uint32_t)kGatherCap);
    uint32_t P = 1;
    while (P < n) P <<= 1;
    for (uint32_t i = n + tid; i < P; i += NT) sm.u.gather[i] = ~0ull;
    __syncthreads();
    for (uint32_t size = 2; size <= P; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t t = tid; t < P / 2; t += NT) {
                const uint32_t i = 2 * t - (t & (stride - 1));
                const uint32_t j = i + stride;
                const bool up = (i & size) == 0;
                const uint64_t x = sm.u.gather[i], z = sm.u.gather[j];
                if ((x > z) == up) { sm.u.gather[i] = z; sm.u.gather[j] = x; }
            }
            __syncthreads();
        }
    }
    return n < (uint32_t)k ? n : (uint32_t)k;
}

// The top k of a row with fewer than k elements that are not NaN (positions [0, n) written):
// positions [n, k) take the row's NaN elements in index order (a sort by key puts them last,
// lowest index first); the caller has set every position to -1 / NaN before.  Called by one
// whole wave, which scans the row 64 elements at a time and stops once it has them (such a row
// is short or mostly NaN).
template <typename T>
__device__ __forceinline__ void topk_fill_nan(const T* row, int V, int n, int k, float* vals,
                                              int32_t* ids) {
    const int lane = threadIdx.x & 63;
    const int need = k - n;
    int found = 0;
    for (int base = 0; base < V && found < need; base += kWave) {
        const int i = base + lane;
        const float xi = i < V ? Elem<T>::load1(row + i) : 0.0f;
        const bool isn = i < V && !(xi == xi);
        const uint64_t bal = wave_ballot(isn);
        const int pos = found + lane_prefix(bal);
        if (isn && pos < need) {
            vals[n + pos] = __builtin_nanf("");
            ids[n + pos] = i;
        }
        found += __popcll(bal);
    }
}

// Exact top-k ids/values of a row for the topk operation, when its single-pass list
// overflowed (ties).
template <typename T>
__device__ __forceinline__ void general_topk_row(const KArgs& a, GenSmem& sm, int r) {
    const int k = a.topk_k;
    for (int i = threadIdx.x; i < k; i += kGenThreads) {
        a.topk_vals[(size_t)r * k + i] = __builtin_nanf("");
        a.topk_ids[(size_t)r * k + i] = -1;
    }
    const uint32_t n = general_topk_select<T>(a, sm, r, k);
    for (uint32_t j = threadIdx.x; j < n; j += kGenThreads) {
        const uint64_t g = sm.u.gather[j];
        a.topk_vals[(size_t)r * k + j] = val_of(~(uint32_t)(g >> 32));
        a.topk_ids[(size_t)r * k + j] = (int32_t)(uint32_t)g;
    }
    if ((int)n < k && threadIdx.x < kWave)
        topk_fill_nan<T>(reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride, a.V, (int)n,
                         k, a.topk_vals + (size_t)r * k, a.topk_ids + (size_t)r * k);
}

}  // namespace vws
