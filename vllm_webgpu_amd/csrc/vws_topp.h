// vws_topp.h -- single-pass sampling of rows whose survivors are cut by top-p alone (top-k off,
// 0 < top_p < 1), and of greedy rows that ask for raw logprobs.
//
// One 1024-thread workgroup streams the row once (16-byte non-temporal buffer loads, two
// iterations in flight, as in the single-pass kernel).  Each wave stores the elements of its
// share at or above a threshold in an LDS candidate buffer (the threshold is seeded from the
// first iteration so that the buffers hold a few percent of the row, and raised when a buffer
// would overflow) and adds every other element into an approximate mass sum: the term 2^z,
// z = (x - a) c, from the hardware exp2, c = log2(e) / T, a the row's anchor (its seed), plus
// the sum of |z| 2^z for the error bound.  After the stream:
//   * the row maximum is the largest candidate; candidates below the highest wave threshold
//     join the sum exactly; the others get exact masses floor(exp_det(y - max) 2^44) in 2048
//     buckets of max - y;
//   * the exact mass of everything below the threshold lies in an interval [S_lo, S_hi] built
//     from the approximate sum and its error bound.  Top-p's threshold, boundary bucket, cut
//     inside that bucket and near-tie flags are computed at both ends of the interval; when
//     they differ, or when the boundary lies below the candidates (or min-p keeps elements
//     below them), one more pass over the row adds the exact masses of everything below the
//     candidates into the buckets and the decision is taken again on exact values;
//   * when the boundary bucket then reaches the values below the candidates (a wide row), a
//     further pass over the logits and the uniforms races the survivors it keeps there and
//     gathers the boundary bucket's members there;
//   * the race runs over the kept candidates (uniforms read at their positions only), and raw
//     logprobs come from the candidates (top-L, rank) and the sums (log-sum-exp); a sampled
//     token below the candidates is ranked by one more pass.
// Rows with penalties from a token-state table that comes with its bitmap of non-zero words
// stream their raw values like any other row; the finish stages the bitmap in LDS, adds the
// history tokens the stream did not buffer to the buffers (taking their terms out of the sums),
// so that nothing outside the buffers is penalised, and gives every history token its processed
// value from its word.  Rows with penalties from id lists, logits processors, an allowed mask or
// the soft cap, rows whose buffers overflow (ties) and the rare rows listed under VWS_FALLBACK_*
// take the multi-pass path
// instead; nothing is written for them here.
#pragma once

#include "vws_row.h"

namespace vws {

constexpr int kTpWaves = kGenWaves;       // 16
constexpr int kTpCapW = 832;              // candidate slots per wave
constexpr int kTpSlots = kTpCapW + kWave; // slots per wave: the candidates, then one spare per lane
constexpr int kTpSoft = 704;              // a wave holding more after half an iteration compacts
constexpr int kTpKeep = 512;              // entries a compaction keeps (ties included)
constexpr float kTpFill = 0.65f;          // share of the slots the seed threshold aims to fill
constexpr int kTpBuckets = 2048;          // exact-mass buckets of width 1/64 over max - y in [0, 32)
constexpr int kTpGather = 2048;           // members of the boundary bucket resolved in LDS
constexpr int kTpRankCap = 512;           // up to this many, ranked without sorting them
constexpr int kTpRankSerial = 64;         // up to this many, one thread ranks each member
constexpr int kTpLpCap = 256;             // candidates gathered for the top-L logprobs
constexpr float kLog2e = 0x1.715476p+0f;  // log2(e) rounded to fp32
constexpr int kTpHistMaxV = 196608;       // history rows: V up to the LDS bitmap's bits
constexpr int kTpHistWords = kTpHistMaxV / 32 + 2;  // (two words of padding for 64-bit windows)
// Index-word mark of a buffered history token (history rows only: their indices are below 2^18,
// so bit 18 is free; other rows use it for the index).
constexpr uint32_t kTpHist = 1u << 18;
constexpr int kTpRawCap = 512;            // history tokens at or above the threshold by raw value

// Why a row left the single-pass top-p path (recorded in bits 16-23 of its result flags, which
// are diagnostic like VWS_FLAG_GENERAL_PATH).
constexpr int VWS_FALLBACK_OVERFLOW = 1;    // a wave's candidate buffer overflowed (ties)
constexpr int VWS_FALLBACK_SUM = 2;         // the approximate sum is not finite
constexpr int VWS_FALLBACK_DEGENERATE = 3;  // no finite row maximum
constexpr int VWS_FALLBACK_AMBIGUOUS = 6;   // the exact recount still cuts inconsistently
constexpr int VWS_FALLBACK_GATHER = 7;      // the boundary bucket holds too many members
constexpr int VWS_FALLBACK_TOPL = 8;        // the top-L logprobs reach below the candidates
constexpr int VWS_FALLBACK_COOP = 9;        // a cooperative pass was not completed in time


// The finish's further passes over the row (the rarer cases; tp_pass_range).
constexpr int kTpPassExact = 0;     // exact masses below the candidates
constexpr int kTpPassWideRace = 1;  // the race and the boundary members below the candidates
constexpr int kTpPassRank = 2;      // the rank of a sampled token below the candidates

// One further pass over a row, as every workgroup that works on it sees it.
struct TpPassDesc {
    int kind;                   // kTpPass*
    uint32_t key;               // the row's threshold key tauk (rank pass: the sampled token's key)
    int bstar;                  // wide race: the boundary bucket
    float Tt, m, lp_min;        // temperature, max y, min-p's bound on y - max (or -inf)
    uint32_t ksv, kkeep, kmem;  // wide race: key thresholds (tp_wide_keys)
};

// A workgroup's results over its share of a pass (per thread until tp_pass_reduce).
struct TpPassAcc {
    uint64_t sw = 0, n = 0;  // exact: survivors' mass and number; rank: elements at or above the key
    RowRace rs;              // wide race: the kept survivors' race
    uint32_t nrem = 0;       // wide race: survivors top-p removes
};

struct TopPSmem {
    // Each wave's candidates: raw bits during the stream, order keys from the finish on; and
    // their indices.
    uint32_t ck[kTpWaves][kTpSlots];
    int32_t ci[kTpWaves][kTpSlots];
    union {
        uint32_t hb[kTpHistWords];        // finish of a history row, before the masses: bit t = token t's word is non-zero
        struct {
            uint64_t hmass[kTpBuckets];   // finish: exact masses of the surviving candidates
            uint32_t hcnt[kTpBuckets];    // and the number of candidates per bucket (top-L logprobs)
        } h;
    };
    union {
        uint32_t rhist[kTpWaves][256];    // stream: per-wave radix-select scratch
        uint32_t hl[2 * kTpGather];       // finish of a history row: unbuffered history tokens
        struct {
            uint64_t key[kTpGather];      // boundary bucket: key(y) << 32 | index
        } g;
        struct {
            uint64_t key[kTpRankCap];     // the same, for up to kTpRankCap members
            uint64_t w[kTpRankCap];       // their exact masses,
            uint64_t cum[kTpRankCap];     // the mass of the members at or below each one
            uint32_t rnk[kTpRankCap];     // and their number
        } rk;
        struct {
            uint32_t key[kTpLpCap];
            int32_t idx[kTpLpCap];
        } lp;
    };
    // per-wave results of the stream
    double wS[kTpWaves];                  // sum of the approximate terms below the threshold
    double wSR[kTpWaves];                 // the same over raw logits (T != 1, log-sum-exp)
    float wZ[kTpWaves];                   // sum of |z| * term (error bound)
    uint32_t wTau[kTpWaves];              // final threshold key
    uint32_t wCnt[kTpWaves];              // buffered entries
    uint32_t wMax[kTpWaves];              // largest buffered key (raw values)
    uint32_t wMaxP[kTpWaves];             // history rows: largest processed key
    float wS0h[kTpWaves];                 // history rows: their history tokens' raw normaliser terms
    double wSub[kTpWaves], wSRsub[kTpWaves];  // history rows: stream terms of the tokens added after it
    uint32_t hl_n;
    // history rows with raw logprobs: the history tokens at or above the threshold by raw value
    // (their buffered entries hold processed values): raw keys and indices
    uint32_t rl_key[kTpRawCap];
    int32_t rl_idx[kTpRawCap];
    uint32_t rl_n;
    // finish
    uint64_t red[kTpWaves][4];            // per-wave records of the finish's reductions
    double redd[kTpWaves];
    float anchor;                         // the row's anchor a
    // totals of the finish kept here rather than in registers across it: the candidates' mass
    // (updated by an exact pass), the number of survivors buffered below the threshold, the
    // buffered part of the raw log-sum-exp, the raw maximum
    uint64_t tot_wc, tot_nxs;
    double tot_s0b;
    float xr;
    // the wide race pass's results (wide rows): best, second, kept, last (RowRace fields)
    uint64_t wrace[4];
    uint32_t status;                      // bit 0: buffer overflow, bit 1: non-finite sum
    uint32_t bc[16];
    uint64_t bc64[16];
    // cooperative passes: the pass being run, broadcasts, and whether the row holds a count in
    // CoopState::wgs (released when the row is done)
    TpPassDesc pd;
    uint32_t cp[19];
    uint32_t coop_hold;
    uint32_t coop_fail;                   // a cooperative pass of the row was not completed
    uint32_t ninf;                        // masked rows: -inf elements left out of the buffers
};

// Entries dropped by a compaction, as terms of the approximate sum (per lane), and the new
// threshold and count (wave-uniform).
struct TpDrop {
    double s, sr;
    float z;
    uint32_t kth;
    int cnt;
};

// Out of line (compaction is rare); defined next to the LDS it works on.
__device__ __noinline__ TpDrop topp_compact_entry(int w, int cnt, float aw, float c, int want_raw);

// Whether the single-pass top-p path may serve the row.
__device__ __forceinline__ bool topp_eligible(const KArgs& a, const RowP& p) {
    if (p.need_hash) return false;
    // an allowed mask: the stream masks as it loads (rows starting 16-byte aligned, checked by
    // the caller); with raw logprobs such launches take the multi-pass path.  The soft cap: the
    // stream caps as it loads (not together with a mask)
    if (a.allowed && (a.L >= 0 || a.softcap > 0.0f)) return false;
    // penalties: from the token-state table with its bitmap (need_hash covers the lists)
    if (p.has_hist && !(p.tab && a.tbits && a.V <= kTpHistMaxV)) return false;
    if (p.greedy) return a.L >= 0;
    const bool topk_off = p.k <= 0 || p.k >= a.V;
    return topk_off && p.top_p > 0.0f && p.top_p < 1.0f;
}

// Term of the approximate sum, 2^z with z = max((x - aw) c, -256) by the hardware exp2; z is
// returned for the error bound.  NaN and -inf give z = -256 and a zero term.
__device__ __forceinline__ float tp_term(float x, float aw, float c, float& z) {
    z = __builtin_fmaxf((x - aw) * c, -256.0f);
    return __builtin_amdgcn_exp2f(z);
}

// Bucket of d = y - max <= 0: floor(-d * 64), the last bucket from -d >= 32 on (zero masses).
// (d > 0 cannot occur; it would land in bucket 0.)
__device__ __forceinline__ int tp_bucket(float d) {
    const float dd = __builtin_fmaxf(-d, 0.0f);
    return dd < 32.0f ? (int)(dd * 64.0f) : kTpBuckets - 1;
}

// A buffered entry's index word from the finish on: the element index (bits 0-18; V <= 2^19),
// the entry's bucket (bits 19-29), a survivor bit and a bit for entries below the row's final
// threshold, so that later phases need no division or bucket of their own.
constexpr uint32_t kTpIdxMask = (1u << 19) - 1u;
constexpr uint32_t kTpSurv = 1u << 30;
constexpr uint32_t kTpBelow = 1u << 31;
__device__ __forceinline__ int tp_code_bucket(uint32_t c) { return (int)((c >> 19) & 0x7FFu); }
__device__ __forceinline__ bool tp_code_cand(uint32_t c) { return (c & (kTpBelow | kTpSurv)) == kTpSurv; }

__device__ __forceinline__ uint32_t tp_u(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint64_t tp_u64(uint64_t v) {
    return ((uint64_t)tp_u((uint32_t)(v >> 32)) << 32) | tp_u((uint32_t)v);
}
__device__ __forceinline__ float tp_uf(float v) { return u2f(tp_u(f2u(v))); }

// Per-wave candidate buffer of the top-p stream: every element of the wave's share at or above
// tau (raw bits and index); the rest joins the approximate sum (also the entries a compaction
// drops).
struct TpBuf {
    int w, cnt;
    uint32_t tau;
    float tauf;
    bool ovf;
    __device__ __forceinline__ void init(int w_) {
        w = w_; cnt = 0; tau = 0u; tauf = -__builtin_inff(); ovf = false;
    }
    __device__ __forceinline__ void set_tau(uint32_t t) {
        if (t > tau) {
            tau = t;
            tauf = (tau > 0x007FFFFFu) ? val_of(tau) : -__builtin_inff();
        }
    }
    // Stores the candidates of one vector of every lane (elements v[j] >= tauf of a vector in
    // the row, okv; first index i0; bal[j] the wave's ballot of element j's test), with one
    // capacity check for the whole vector: every lane writes, without branches, a candidate into
    // its slot (placed by mbcnt) and anything else into its spare slot past the capacity.
    // Wave-uniform call.  A full buffer marks the row for the multi-pass path (the stream
    // compacts every half iteration, from kTpSoft entries on, so this takes more than
    // kTpCapW - kTpSoft candidates in half an iteration of one wave).
    template <int VEC>
    __device__ __forceinline__ void append_vec(TopPSmem& sm, const float* v, const uint64_t* bal,
                                               bool okv, int i0) {
        int tot = 0;
#pragma unroll
        for (int j = 0; j < VEC; ++j) tot += __popcll(bal[j]);
        if (ovf || cnt + tot > kTpCapW) {
            if (!ovf && lane_id() == 0) atomicOr(&sm.status, 1u);
            ovf = true;
            return;
        }
        int base = cnt;
        const int spare = kTpCapW + lane_id();
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const int at = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal[j] >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((uint32_t)bal[j], (uint32_t)base));
            const bool c = okv & (v[j] >= tauf);  // the lanes of bal[j] (no short-circuit branch)
            const int pos = c ? at : spare;
            sm.ck[w][pos] = f2u(v[j]);
            sm.ci[w][pos] = i0 + j;
            base += __popcll(bal[j]);
        }
        cnt = base;
    }
};

// Boundary buckets of kTpRankSerial < ng <= kTpRankCap members (sm.rk.key, in any order): each
// member's exact mass (sm.rk.w), rank (the members at or below it, itself included: sm.rk.rnk)
// and the mass of the members at or below it (sm.rk.cum), counted by S threads per member over
// slices of at least 32 members each and added up in LDS (the keys are distinct: they hold the
// index).  Every thread calls it; the results are read after the caller's next barrier.
__device__ __forceinline__ void topp_rank_members(TopPSmem& sm, uint32_t ng, float m) {
    constexpr int NT = kGenThreads;
    const int tid = threadIdx.x;
    const int S = min(NT / (int)ng, (int)ng / 32);
    if (tid < (int)ng) {
        sm.rk.w[tid] = mass_of(exp_det(val_of((uint32_t)(sm.rk.key[tid] >> 32)) - m));
        sm.rk.cum[tid] = 0ull;
        sm.rk.rnk[tid] = 0u;
    }
    __syncthreads();
    if (tid < S * (int)ng) {
        const int c = tid % (int)ng, sl = tid / (int)ng;
        const int i0 = sl * (int)ng / S, i1 = (sl + 1) * (int)ng / S;
        const uint64_t gc = sm.rk.key[c];
        uint64_t cj = 0ull;
        uint32_t rj = 0u;
#pragma unroll 8
        for (int i = i0; i < i1; ++i) {
            const bool le = sm.rk.key[i] <= gc;
            cj += le ? sm.rk.w[i] : 0ull;
            rj += le ? 1u : 0u;
        }
        if (cj) atomicAdd((unsigned long long*)&sm.rk.cum[c], (unsigned long long)cj);
        if (rj) atomicAdd(&sm.rk.rnk[c], rj);
    }
}

// Out of line (defined next to the LDS it works on).
__device__ __noinline__ void topp_rank_members_entry(uint32_t ng, float m);

// Keeps the kTpKeep largest values (ties included) of wave w's buffer and raises its threshold
// to the smallest kept value; the dropped entries are returned as terms of the approximate sum.
__device__ __forceinline__ TpDrop topp_compact(TopPSmem& sm, int w, int cnt, float aw, float c,
                                               bool want_raw) {
    TpDrop d{0.0, 0.0, 0.0f, 0u, 0};
    const int lane = lane_id();
    uint32_t* ck = sm.ck[w];
    int32_t* ci = sm.ci[w];
    for (int i = lane; i < cnt; i += kWave) ck[i] = key_of(u2f(ck[i]));  // raw bits -> keys
    wave_sync();
    const uint32_t kth = wave_kth_largest(ck, cnt, kTpKeep, sm.rhist[w]);
    int out = 0;
    for (int base = 0; base < cnt; base += kWave) {
        const int i = base + lane;
        bool keep = false;
        uint32_t kk = 0u;
        int32_t ii = 0;
        if (i < cnt) {
            kk = ck[i];
            ii = ci[i];
            keep = kk >= kth;
            if (!keep) {
                const float x = val_of(kk);
                float z;
                const float t = tp_term(x, aw, c, z);
                d.s += (double)t;
                d.z = __builtin_fmaf(__builtin_fabsf(z), t, d.z);
                if (want_raw) {
                    float z2;
                    d.sr += (double)tp_term(x, aw, kLog2e, z2);
                }
            }
        }
        const uint64_t bal = wave_ballot(keep);
        if (keep) {
            const int pos = out + lane_prefix(bal);
            ck[pos] = f2u(val_of(kk));  // back to raw bits
            ci[pos] = ii;
        }
        out += __popcll(bal);
        wave_sync();
    }
    d.kth = kth;
    d.cnt = out;
    return d;
}

// The stream over row r.  Publishes each wave's results into sm; topp_finish completes the row.
// fill: the entries per wave the seed threshold aims at (less than kTpFill of the slots when
// history tokens will need some).
template <typename T, int XF>
__device__ __forceinline__ void topp_stream(const KArgs& a, TopPSmem& sm, int r, const RowP& prm,
                                            float fill) {
    constexpr bool MASK = XF == kXfMask, CAP = XF == kXfCap;
    constexpr int NT = kGenThreads;
    constexpr int VEC = Elem<T>::kVec;
    constexpr int U = 32 / VEC;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int V = a.V;
    const T* row = reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride;
    Slice<T> sl;
    sl.init(row, 0, V);
    const int nbody = sl.nbody;
    const int nit = (nbody + NT * U - 1) / (NT * U);
    const __amdgpu_buffer_rsrc_t lrs = make_rsrc(row + sl.a, 16u * (uint32_t)nbody);
    auto tid_now = [&]() __attribute__((always_inline)) { return wave * kWave + lane_now(); };
    // every byte offset in the vector offset: loads past the row's end return zeros
    auto load_iter = [&](float (&buf)[U][VEC], int it) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < U; ++q) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(
                lrs, 16u * (uint32_t)(tid_now() + (it * U + q) * NT), 0u, 2 /* nt */);
            Elem<T>::from_words((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3], buf[q]);
        }
    };
    // MASK: the row's allowed-token words, one per lane and iteration (lane l: word l % (2 VEC)
    // of the wave's vector group l / (2 VEC)); elements outside the mask become -inf as they
    // are loaded (the row starts 16-byte aligned, so the words line up with the vectors)
    const uint32_t* mrow = MASK ? a.allowed + (size_t)r * (size_t)a.astride : nullptr;
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(mrow, MASK ? 4u * (uint32_t)((V + 31) >> 5) : 0u);
    auto load_mask = [&](uint32_t& mw, int it) __attribute__((always_inline)) {
        if (MASK) {
            const int ln = lane_now();
            const uint32_t wi = (uint32_t)((((it * U + ln / (2 * VEC)) * NT + wave * kWave) * VEC) >> 5) +
                                (uint32_t)(ln % (2 * VEC));
            mw = __builtin_amdgcn_raw_buffer_load_b32(mrs, 4u * wi, 0u, 0);
        }
    };
    // CAP: every element of the iteration capped
    auto xf_iter = [&](float (&buf)[U][VEC], uint32_t mw) __attribute__((always_inline)) {
        if (CAP) {
            const bool f16 = a.softcap_f16 != 0;
#pragma unroll
            for (int q = 0; q < U; ++q)
#pragma unroll
                for (int j = 0; j < VEC; ++j) buf[q][j] = softcap_out(buf[q][j], a.inv_softcap, a.softcap, f16);
        }
        if (MASK) {
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
    float A[U][VEC], Bq[U][VEC];
    uint32_t MA = 0u, MB = 0u;
    load_iter(A, 0);
    load_mask(MA, 0);
    load_iter(Bq, 1);
    load_mask(MB, 1);
    xf_iter(A, MA);
    // seed: a threshold from the lane maxima over the first iteration.  A lane's maximum over its
    // E elements reaches tau with probability 1 - (1 - phi)^E when a fraction phi of the
    // elements does, so a wave's m-th largest lane maximum, m = 64 (1 - (1 - phi)^E), admits
    // about phi of the row; phi aims at kTpFill of the buffers' capacity.  Every wave uses the
    // median of the 16 waves' estimates (the row keeps every element at or above the highest
    // threshold any wave used, so one common threshold wastes no slots).
    float lmax = -__builtin_inff();
#pragma unroll
    for (int q = 0; q < U; ++q) {
        const bool ok = q * NT + tid < nbody;
#pragma unroll
        for (int j = 0; j < VEC; ++j) lmax = ok ? __builtin_fmaxf(lmax, A[q][j]) : lmax;
    }
    const float share = (float)V / (float)kTpWaves;
    const float phi = __builtin_fminf(1.0f, fill / share);
    const bool seeded = phi < 1.0f && nbody > 0;
    uint32_t tw = 0u;
    if (seeded) {
        // elements per lane in the first iteration (fewer when the row is shorter than it)
        const float e = __builtin_fminf((float)(U * VEC), __builtin_fmaxf(1.0f, (float)nbody * VEC / NT));
        const float pl = 1.0f - __builtin_amdgcn_exp2f(e * __builtin_amdgcn_logf(1.0f - phi));
        const int msel = min(64, max(1, (int)__builtin_ceilf(64.0f * pl)));
        tw = wave_mth_largest64(key_of(lmax), msel);
    }
    if (tid == 0) {
        sm.status = 0u;
        if (MASK) sm.ninf = 0u;
    }
    if (lane == 0) sm.bc[wave] = tw;  // bc is free until the finish's first barrier
    __syncthreads();
    VWS_TRACE_MARK(a, VWS_TRACE_SEED);
    uint32_t tau0 = 0u;
    if (seeded) tau0 = wave_mth_largest64_count<kTpWaves>(lane < kTpWaves ? sm.bc[lane] : 0u, kTpWaves / 2);
    if (tau0 <= 0x007FFFFFu || tau0 >= 0xFF800000u) tau0 = 0u;  // -inf, or +inf (degenerate row)
    const float aw = tau0 ? val_of(tau0) : 0.0f;
    const bool greedy = prm.greedy;
    const float c = greedy ? kLog2e : kLog2e / prm.T;
    const bool want_raw = a.L >= 0 && !greedy && prm.T != 1.0f;

    TpBuf cb;
    cb.init(wave);
    cb.set_tau(tau0);
    double acc = 0.0, accr = 0.0;
    float accz = 0.0f;
    uint64_t ninf = 0ull;  // MASK: -inf elements kept out of the buffers (some lane had one)
    // one vector of VEC elements starting at element i0 (okv: in the row; hv: the elements whose
    // history bit counts): candidates into the buffer, every other element into the sums (a zero
    // term for NaN and -inf).  The ballots of the element tests decide whether any lane appends
    // (no separate vector test: a wave almost always has a candidate somewhere in a vector
    // position).
    auto consume = [&](const float* v, int i0, bool okv) __attribute__((always_inline)) {
        uint64_t bal[VEC];
        uint64_t any = 0ull;
        // ballots of single compares (the compiler takes their lane masks as they are)
        const uint64_t okm = wave_ballot(okv);
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            // MASK: only finite values are candidates (a heavily masked row leaves no seed, and
            // its -inf elements would fill the buffers); they are survivors of zero mass, noted
            // for the finish
            bal[j] = wave_ballot(v[j] >= cb.tauf && (!MASK || v[j] > -__builtin_inff())) & okm;
            if (MASK) ninf |= wave_ballot(v[j] == -__builtin_inff()) & okm;
            any |= bal[j];
        }
        if (any) cb.append_vec<VEC>(sm, v, bal, okv, i0);
        float s = 0.0f, z = 0.0f, sr = 0.0f;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const bool inc = okv && !(v[j] >= cb.tauf);
            float zj;
            const float t = tp_term(v[j], aw, c, zj);
            const float tt = inc ? t : 0.0f;
            s += tt;
            z = __builtin_fmaf(__builtin_fabsf(zj), tt, z);
            if (want_raw) {
                float z2;
                const float tr = tp_term(v[j], aw, kLog2e, z2);
                sr += inc ? tr : 0.0f;
            }
        }
        acc += (double)s;
        accz += z;
        if (want_raw) accr += (double)sr;
    };
    // keeps the buffer's fill at most kTpSoft every half iteration: the dropped entries join the sum
    auto shrink = [&]() __attribute__((always_inline)) {
        if (cb.cnt > kTpSoft && !cb.ovf) {
            const TpDrop d = topp_compact_entry(wave, cb.cnt, aw, c, want_raw ? 1 : 0);
            acc += d.s;
            accr += d.sr;
            accz += d.z;
            cb.cnt = __builtin_amdgcn_readfirstlane(d.cnt);
            cb.set_tau(__builtin_amdgcn_readfirstlane(d.kth));
        }
    };
    auto examine = [&](float (&buf)[U][VEC], int it) __attribute__((always_inline)) {
        const int t = tid_now();
#pragma unroll
        for (int q = 0; q < U; ++q) {
            if (q == U / 2) shrink();
            const int vi = (it * U + q) * NT + t;
            consume(buf[q], sl.a + vi * VEC, vi < nbody);
        }
    };
    // MASK: each vector's registers take vector q of iteration nxt as soon as vector q is
    // consumed (measured faster for masked launches only: C5 with one masked row 431 -> 425 us;
    // C5 +3 us and capped C5 +5 us with the same change in their streams)
    auto examine_pv = [&](float (&buf)[U][VEC], int it, int nxt, bool run) __attribute__((always_inline)) {
        const int t = tid_now();
#pragma unroll
        for (int q = 0; q < U; ++q) {
            if (run) {
                if (q == U / 2) shrink();
                const int vi = (it * U + q) * NT + t;
                consume(buf[q], sl.a + vi * VEC, vi < nbody);
            }
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(
                lrs, 16u * (uint32_t)(tid_now() + (nxt * U + q) * NT), 0u, 2 /* nt */);
            Elem<T>::from_words((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3], buf[q]);
        }
    };
    if (MASK) {
        for (int it = 0; it < nit && !cb.ovf; it += 2) {
            if (it > 0) xf_iter(A, MA);  // (the first iteration was handled before the seed)
            examine_pv(A, it, it + 2, true);
            load_mask(MA, it + 2);
            shrink();
            const bool run = it + 1 < nit && !cb.ovf;
            if (run) xf_iter(Bq, MB);
            examine_pv(Bq, it + 1, it + 3, run);
            load_mask(MB, it + 3);
            shrink();
        }
    } else {
        for (int it = 0; it < nit && !cb.ovf; it += 2) {
            if (it > 0) xf_iter(A, MA);  // (the first iteration was handled before the seed)
            examine(A, it);
            load_iter(A, it + 2);
            load_mask(MA, it + 2);
            shrink();
            if (it + 1 < nit && !cb.ovf) {
                xf_iter(Bq, MB);
                examine(Bq, it + 1);
            }
            load_iter(Bq, it + 3);
            load_mask(MB, it + 3);
            shrink();
        }
    }
    if (wave == 0 && !cb.ovf) {
        // unaligned head (thread 0) and tail (thread 1), element by element
        float v[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) v[j] = __builtin_nanf("");
        int i0 = 0;
        if (tid <= 1) i0 = sl.load_edge(tid, v);
        const int end = tid == 0 ? sl.a : V;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            if (!(tid <= 1 && i0 + j < end)) {
                v[j] = __builtin_nanf("");  // NaN: neither stored nor summed
            } else if (MASK && !((mrow[(i0 + j) >> 5] >> ((i0 + j) & 31)) & 1u)) {
                v[j] = -__builtin_inff();
            } else if (CAP) {
                v[j] = softcap_out(v[j], a.inv_softcap, a.softcap, a.softcap_f16 != 0);
            }
        }
        consume(v, i0, true);
    }

    // publish the wave's results
    double s = acc, sr = accr;
    float z = accz;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        s += __shfl_xor(s, o, kWave);
        sr += __shfl_xor(sr, o, kWave);
        z += __shfl_xor(z, o, kWave);
    }
    uint32_t kmax = 0u;
    for (int i = lane; i < cb.cnt; i += kWave) {
        const uint32_t kk = key_of(u2f(sm.ck[wave][i]));
        kmax = kk > kmax ? kk : kmax;
    }
    kmax = wave_max_u32(kmax);
    if (lane == 0) {
        sm.wS[wave] = s;
        sm.wSR[wave] = sr;
        sm.wZ[wave] = z;
        sm.wTau[wave] = cb.tau;
        sm.wCnt[wave] = (uint32_t)cb.cnt;
        sm.wMax[wave] = kmax;
        if (wave == 0) sm.anchor = aw;
        if (MASK && ninf) atomicOr(&sm.ninf, 1u);
        const bool finite = (s == s) && s < 1e300 && (z == z) && z < 3e38f && (sr == sr) && sr < 1e300;
        if (!finite) atomicOr(&sm.status, 2u);
    }
}

// Block scan of v: *excl = sum over the threads below this one (ascending order), returns the
// total.  Two barriers; `slot` picks the LDS column (consecutive scans may share it).
__device__ __forceinline__ uint64_t tp_scan(uint64_t v, TopPSmem& sm, int slot, uint64_t* excl) {
    const int lane = lane_id(), w = threadIdx.x >> 6;
    uint64_t s = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint64_t t = __shfl_up(s, o, kWave);
        if (lane >= o) s += t;
    }
    __syncthreads();
    if (lane == kWave - 1) sm.red[w][slot] = s;
    __syncthreads();
    uint64_t below = 0ull, total = 0ull;
#pragma unroll
    for (int i = 0; i < kTpWaves; ++i) {
        const uint64_t x = sm.red[i][slot];
        below += i < w ? x : 0ull;
        total += x;
    }
    *excl = below + (s - v);
    return tp_u64(total);
}

// Sum of the per-wave records sm.red[*][slot] (after a barrier), as a scalar.
__device__ __forceinline__ uint64_t tp_sum16(const TopPSmem& sm, int slot) {
    uint64_t t = 0ull;
#pragma unroll
    for (int i = 0; i < kTpWaves; ++i) t += sm.red[i][slot];
    return tp_u64(t);
}

// Sum over the wave of a double (butterfly).
__device__ __forceinline__ double tp_wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// ---- further passes over the row ------------------------------------------------------

// Penalties of a history row in a further pass: the row's token-state words and parameters.
struct TpPen {
    const uint32_t* wrow;
    float rep, inv_rep, freq, pres;
};

// The aligned body vectors [v0, v1) of row r, and its unaligned head and tail when `edges`
// (every thread calls it): 16-byte buffer loads over just that range (loads past its end read
// zeros and fetch nothing), one vector per thread per step with the next step's load in flight
// (a range is a chunk of a few steps: the second load overlaps the first step's work).  f(v, u, i0, ok) gets the VEC elements of one vector from element i0 on (ok: the
// vector lies in the range; head and tail are NaN-padded) and, with WITH_U, their uniforms
// (dword-aligned 16-byte loads).  PEN: the elements are penalised first from their token-state
// words (streamed like the uniforms), so that f sees processed values.  XF = kXfMask: elements
// outside the row's allowed mask become -inf first (one mask word per vector; the row starts
// 16-byte aligned, so a vector's bits lie in one word); kXfCap: every element is capped first.
template <typename T, bool WITH_U, bool PEN, int XF, typename F>
__device__ __forceinline__ void tp_row_range(const KArgs& a, int r, int v0, int v1, bool edges,
                                             const TpPen& pen, F&& f) {
    constexpr bool MSK = XF == kXfMask, CAP = XF == kXfCap;
    constexpr int NT = kGenThreads;
    constexpr int VEC = Elem<T>::kVec;
    constexpr int UW = WITH_U ? VEC / 4 : 0;  // uniform loads per vector
    constexpr int WW = PEN ? VEC / 4 : 0;     // token-state word loads per vector
    constexpr int UP = 1;                     // vectors per thread per step
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int V = a.V;
    const T* row = reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride;
    const float* urow = WITH_U ? a.u + (size_t)r * a.ustride : nullptr;
    Slice<T> sl;
    sl.init(row, 0, V);
    const int nv = v1 - v0;
    const int nit = (nv + NT * UP - 1) / (NT * UP);
    const int e0 = sl.a + v0 * VEC;  // first element of the range
    const __amdgpu_buffer_rsrc_t lrs = make_rsrc(row + e0, 16u * (uint32_t)nv);
    const __amdgpu_buffer_rsrc_t urs = make_rsrc(WITH_U ? (const void*)(urow + e0) : (const void*)row,
                                                 WITH_U ? 4u * (uint32_t)(nv * VEC) : 0u);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(PEN ? (const void*)(pen.wrow + e0) : (const void*)row,
                                                 PEN ? 4u * (uint32_t)(nv * VEC) : 0u);
    const uint32_t* arow = MSK ? a.allowed + (size_t)r * (size_t)a.astride : nullptr;
    const __amdgpu_buffer_rsrc_t mrs = make_rsrc(MSK ? (const void*)arow : (const void*)row,
                                                 MSK ? 4u * (uint32_t)((V + 31) >> 5) : 0u);
    auto tid_now = [&]() __attribute__((always_inline)) { return wave * kWave + lane_now(); };
    using W4 = decltype(__builtin_amdgcn_raw_buffer_load_b128(lrs, 0u, 0u, 0));
    // a history token's processed value (a zero word: the value itself)
    auto penal = [&](float x, uint32_t wd) __attribute__((always_inline)) {
        wd &= kStateMask;
        return wd ? apply_hashed(x, wd, 0.0f, pen.rep, pen.inv_rep, pen.freq, pen.pres) : x;
    };
    // vectors (it * UP + q) * NT + tid lie past the range for every thread once
    // (it * UP + q) * NT >= nv: such loads and their work are skipped (a uniform test)
    auto load = [&](W4 (&lw)[UP], W4 (&uw)[UP][UW > 0 ? UW : 1], W4 (&ww)[UP][WW > 0 ? WW : 1],
                    uint32_t (&mw)[UP], int it) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < UP; ++q) {
            if ((it * UP + q) * NT >= nv) break;
            const uint32_t vi = (uint32_t)(tid_now() + (it * UP + q) * NT);
            lw[q] = __builtin_amdgcn_raw_buffer_load_b128(lrs, 16u * vi, 0u, 2 /* nt */);
            if (MSK)
                mw[q] = __builtin_amdgcn_raw_buffer_load_b32(
                    mrs, 4u * (((uint32_t)e0 + vi * (uint32_t)VEC) >> 5), 0u, 0);
#pragma unroll
            for (int g = 0; g < UW; ++g)
                uw[q][g] = __builtin_amdgcn_raw_buffer_load_b128(
                    urs, 4u * (vi * (uint32_t)VEC + 4u * (uint32_t)g), 0u, 2);
#pragma unroll
            for (int g = 0; g < WW; ++g)
                ww[q][g] = __builtin_amdgcn_raw_buffer_load_b128(
                    wrs, 4u * (vi * (uint32_t)VEC + 4u * (uint32_t)g), 0u, 2);
        }
    };
    auto consume = [&](W4 (&lw)[UP], W4 (&uw)[UP][UW > 0 ? UW : 1], W4 (&ww)[UP][WW > 0 ? WW : 1],
                       const uint32_t (&mw)[UP], int it) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < UP; ++q) {
            if ((it * UP + q) * NT >= nv) break;
            const int vi = (it * UP + q) * NT + tid_now();
            float v[VEC], u[VEC];
            Elem<T>::from_words((uint32_t)lw[q][0], (uint32_t)lw[q][1], (uint32_t)lw[q][2],
                                (uint32_t)lw[q][3], v);
#pragma unroll
            for (int j = 0; j < VEC; ++j) u[j] = WITH_U ? u2f((uint32_t)uw[q][j / 4][j % 4]) : 0.0f;
            if (MSK) {
                const uint32_t bits = mw[q] >> ((uint32_t)(e0 + vi * VEC) & 31u);
#pragma unroll
                for (int j = 0; j < VEC; ++j) v[j] = ((bits >> j) & 1u) ? v[j] : -__builtin_inff();
            }
            if (CAP) {
#pragma unroll
                for (int j = 0; j < VEC; ++j)
                    v[j] = softcap_out(v[j], a.inv_softcap, a.softcap, a.softcap_f16 != 0);
            }
            if (PEN) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) v[j] = penal(v[j], (uint32_t)ww[q][j / 4][j % 4]);
            }
            f(v, u, e0 + vi * VEC, vi < nv);
        }
    };
    W4 la[UP], lb[UP];
    W4 ua[UP][UW > 0 ? UW : 1], ub[UP][UW > 0 ? UW : 1];
    W4 wa[UP][WW > 0 ? WW : 1], wb[UP][WW > 0 ? WW : 1];
    uint32_t ma[UP] = {}, mb[UP] = {};
    load(la, ua, wa, ma, 0);
    load(lb, ub, wb, mb, 1);
    for (int it = 0; it < nit; it += 2) {
        consume(la, ua, wa, ma, it);
        load(la, ua, wa, ma, it + 2);
        if (it + 1 < nit) consume(lb, ub, wb, mb, it + 1);
        load(lb, ub, wb, mb, it + 3);
    }
    if (edges && wave == 0) {
        float v[VEC], u[VEC];
        int i0 = 0, end = 0;
        if (tid <= 1) {
            i0 = sl.load_edge(tid, v);
            end = tid == 0 ? sl.a : V;
        } else {
#pragma unroll
            for (int j = 0; j < VEC; ++j) v[j] = __builtin_nanf("");
        }
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            u[j] = (WITH_U && i0 + j < end) ? urow[i0 + j] : 0.0f;
            if (MSK && i0 + j < end && !((arow[(i0 + j) >> 5] >> ((i0 + j) & 31)) & 1u))
                v[j] = -__builtin_inff();
            if (CAP && i0 + j < end) v[j] = softcap_out(v[j], a.inv_softcap, a.softcap, a.softcap_f16 != 0);
            if (PEN && i0 + j < end) v[j] = penal(v[j], pen.wrow[i0 + j]);
        }
        f(v, u, i0, tid <= 1);
    }
}

// Smallest key k in [key(-inf), tauk) with P(k), for a predicate that holds from some key on;
// tauk when none does.  One wave searches together: each round the 64 lanes test 64 evenly
// spaced keys of the open range (keys at or above its end count as holding) and the range
// shrinks to the gap below the first key that holds, so the 32-bit range takes six rounds.
// Wave-uniform call; the result is uniform.
template <typename P>
__device__ __forceinline__ uint32_t tp_first_key(uint32_t tauk, P&& pred) {
    const uint32_t lane = (uint32_t)lane_id();
    uint32_t lo = 0x007FFFFFu, hi = tauk > lo ? tauk : lo;
    while (lo < hi) {
        const uint32_t n = hi - lo;                             // < 2^32 - 2^23
        const uint32_t step = n <= (uint32_t)kWave ? 1u : (n + (uint32_t)kWave - 1u) / (uint32_t)kWave;
        const uint32_t p = lo + (lane + 1u) * step - 1u;       // 64 step <= n + 63: no overflow
        const uint64_t b = wave_ballot(p >= hi || pred(p));
        if (b == 0ull) {
            lo = hi;  // every key of the range fails
        } else {
            const uint32_t f = (uint32_t)__builtin_ctzll(b);
            const uint32_t pf = lo + (f + 1u) * step - 1u;
            const uint32_t nlo = f == 0u ? lo : lo + f * step;  // just above the last failing key
            hi = pf < hi ? pf : hi;
            lo = nlo;
        }
        lo = __builtin_amdgcn_readfirstlane(lo);
        hi = __builtin_amdgcn_readfirstlane(hi);
    }
    return lo;
}

// Wide rows (the boundary bucket bstar reaches the values below the candidates): the bucket of a
// value never rises as the value grows (x / T, y - m and the bucket all round monotonically),
// and neither does min-p's test fail, so the survivors top-p keeps, bstar's members and the
// removed ones are key ranges, found by bisection over the whole key range (the candidates top-p
// keeps are kept survivors too): min-p survivors from ksv on, bstar's members from kmem on, kept
// survivors from kkeep on.  The three searches run in waves 0-2; the keys reach every thread
// through LDS (*out, read after the next barrier).
__device__ __forceinline__ void tp_wide_keys(const TpPassDesc& d, uint32_t* out) {
    const int which = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (which >= 3) return;
    const float Tt = d.Tt, m = d.m, lp_min = d.lp_min;
    const int bstar = d.bstar;
    uint32_t k = 0x007FFFFFu;
    if (which > 0 || lp_min > -__builtin_inff()) {
        k = tp_first_key(0xFF800000u, [&](uint32_t x) __attribute__((always_inline)) {
            const float dd = val_of(x) / Tt - m;
            if (which == 0) return dd >= lp_min;
            const int bk = tp_bucket(dd);
            return which == 1 ? bk < bstar : bk <= bstar;
        });
    }
    if (lane_id() == 0) out[which] = k;
}

// A workgroup's share of a pass over row r: the body vectors [v0, v1), and the unaligned head
// and tail when `edges`.
//   * exact pass (rows whose decision the interval leaves open or puts below the candidates,
//     min-p rows with survivors below them): the exact masses of the survivors below the
//     candidates (key below tauk) into their buckets of sm.h.hmass, their total mass and number
//     into acc.sw and acc.n;
//   * wide race (once bstar is known): the race over every survivor top-p keeps (buckets above
//     bstar: the candidates among them too, so the finish races only the boundary members) into
//     acc.rs, bstar's members below the candidates appended to sm.g.key (key(y) << 32 | index,
//     counter sm.bc[4]), the removed survivors below the candidates counted in acc.nrem.  The
//     pass compares keys, and only kept elements compute their race key (from the uniforms
//     streamed with the logits, or generated);
//   * rank pass: the elements at or above the key (the rank of a sampled token that is not a
//     candidate) into acc.n.
// PEN (rows with penalties from the token-state table, exact and wide passes only): the pass
// sees processed values (the rank pass ranks raw ones).
template <typename T, bool PEN, int XF>
__device__ __forceinline__ void tp_pass_range(const KArgs& a, TopPSmem& sm, int r, const TpPassDesc& d,
                                              int v0, int v1, bool edges, TpPassAcc& acc) {
    constexpr int VEC = Elem<T>::kVec;
    const uint32_t tauk = d.key;
    const float Tt = d.Tt, m = d.m, lp_min = d.lp_min;
    TpPen pen{nullptr, 1.0f, 1.0f, 0.0f, 0.0f};
    if (PEN) {
        pen.rep = a.rep ? a.rep[r] : 1.0f;
        pen.pres = a.pres ? a.pres[r] : 0.0f;
        pen.freq = a.freq ? a.freq[r] : 0.0f;
        pen.inv_rep = 1.0f / pen.rep;
        pen.wrow = a.tstate + (size_t)(a.trows ? a.trows[r] : r) * (size_t)a.tstride;
    }
    auto range = [&](auto with_u, auto&& f) __attribute__((always_inline)) {
        tp_row_range<T, decltype(with_u)::value, PEN, XF>(a, r, v0, v1, edges, pen, f);
    };
    if (d.kind == kTpPassExact) {
        range(BoolC<false>{}, [&](const float* v, const float*, int, bool ok)
                                  __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const uint32_t kx = key_of(v[j]);
                const float y = v[j] / Tt;
                const float dd = y - m;
                const bool s = ok && kx != 0u && kx < tauk && key_of(y) != 0u && dd >= lp_min;
                const uint64_t w = s ? mass_of(exp_det(dd)) : 0ull;
                if (w) atomicAdd((unsigned long long*)&sm.h.hmass[tp_bucket(dd)], (unsigned long long)w);
                acc.sw += w;
                acc.n += s ? 1ull : 0ull;
            }
        });
    } else if (d.kind == kTpPassWideRace) {
        const uint32_t ksv = d.ksv, kkeep = d.kkeep, kmem = d.kmem;
        // gen: the uniforms are generated (at the kept elements only) instead of streamed
        const uint64_t gseed = a.u ? 0ull : row_rng_seed(a, r);
        const uint64_t goff = a.u ? 0ull : row_rng_offset(a, r);
        auto body = [&](const float* v, const float* u, int i0, bool ok, bool gen) __attribute__((always_inline)) {
            // generated uniforms: one Philox block per 4 tokens when the vector starts on a
            // block (the body's vectors all do when the row's aligned start does), else token
            // by token
            float ug[VEC];
            const bool blocks = gen && (i0 & 3) == 0;
            bool anykept = false;
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const uint32_t kx = ok ? key_of(v[j]) : 0u;
                anykept = anykept || kx >= kkeep;
            }
            if (blocks && anykept) philox_uniforms_aligned<VEC>(gseed, goff, (uint32_t)i0, ug);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const uint32_t kx = ok ? key_of(v[j]) : 0u;
                if (kx >= kkeep) {
                    const float y = v[j] / Tt;
                    const float dd = y - m;
                    acc.rs.nkept++;
                    const uint64_t lk = ((uint64_t)key_of(y) << 32) | (uint32_t)(i0 + j);
                    acc.rs.last = acc.rs.last > lk ? acc.rs.last : lk;
                    const float uu = !gen ? u[j] : (blocks ? ug[j] : row_uniform(a, r, i0 + j));
                    acc.rs.add_key(exp_det(dd) / (0.0f - log_det(uu)), i0 + j);
                } else if (kx >= tauk) {
                    continue;  // a candidate member of bstar: gathered from the buffers
                } else if (kx >= kmem) {
                    const uint32_t pos = atomicAdd(&sm.bc[4], 1u);
                    if (pos < (uint32_t)kTpGather)
                        sm.g.key[pos] = ((uint64_t)key_of(v[j] / Tt) << 32) | (uint32_t)(i0 + j);
                } else {
                    acc.nrem += kx >= ksv ? 1u : 0u;
                }
            }
        };
        if (a.u) {
            range(BoolC<true>{}, [&](const float* v, const float* u, int i0, bool ok)
                                     __attribute__((always_inline)) { body(v, u, i0, ok, false); });
        } else {
            range(BoolC<false>{}, [&](const float* v, const float* u, int i0, bool ok)
                                      __attribute__((always_inline)) { body(v, u, i0, ok, true); });
        }
    } else {
        tp_row_range<T, false, false, XF>(a, r, v0, v1, edges, pen, [&](const float* v, const float*, int, bool ok)
                                                                   __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < VEC; ++j) acc.n += (ok && key_of(v[j]) >= tauk) ? 1ull : 0ull;
        });
    }
}

// Workgroup totals of acc: thread 0 leaves them in sm.bc64[10..14] (exact pass: mass, number;
// wide race: best, second, kept, removed, last (RowRace fields); rank pass: number), for every
// thread after the next barrier.  Every thread calls it.
__device__ __forceinline__ void tp_pass_reduce(TopPSmem& sm, int kind, TpPassAcc& acc) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    uint64_t x0, x1, x2 = 0ull, x3 = 0ull;
    if (kind == kTpPassWideRace) {
        acc.rs.shfl_merge(32); acc.rs.shfl_merge(16); acc.rs.shfl_merge(8);
        acc.rs.shfl_merge(4); acc.rs.shfl_merge(2); acc.rs.shfl_merge(1);
        x0 = acc.rs.best;
        x1 = ((uint64_t)acc.rs.second << 32) | acc.rs.nkept;
        x2 = wave_sum_u64(acc.nrem);
        x3 = acc.rs.last;
    } else {
        x0 = wave_sum_u64(acc.sw);
        x1 = wave_sum_u64(acc.n);
    }
    __syncthreads();  // the per-wave records' last readers are done
    if (lane == 0) {
        sm.red[w][0] = x0;
        sm.red[w][1] = x1;
        sm.red[w][2] = x2;
        sm.red[w][3] = x3;
    }
    __syncthreads();
    if (tid == 0) {
        if (kind == kTpPassWideRace) {
            RowRace all;
            uint64_t nremt = 0ull;
            for (int i = 0; i < kTpWaves; ++i) {
                RowRace o;
                o.best = sm.red[i][0];
                o.second = (uint32_t)(sm.red[i][1] >> 32);
                o.nkept = (uint32_t)sm.red[i][1];
                o.last = sm.red[i][3];
                all.merge(o);
                nremt += sm.red[i][2];
            }
            sm.bc64[10] = all.best;
            sm.bc64[11] = all.second;
            sm.bc64[12] = all.nkept;
            sm.bc64[13] = nremt;
            sm.bc64[14] = all.last;
        } else {
            uint64_t t0 = 0ull, t1 = 0ull;
            for (int i = 0; i < kTpWaves; ++i) {
                t0 += sm.red[i][0];
                t1 += sm.red[i][1];
            }
            sm.bc64[10] = kind == kTpPassRank ? t1 : t0;
            sm.bc64[11] = t1;
        }
    }
}

// ---- cooperative passes ------------------------------------------------------------------
//
// A row that needs a further pass over V >= kCoopMinChunks chunks takes a free slot of the
// workspace's CoopState, describes the pass there, opens its chunks and works through them
// itself; workgroups that have no row left (or that are between rows) claim chunks too, run
// them, add their totals into the slot (global atomics: bucket masses, sums, gathered members;
// per-chunk race records) and count them done.  The owner waits until every chunk it did not
// run is done, adds the slot's totals to its own and frees the slot.  Every sum is of integers
// (masses, counts) and the race merge is order-independent, so the result does not depend on
// who ran which chunk.
//
// claim: generation (bits 40-63) | chunks of the pass (bits 32-39) | next chunk (bits 0-31).
// One atomic add claims a chunk and tells whether it exists; only the owner changes the
// generation and the chunk count (nothing open: 0 chunks).  The owner describes the pass
// before it opens the chunks, and a claimed chunk keeps the owner waiting, so a helper that
// claimed one reads a stable description.
constexpr int kCoopMinChunks = 4;
constexpr uint32_t kCoopNone = 0xFFFFFFFFu;
constexpr int kCoopHelpPolls = 1 << 16;  // a helper's polls for chunks while rows hold slots
static_assert(kCoopBuckets == kTpBuckets && kCoopGather == kTpGather, "cooperative slot sizes");
static_assert(kTpRankCap * 28 <= kTpGather * 8 && 2 * kTpRankCap <= kGenThreads, "ranked members fit the gather buffer");
static_assert(kCoopMaxChunks < 256, "chunk count field");

__device__ __forceinline__ uint64_t coop_claim_word(uint32_t gen, uint32_t nch) {
    return ((uint64_t)(gen & 0xFFFFFFu) << 40) | ((uint64_t)nch << 32);
}
// the chunk a claim returned, or kCoopNone
__device__ __forceinline__ uint32_t coop_chunk_of(uint64_t x) {
    const uint32_t nch = (uint32_t)(x >> 32) & 0xFFu;
    return (uint32_t)x < nch ? (uint32_t)x : kCoopNone;
}

// The finish's further passes run out of line, so that their registers stay out of the stream
// and the finish; defined next to the LDS they use.  Every thread calls them.
//   topp_pass_entry: one whole pass over row r (cooperative when a slot is free); its scalar
//     results are in sm.bc64[10..13] after a barrier; sets sm.coop_fail when a cooperative
//     pass was not completed (the row then takes the multi-pass path).  PEN: a row with
//     penalties from the token-state table (its range functions are separate, and so are the
//     functions that call them, so that the others keep their registers); XF: the launch's
//     transform of each loaded logit (kXfNone, kXfMask, kXfCap);
//   topp_range_entry<T, PEN, XF>: the pass sm.pd over the body vectors [v0, v1) of row r (and
//     the edges), its workgroup totals into sm.bc64[10..13] as tp_pass_reduce leaves them.
template <typename T, bool PEN, int XF>
__device__ __noinline__ void topp_pass_entry(int kind, int r, uint64_t kernarg, float Tt, float m,
                                             float lp_min, uint32_t key, int bstar);
template <typename T>
__device__ __noinline__ int topp_hist_entry(int r, uint64_t kernarg, uint32_t tauk, float xmaxr);

// Whether a pass of `kind` over row r reads the rows' token-state words (penalties from the
// table, exact and wide passes): such passes run in topp_range_entry<T, true, XF>.
__device__ __forceinline__ bool tp_pass_pen(const KArgs& a, int r, int kind) {
    if (!a.tstate || kind == kTpPassRank) return false;
    const float rp = a.rep ? a.rep[r] : 1.0f;
    const float pr = a.pres ? a.pres[r] : 0.0f;
    const float fr = a.freq ? a.freq[r] : 0.0f;
    return __builtin_amdgcn_readfirstlane((rp == 1.0f && pr == 0.0f && fr == 0.0f) ? 0 : 1) != 0;
}

// History rows, before the stream: the row's bitmap of history tokens into LDS (sm.hb, kept
// through the stream), and the seed's fill target less the history tokens' share of the
// slots (the finish adds every history token the stream does not buffer).  Uniform result.
__device__ __forceinline__ float topp_hist_begin(const KArgs& a, TopPSmem& sm, const RowP& prm) {
    constexpr int NT = kGenThreads;
    const int tid = threadIdx.x;
    const int V = a.V;
    const int nhw = (V + 31) >> 5;
    const uint32_t* brow = a.tbits + (size_t)prm.trow * (size_t)a.tbstride;
    uint32_t n = 0u;
    for (int i = tid; i < nhw; i += NT) {
        uint32_t b = brow[i];
        if (i == nhw - 1 && (V & 31)) b &= (1u << (V & 31)) - 1u;  // no token past V
        sm.hb[i] = b;
        n += (uint32_t)__popc(b);
    }
    n = (uint32_t)wave_sum_u64(n);
    if (tid == 0) sm.bc[0] = 0u;
    __syncthreads();
    if ((tid & 63) == 0) atomicAdd(&sm.bc[0], n);
    __syncthreads();
    const float nh = (float)tp_u(sm.bc[0]);
    __syncthreads();  // bc is the stream's from here on
    return __builtin_fmaxf(kTpFill * (float)kTpCapW - 1.1f * nh / (float)kTpWaves, (float)kWave);
}

// History rows (penalties from the token-state table with its bitmap), after the stream (the
// bitmap is in LDS: topp_hist_begin): the buffered history tokens are marked (bit 18 of the index word is
// free: V <= kTpHistMaxV) and take their processed values from their token-state words, in
// place; the others, which the stream summed, join the buffers with their processed values and
// their terms come out of the sums (wSub, wSRsub).  With raw logprobs, the history tokens' raw
// normaliser terms are added up (wS0h) and those at or above the threshold by raw value are
// listed (rl_*: the raw top-L and rank need them).  Leaves the waves' largest processed keys in
// wMaxP.  Returns 0, or the reason the row takes the multi-pass path (uniform).
template <typename T>
__device__ __forceinline__ int topp_hist_prepare(const KArgs& a, TopPSmem& sm, int r, const RowP& prm,
                                                 uint32_t tauk, float xmaxr) {
    constexpr int NT = kGenThreads;
    constexpr int G = 16;  // buffered entries per lane whose words are gathered together
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int L = a.L;
    const bool greedy = prm.greedy;
    const int V = a.V;
    const uint32_t* trw = a.tstate + (size_t)prm.trow * (size_t)a.tstride;
    // the row's allowed-token words (a masked history token's raw value is -inf), or null
    const uint32_t* arow = a.allowed ? a.allowed + (size_t)r * (size_t)a.astride : nullptr;
    // a history token: its processed value, and with raw logprobs its raw normaliser term and
    // (at or above the threshold by raw value) its listing
    float s0h = 0.0f;
    uint32_t mx = 0u;
    auto history = [&](float x, uint32_t wd, uint32_t t) __attribute__((always_inline)) {
        const float y = apply_hashed(x, wd & kStateMask, 0.0f, prm.rep, prm.inv_rep, prm.freq, prm.pres);
        if (L >= 0) {
            s0h += exp_det(x - xmaxr);
            const uint32_t kx = key_of(x);
            // NaN (key 0) sorts after every value: never listed, also when a short row keeps
            // every element (threshold key 0); a row with fewer than L other candidates falls
            // back to the multi-pass path, which lists its NaN elements last
            if (kx >= tauk && kx != 0u) {
                const uint32_t pos = atomicAdd(&sm.rl_n, 1u);
                if (pos < (uint32_t)kTpRawCap) {
                    sm.rl_key[pos] = kx;
                    sm.rl_idx[pos] = (int32_t)t;
                }
            }
        }
        return y;
    };
    // (the row's bitmap of history tokens was staged in LDS before the stream)
    const int nhw = (V + 31) >> 5;
    if (tid == 0) {
        sm.rl_n = 0u;
        sm.hl_n = 0u;
    }
    __syncthreads();
    // the buffered history tokens: marked, their bits cleared, their words gathered (G entries
    // per lane at a time) and their processed values written in place
    const int cnt0 = (int)tp_u(sm.wCnt[wave]);
    for (int base = 0; base < cnt0; base += G * kWave) {
        uint32_t cw[G], wd[G];
        bool h[G];
#pragma unroll
        for (int q = 0; q < G; ++q) {
            const int i = base + q * kWave + lane;
            cw[q] = i < cnt0 ? (uint32_t)sm.ci[wave][i] : 0u;
            const uint32_t bit = 1u << (cw[q] & 31u);
            h[q] = i < cnt0 && (sm.hb[(cw[q] & kTpIdxMask) >> 5] & bit) != 0u;
            if (h[q]) atomicAnd(&sm.hb[(cw[q] & kTpIdxMask) >> 5], ~bit);
        }
#pragma unroll
        for (int q = 0; q < G; ++q) wd[q] = h[q] ? trw[cw[q] & kTpIdxMask] : 0u;
#pragma unroll
        for (int q = 0; q < G; ++q) {
            const int i = base + q * kWave + lane;
            if (i >= cnt0) continue;
            float y = u2f(sm.ck[wave][i]);
            if (h[q]) {
                y = history(y, wd[q], cw[q] & kTpIdxMask);
                sm.ck[wave][i] = f2u(y);
                sm.ci[wave][i] = (int32_t)(cw[q] | kTpHist);
            }
            const uint32_t ky = key_of(y);
            mx = ky > mx ? ky : mx;
        }
    }
    __syncthreads();
    // the others were summed by the stream: listed (a chunk of NT bitmap words at a time) and,
    // once the list holds half its capacity or the bitmap is done, their logits and words
    // gathered together; their exact terms (of the approximate sum and of the raw one, as the
    // stream computed them) come out of the sums, and they join the buffers with their processed
    // values, consecutive entries in different waves
    const T* lrow = reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride;
    const float cz = greedy ? kLog2e : kLog2e / prm.T;
    const bool want_raw = L >= 0 && !greedy && prm.T != 1.0f;
    const float aws = tp_uf(sm.anchor);
    constexpr uint32_t kCap = 2u * (uint32_t)kTpGather;
    double sub = 0.0, subr = 0.0;
    int cntw = cnt0;
    for (int w0 = 0; w0 < nhw; w0 += NT) {
        if (w0 + tid < nhw) {
            uint32_t b = sm.hb[w0 + tid];
            while (b) {
                const uint32_t j = (uint32_t)__builtin_ctz(b);
                b &= b - 1u;
                const uint32_t pos = atomicAdd(&sm.hl_n, 1u);
                if (pos < kCap) sm.hl[pos] = (uint32_t)(w0 + tid) * 32u + j;
            }
        }
        __syncthreads();
        const uint32_t nl = tp_u(sm.hl_n);
        if (nl > kCap) return VWS_FALLBACK_OVERFLOW;
        if (nl < kCap / 2 && w0 + NT < nhw) continue;  // (uniform)
        for (uint32_t base = 0; base < nl; base += NT) {
            const uint32_t j = base + (uint32_t)(lane * kTpWaves + wave);
            const bool in = j < nl;
            const uint32_t t = in ? sm.hl[j] : 0u;
            float x = in ? Elem<T>::load1(lrow + t) : 0.0f;
            if (in && arow && !((arow[t >> 5] >> (t & 31)) & 1u)) x = -__builtin_inff();  // masked
            if (in && a.softcap > 0.0f) x = softcap_out(x, a.inv_softcap, a.softcap, a.softcap_f16 != 0);
            const uint32_t wd = in ? trw[t] : 0u;
            float y = 0.0f;
            if (in) {
                float z;
                sub += (double)tp_term(x, aws, cz, z);
                if (want_raw) subr += (double)tp_term(x, aws, kLog2e, z);
                y = history(x, wd, t);
                const uint32_t ky = key_of(y);
                mx = ky > mx ? ky : mx;
            }
            const uint64_t bal = wave_ballot(in);
            const int pos = cntw + lane_prefix(bal);
            if (in && pos < kTpCapW) {
                sm.ck[wave][pos] = f2u(y);
                sm.ci[wave][pos] = (int32_t)(t | kTpHist);
            }
            cntw += __popcll(bal);
        }
        __syncthreads();  // the list's last readers are done
        if (tid == 0) sm.hl_n = 0u;
        __syncthreads();
    }
    sub = tp_wave_sum_f64(sub);
    subr = tp_wave_sum_f64(subr);
    mx = wave_max_u32(mx);
    s0h = (float)tp_wave_sum_f64((double)s0h);
    if (lane == 0) {
        sm.wSub[wave] = sub;
        sm.wSRsub[wave] = subr;
        sm.wMaxP[wave] = mx;
        sm.wS0h[wave] = s0h;
        sm.wCnt[wave] = (uint32_t)(cntw < kTpCapW ? cntw : kTpCapW);
        if (cntw > kTpCapW) atomicOr(&sm.status, 1u);
    }
    __syncthreads();
    if (sm.status != 0u) return VWS_FALLBACK_OVERFLOW;
    if (tp_u(sm.rl_n) > (uint32_t)kTpRawCap) return VWS_FALLBACK_TOPL;
    return 0;
}

// Completes a row after topp_stream.  Returns 0, or (nothing written) the reason the row must
// take the multi-pass path (VWS_FALLBACK_*).  Every return decision is uniform over the
// workgroup: values that decide are read from LDS after a barrier, or are scalars.
template <typename T, int XF>
__device__ __forceinline__ int topp_finish(const KArgs& a, TopPSmem& sm, int r, const RowP& prm,
                                           uint64_t kernarg) {
    constexpr bool MASK = XF == kXfMask;
    constexpr int NT = kGenThreads;
    constexpr int VEC = Elem<T>::kVec;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int L = a.L;
    const bool greedy = prm.greedy;
    const float Tt = tp_uf(greedy ? 1.0f : prm.T);
    if (tid == 0) {
        sm.coop_hold = 0u;  // read by thread 0 once the row is done
        sm.coop_fail = 0u;
    }
    __syncthreads();  // every wave's stream results are published
    VWS_TRACE_MARK(a, VWS_TRACE_STREAM);
    if (sm.status != 0u) return (sm.status & 1u) ? VWS_FALLBACK_OVERFLOW : VWS_FALLBACK_SUM;
    const bool hist = prm.has_hist;
    // an entry's element index (history rows mark their history tokens in bit 18)
    const uint32_t imask = hist ? kTpHist - 1u : kTpIdxMask;
    uint32_t tauk = 0u, maxr = 0u;
#pragma unroll
    for (int w = 0; w < kTpWaves; ++w) {
        tauk = sm.wTau[w] > tauk ? sm.wTau[w] : tauk;
        maxr = sm.wMax[w] > maxr ? sm.wMax[w] : maxr;
    }
    tauk = tp_u(tauk);
    maxr = tp_u(maxr);
    // a finite row maximum (always a candidate: no threshold exceeds a wave's own maximum)
    if (maxr <= 0x007FFFFFu || maxr >= 0xFF800000u) return VWS_FALLBACK_DEGENERATE;
    const float xmaxr = val_of(maxr);  // raw maximum (the raw logprobs)
    uint32_t maxk = maxr;
    if (hist) {
        // every history token into the buffers with its processed value (out of line)
        if (const int why = topp_hist_entry<T>(r, kernarg, tauk, xmaxr)) return why;
        VWS_TRACE_MARK(a, VWS_TRACE_TP_HIST);
        maxk = 0u;
#pragma unroll
        for (int w = 0; w < kTpWaves; ++w) maxk = sm.wMaxP[w] > maxk ? sm.wMaxP[w] : maxk;
        maxk = tp_u(maxk);
    }
    // the processed maximum: finite, and in history rows at or above every threshold (nothing
    // outside the buffers, whose values are raw, can then exceed it)
    if (maxk <= 0x007FFFFFu || maxk >= 0xFF800000u || maxk < tauk) return VWS_FALLBACK_DEGENERATE;
    const float xmax = val_of(maxk);   // processed maximum (top-p)
    const float m = greedy ? xmax : xmax / Tt;  // max y (the division is monotone)
    if (!(m > -__builtin_inff() && m < __builtin_inff())) return VWS_FALLBACK_DEGENERATE;
    const float lp_min = (!greedy && prm.min_p > 0.0f)
                             ? tp_uf(log_det(prm.min_p < 1.0f ? prm.min_p : 1.0f)) : -__builtin_inff();
    const float aw = tp_uf(sm.anchor);
    // a cooperative pass that was not completed marks sm.coop_fail; the row is handed over right
    // after it, before anything is written
    auto pass = [&](int kind, uint32_t key, int bs) __attribute__((always_inline)) {
        if (hist) topp_pass_entry<T, true, XF>(kind, r, kernarg, Tt, m, lp_min, key, bs);
        else topp_pass_entry<T, false, XF>(kind, r, kernarg, Tt, m, lp_min, key, bs);
        __syncthreads();
    };
    for (int i = tid; i < kTpBuckets; i += NT) {
        sm.h.hmass[i] = 0ull;
        sm.h.hcnt[i] = 0u;
    }
    if (tid == 0) {
        sm.bc[7] = 0u;  // top-L members gathered
        sm.xr = xmaxr;
    }
    __syncthreads();

    // exact masses of the buffered entries (now turned into order keys): candidates into the
    // buckets, the others into Sx
    const int cnt = (int)tp_u(sm.wCnt[wave]);
    // history rows: the marked entries hold processed values; their raw parts (normaliser terms,
    // raw entries at or above the threshold) come from the pre-pass
    {
        const float mr = (greedy || Tt == 1.0f) ? xmaxr : xmaxr / Tt;  // history rows: raw buckets
        const bool same_max = maxk == maxr;  // x - max x is then what the rows without a history use
        uint64_t wc = 0ull, sx = 0ull;
        uint32_t nxs = 0u;
        float s0b = 0.0f;
        // unit: y = x (greedy rows and T = 1, where x / T is x itself): the loop without the
        // division, chosen once for the wave; hc: a history row (a separate loop, so that rows
        // without one compute nothing of it)
        auto masses = [&](auto unit, auto hc) __attribute__((always_inline)) {
            constexpr bool H = decltype(hc)::value;
            for (int i = lane; i < cnt; i += kWave) {
                const uint32_t c0 = (uint32_t)sm.ci[wave][i];
                const bool hm = H && (c0 & kTpHist);  // a history token (processed value)
                const float x = u2f(sm.ck[wave][i]);
                const uint32_t kk = key_of(x);
                const float y = decltype(unit)::value ? x : x / Tt;
                const float d = y - m;
                const bool surv = !greedy && key_of(y) != 0u && d >= lp_min;
                const float e = exp_det(d);
                const uint64_t w = surv ? mass_of(e) : 0ull;
                // raw logprobs' normaliser: x - max x is d itself for greedy rows and T = 1
                // (without a history)
                if (L >= 0 && !hm) s0b += (H && !same_max) ? exp_det(x - xmaxr) : (decltype(unit)::value ? e : exp_det(x - xmax));
                const int b = tp_bucket(d);
                const bool below = kk < tauk;
                sm.ck[wave][i] = kk;
                sm.ci[wave][i] = (int32_t)((c0 & kTpIdxMask) | ((uint32_t)b << 19) |
                                           (surv ? kTpSurv : 0u) | (below ? kTpBelow : 0u));
                if (!below) {
                    if (L > 0 && !H) atomicAdd(&sm.h.hcnt[b], 1u);  // counts for the top-L logprobs
                    if (w) atomicAdd((unsigned long long*)&sm.h.hmass[b], (unsigned long long)w);
                    wc += w;
                } else {
                    sx += w;
                    nxs += surv ? 1u : 0u;
                }
                // history rows: the top-L counts by raw bucket
                if (H && L > 0 && !hm && kk >= tauk) atomicAdd(&sm.h.hcnt[tp_bucket(y - mr)], 1u);
            }
        };
        if (hist) {
            if (greedy || Tt == 1.0f) masses(BoolC<true>{}, BoolC<true>{});
            else masses(BoolC<false>{}, BoolC<true>{});
        } else {
            if (greedy || Tt == 1.0f) masses(BoolC<true>{}, BoolC<false>{});
            else masses(BoolC<false>{}, BoolC<false>{});
        }
        if (hist && L > 0) {
            // the listed raw entries in the top-L counts
            const uint32_t nrl = tp_u(sm.rl_n);
            for (uint32_t j = (uint32_t)tid; j < nrl; j += NT) {
                const float xr = val_of(sm.rl_key[j]);
                atomicAdd(&sm.h.hcnt[tp_bucket(((greedy || Tt == 1.0f) ? xr : xr / Tt) - mr)], 1u);
            }
        }
        wc = wave_sum_u64(wc);
        sx = wave_sum_u64(sx);
        const uint64_t nn = wave_sum_u64(nxs);
        double sb = tp_wave_sum_f64((double)s0b);
        if (hist && L >= 0) sb += (double)sm.wS0h[wave];
        if (lane == 0) {
            sm.red[wave][0] = wc;
            sm.red[wave][1] = sx;
            sm.red[wave][2] = nn;
            sm.redd[wave] = sb;
        }
    }
    __syncthreads();
    if (tid == 0) {
        // candidates' mass (wide rows: every survivor's), survivors below the threshold, the
        // buffered raw normaliser: read from LDS after the next barrier
        uint64_t wc = 0ull, nx = 0ull;
        double sb = 0.0;
#pragma unroll
        for (int w = 0; w < kTpWaves; ++w) {
            wc += sm.red[w][0];
            nx += sm.red[w][2];
            sb += sm.redd[w];
        }
        sm.tot_wc = wc;
        sm.tot_nxs = nx;
        sm.tot_s0b = sb;
    }

    int32_t token = 0;
    uint32_t flags = VWS_FLAG_STREAM_TOPP;
    int32_t nkept = 1;
    if (greedy) {
        // the lowest index at the maximum
        uint64_t best = 0ull;
        for (int i = lane; i < cnt; i += kWave) {
            if (sm.ck[wave][i] == maxk) {
                const uint64_t pk = ((uint64_t)maxk << 32) |
                                    (0x7FFFFFFFu - ((uint32_t)sm.ci[wave][i] & imask));
                best = pk > best ? pk : best;
            }
        }
        best = wave_max_u64(best);
        __syncthreads();
        if (lane == 0) sm.red[wave][3] = best;
        __syncthreads();
        best = 0ull;
#pragma unroll
        for (int w = 0; w < kTpWaves; ++w) best = sm.red[w][3] > best ? sm.red[w][3] : best;
        token = (int32_t)(0x7FFFFFFFu - tp_u((uint32_t)best));
        flags |= VWS_FLAG_GREEDY;
    } else {
        VWS_TRACE_MARK(a, VWS_TRACE_TP_MASS);
        // ---- wave 0: the interval of the exact mass below the candidates (the anchor's
        // scale, then the error bound of the terms), and whether survivors lie below them
        const float q32 = 1.0f - prm.top_p;  // in (0, 1)
        if (wave == 0) {
            const double tt = (double)Tt, md = (double)m;
            const double ln2 = 0.6931471805599453;
            const double ad = (double)aw;
            const double mw = 0x1p44 * exp(ad / tt - md);
            // relative error of a term against its exact mass: exp_det (1 ulp), the hardware
            // exp2 (assumed 4 ulp), the vector partial sum (VEC - 1 roundings), the rounding of
            // d = fl(y - max) and, for T != 1, of y = fl(x / T) (|d|, |y| <= |z| ln2 +
            // |a/T - m|, |a/T|), and the argument (x - a) * c (three roundings of |z|, plus c's
            // own)
            const double k0 = 0x1p-23 + 0x1p-21 + (double)(VEC - 1) * 0x1p-24 +
                              fabs(ad / tt - md) * 0x1p-24 +
                              (Tt != 1.0f ? fabs(ad / tt) * 0x1p-24 : 0.0) + 0x1p-40;
            const double k1 = ((Tt != 1.0f ? 2.0 : 1.0) + 4.0) * ln2 * 0x1p-24;
            const double ws = lane < kTpWaves ? sm.wS[lane] : 0.0;
            const double wz = lane < kTpWaves ? (double)sm.wZ[lane] : 0.0;
            // history rows: the terms of the tokens added to the buffers after the stream come
            // out of the centre (the error bound stays that of the stream's sum)
            const double wsub = (hist && lane < kTpWaves) ? sm.wSub[lane] : 0.0;
            const double sap = tp_wave_sum_f64(mw * (ws - wsub));
            const double err0 = tp_wave_sum_f64(mw * (k0 * ws + k1 * wz * (1.0 + 0x1p-8)));
            if (lane == 0) {
                uint64_t Sx = 0ull;  // exact mass of the survivors buffered below the threshold
#pragma unroll
                for (int w = 0; w < kTpWaves; ++w) Sx += sm.red[w][1];
                int why = 0;
                // every element of the row outside the buffers may be a term (the floor of each
                // exact mass loses less than one unit)
                const double nterms = (double)a.V;
                const double err = err0 * 1.01 + 2.0;
                uint64_t nlo = 0ull, nhi = 0ull;
                if (!(sap < 1e30 && err < 1e30)) why = VWS_FALLBACK_SUM;
                sm.bc[10] = 0u;
                if (lp_min > -__builtin_inff()) {
                    // min-p: the sum is exact (zero) only when no element below the candidates
                    // survives it (the largest of them is the float just below the threshold);
                    // otherwise the wide pass sums the survivors below the candidates exactly
                    if (tauk > 0x00800000u && val_of(tauk - 1u) / Tt - m >= lp_min) sm.bc[10] = 1u;
                    sm.bc[9] = 0u;
                } else {
                    const double lo = floor(sap - err) - nterms;
                    nlo = lo > 0.0 ? (uint64_t)lo : 0ull;
                    nhi = (uint64_t)ceil(sap + err);
                    // elements below the candidates survive (masked rows: the -inf elements
                    // outside the buffers are survivors of zero mass)
                    sm.bc[9] = (tauk > 0x007FFFFFu || (MASK && sm.ninf != 0u)) ? 1u : 0u;
                }
                sm.bc[8] = (uint32_t)why;
                sm.bc64[0] = nlo + Sx;
                sm.bc64[1] = nhi + Sx;
            }
        }
        __syncthreads();
        if (const int why = (int)tp_u(sm.bc[8])) return why;
        // survivors below every candidate: the stream's terms (all survive without min-p) and
        // the buffered ones below the threshold
        bool any_below_nc = tp_u(sm.bc[9]) != 0u || tp_u64(sm.tot_nxs) > 0ull;
        uint64_t S[2] = {tp_u64(sm.bc64[0]), tp_u64(sm.bc64[1])};

        // decides top-p for S[0] and S[1]; when they differ, or when the boundary lies below
        // the candidates, the exact pass puts every survivor's exact mass into the buckets (S is
        // 0 from then on) and the decision is taken once more.  A boundary bucket at or below
        // the largest value under the candidates makes the row wide: one more pass races the
        // kept survivors below the candidates and gathers the boundary bucket's members there.
        int bstar = -1, gathered = -1;
        uint32_t ng = 0u, cpos = 0u, tflags = 0u;
        bool ranked = false, serial = false;
        bool exact = false, wide = false, go_exact = tp_u(sm.bc[10]) != 0u;
        int bnc = kTpBuckets;       // bucket of the largest value below the candidates
        if (tid == 0) {
            // the wide race pass's survivors (wide rows: every one outside the boundary bucket)
            // and their race: none until that pass runs
            sm.wrace[0] = sm.wrace[1] = sm.wrace[2] = sm.wrace[3] = 0ull;
        }
        for (;;) {
            if (go_exact && !exact) {
                pass(kTpPassExact, tauk, 0);
                if (tp_u(sm.coop_fail)) return VWS_FALLBACK_COOP;
                if (tid == 0) sm.tot_wc += sm.bc64[10];
                __syncthreads();
                any_below_nc = tp_u64(sm.bc64[11]) > 0ull;
                S[0] = S[1] = 0ull;
                exact = true;
                if (tauk > 0x007FFFFFu) bnc = tp_bucket(val_of(tauk - 1u) / Tt - m);
                flags |= VWS_FLAG_TOPP_RECOUNT;
            }
            uint64_t thr[2], W[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                W[e] = S[e] + tp_u64(sm.tot_wc);
                thr[e] = scale_floor(q32, W[e]);
            }
            bool decided = false;
            if (S[0] > thr[0] && S[1] > thr[1]) {  // the boundary lies below the candidates
                go_exact = true;
                continue;
            }
            if (S[0] <= thr[0] && S[1] <= thr[1]) {
                // ---- boundary bucket: the last b (from the top) with S + suffix(b) > thr
                if (tid == 0) {
                    sm.bc[0] = 0xFFFFFFFFu;
                    sm.bc[1] = 0xFFFFFFFFu;
                }
                {
                    const int b0 = 2 * tid, b1 = 2 * tid + 1;
                    const uint64_t m0 = sm.h.hmass[b0], m1 = sm.h.hmass[b1];
                    uint64_t below_me;                                        // buckets < b0
                    const uint64_t tot = tp_scan(m0 + m1, sm, 0, &below_me);  // (barriers)
                    const uint64_t suf0 = tot - below_me;                     // buckets >= b0
                    const uint64_t suf1 = suf0 - m0;                          // buckets >= b1
                    const uint64_t suf2 = suf1 - m1;                          // buckets > b1
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        if (S[e] + suf1 > thr[e] && S[e] + suf2 <= thr[e]) { sm.bc[e] = (uint32_t)b1; sm.bc64[2 + e] = suf2; }
                        if (S[e] + suf0 > thr[e] && S[e] + suf1 <= thr[e]) { sm.bc[e] = (uint32_t)b0; sm.bc64[2 + e] = suf1; }
                    }
                }
                __syncthreads();
                const int b0s = (int)tp_u(sm.bc[0]);
                if (b0s >= kTpBuckets - 1) return VWS_FALLBACK_GATHER;  // not found, or the zero-mass bucket
                if (b0s == (int)tp_u(sm.bc[1])) {
                    bstar = b0s;
                    const uint64_t below = tp_u64(sm.bc64[2]);  // mass of the candidates in buckets > bstar
                    // ---- the boundary bucket's members
                    if (gathered != bstar) {
                        gathered = bstar;
                        wide = exact && bstar >= bnc;
                        __syncthreads();
                        if (tid == 0) sm.bc[4] = 0u;
                        __syncthreads();
                        for (int i = lane; i < cnt; i += kWave) {
                            const uint32_t c = (uint32_t)sm.ci[wave][i];
                            if (!tp_code_cand(c) || tp_code_bucket(c) != bstar) continue;
                            const float y = val_of(sm.ck[wave][i]) / Tt;
                            const uint32_t pos = atomicAdd(&sm.bc[4], 1u);
                            if (pos < (uint32_t)kTpGather)
                                sm.g.key[pos] = ((uint64_t)key_of(y) << 32) | (c & imask);
                        }
                        if (wide) {
                            pass(kTpPassWideRace, tauk, bstar);
                            if (tp_u(sm.coop_fail)) return VWS_FALLBACK_COOP;
                            if (tid == 0) {
                                sm.wrace[0] = sm.bc64[10];
                                sm.wrace[1] = sm.bc64[11];
                                sm.wrace[2] = sm.bc64[12];
                                sm.wrace[3] = sm.bc64[14];
                            }
                            any_below_nc = tp_u64(sm.bc64[13]) > 0ull;
                            flags |= VWS_FLAG_TOPP_WIDE;
                        }
                        __syncthreads();
                        ng = tp_u(sm.bc[4]);
                        if (ng == 0u || ng > (uint32_t)kTpGather) return VWS_FALLBACK_GATHER;
                        ranked = ng <= (uint32_t)kTpRankCap;
                        serial = ng <= (uint32_t)kTpRankSerial;
                        if (serial) {
                            // members in any order, with their exact masses
                            if (tid < (int)ng)
                                sm.rk.w[tid] = mass_of(exp_det(val_of((uint32_t)(sm.rk.key[tid] >> 32)) - m));
                        } else if (ranked) {
                            topp_rank_members_entry(ng, m);  // out of line: rare, and large
                        } else {
                            uint32_t P = 1u;
                            while (P < ng) P <<= 1;
                            for (uint32_t i = ng + tid; i < P; i += NT) sm.g.key[i] = ~0ull;
                            __syncthreads();
                            for (uint32_t size = 2; size <= P; size <<= 1) {
                                for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                                    for (uint32_t t = tid; t < P / 2; t += NT) {
                                        const uint32_t i = 2 * t - (t & (stride - 1));
                                        const uint32_t j = i + stride;
                                        const bool up = (i & size) == 0;
                                        const uint64_t x = sm.g.key[i], z = sm.g.key[j];
                                        if ((x > z) == up) { sm.g.key[i] = z; sm.g.key[j] = x; }
                                    }
                                    __syncthreads();
                                }
                            }
                        }
                        __syncthreads();
                    }
                    // ---- the cut: the first member (ascending) whose cumulative mass exceeds
                    // thr, at both ends of the interval
                    if (tid == 0) {
                        sm.bc[5] = 0xFFFFFFFFu;
                        sm.bc[6] = 0xFFFFFFFFu;
                    }
                    __syncthreads();
                    if (ranked) {
                        // a member's cumulative mass counts the members at or below it
                        if (tid < (int)ng) {
                            const uint64_t wj = sm.rk.w[tid];
                            uint64_t cj = 0ull;
                            uint32_t rankj = 0u;
                            if (serial) {
                                const uint64_t gj = sm.rk.key[tid];
                                for (uint32_t i = 0; i < ng; ++i) {
                                    const bool le = sm.rk.key[i] <= gj;
                                    cj += le ? sm.rk.w[i] : 0ull;
                                    rankj += le ? 1u : 0u;
                                }
                            } else {
                                cj = sm.rk.cum[tid];
                                rankj = sm.rk.rnk[tid];
                            }
#pragma unroll
                            for (int e = 0; e < 2; ++e) {
                                const uint64_t base = S[e] + below;
                                if (base + cj > thr[e] && base + cj - wj <= thr[e]) {
                                    sm.bc[5 + e] = rankj - 1u;
                                    sm.bc64[4 + 2 * e] = base + cj - wj;
                                    sm.bc64[5 + 2 * e] = base + cj;
                                }
                            }
                        }
                    } else {
                        const uint32_t j0 = 2 * tid, j1 = 2 * tid + 1;
                        const uint64_t w0 = j0 < ng ? mass_of(exp_det(val_of((uint32_t)(sm.g.key[j0] >> 32)) - m)) : 0ull;
                        const uint64_t w1 = j1 < ng ? mass_of(exp_det(val_of((uint32_t)(sm.g.key[j1] >> 32)) - m)) : 0ull;
                        uint64_t pre;
                        tp_scan(w0 + w1, sm, 1, &pre);
#pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const uint64_t base = S[e] + below;
                            if (j0 < ng && base + pre + w0 > thr[e] && base + pre <= thr[e]) {
                                sm.bc[5 + e] = j0;
                                sm.bc64[4 + 2 * e] = base + pre;
                                sm.bc64[5 + 2 * e] = base + pre + w0;
                            }
                            if (j1 < ng && base + pre + w0 + w1 > thr[e] && base + pre + w0 <= thr[e]) {
                                sm.bc[5 + e] = j1;
                                sm.bc64[4 + 2 * e] = base + pre + w0;
                                sm.bc64[5 + 2 * e] = base + pre + w0 + w1;
                            }
                        }
                    }
                    __syncthreads();
                    cpos = tp_u(sm.bc[5]);
                    if (cpos < ng && cpos == tp_u(sm.bc[6])) {
                        // the two terms of the near-tie test (tol = 1e-6 W) must agree too
                        uint32_t t1[2], t2[2];
#pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const uint64_t cprev = tp_u64(sm.bc64[4 + 2 * e]);
                            const uint64_t cat = tp_u64(sm.bc64[5 + 2 * e]);
                            const uint64_t tol = (uint64_t)((double)W[e] * 1e-6);
                            t1[e] = (thr[e] - cprev <= tol) ? 1u : 0u;
                            t2[e] = (cat > thr[e] && cat - thr[e] <= tol) ? 2u : 0u;
                        }
                        if (t1[0] == t1[1] && t2[0] == t2[1]) {
                            tflags = t1[0] | t2[0];
                            decided = true;
                        }
                    }
                }
            }
            if (decided) break;
            if (exact) return VWS_FALLBACK_AMBIGUOUS;
            go_exact = true;  // ambiguous: once more on the exact masses
        }

        VWS_TRACE_MARK(a, VWS_TRACE_TP_CUT);
        // ---- race over the kept survivors: candidates above the boundary bucket, and the
        // boundary bucket's members from the cut on
        RowRace rs;
        uint32_t below_cands = 0u;  // surviving candidates in buckets below the boundary
        // the boundary bucket's kept members, at most two per thread (ng <= kTpGather = 2 NT),
        // with their uniforms loaded first: that latency overlaps the candidates' race below
        static_assert(kTpGather <= 2 * NT, "two boundary members per thread");
        bool mk[2];
        uint64_t mg[2];
        float mu[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t j = (uint32_t)tid + (uint32_t)(h * NT);
            mk[h] = false;
            mg[h] = 0ull;
            if (j < ng) {
                const uint64_t g = sm.g.key[j];
                if (ranked) {
                    // kept: at or after the cut in ascending order
                    uint32_t rankj = 0u;
                    if (serial) {
                        for (uint32_t i = 0; i < ng; ++i) rankj += sm.rk.key[i] <= g ? 1u : 0u;
                    } else {
                        rankj = sm.rk.rnk[j];
                    }
                    mk[h] = !(rankj - 1u < cpos);
                } else {
                    mk[h] = j >= cpos;
                }
                mg[h] = g;
            }
            mu[h] = mk[h] ? row_uniform(a, r, (int32_t)(uint32_t)mg[h]) : 0.5f;
        }
        // four entries per lane at a time, their uniforms loaded together: a lane waits for one
        // memory latency per four entries, not per kept entry
        constexpr int kRq = 4;
        // (wide rows: the pass raced the kept candidates too, and no candidate lies in a bucket
        // below the boundary one)
        for (int i0 = lane; i0 < (wide ? 0 : cnt); i0 += kRq * kWave) {
            float dq[kRq], uq[kRq];
            uint32_t yq[kRq];
            int32_t iq[kRq];
            bool kq[kRq];
#pragma unroll
            for (int q = 0; q < kRq; ++q) {
                const int i = i0 + q * kWave;
                const uint32_t c = i < cnt ? (uint32_t)sm.ci[wave][i] : kTpBelow;
                const bool sv = tp_code_cand(c);
                const int b = tp_code_bucket(c);
                below_cands += (sv && b > bstar) ? 1u : 0u;
                kq[q] = sv && b < bstar;
                iq[q] = (int32_t)(c & imask);
            }
#pragma unroll
            for (int q = 0; q < kRq; ++q) uq[q] = kq[q] ? row_uniform(a, r, iq[q]) : 0.5f;
#pragma unroll
            for (int q = 0; q < kRq; ++q) {
                if (!kq[q]) continue;
                const float y = val_of(sm.ck[wave][i0 + q * kWave]) / Tt;
                dq[q] = y - m;
                yq[q] = key_of(y);
            }
#pragma unroll
            for (int q = 0; q < kRq; ++q) {
                if (!kq[q]) continue;
                const uint64_t lk = ((uint64_t)yq[q] << 32) | (uint32_t)iq[q];
                rs.nkept++;
                rs.last = rs.last > lk ? rs.last : lk;
                rs.add_key(exp_det(dq[q]) / (0.0f - log_det(uq[q])), iq[q]);
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (!mk[h]) continue;
            const uint64_t g = mg[h];
            rs.nkept++;
            rs.last = rs.last > g ? rs.last : g;
            rs.add_key(exp_det(val_of((uint32_t)(g >> 32)) - m) / (0.0f - log_det(mu[h])),
                       (int32_t)(uint32_t)g);
        }
        rs.shfl_merge(32); rs.shfl_merge(16); rs.shfl_merge(8);
        rs.shfl_merge(4); rs.shfl_merge(2); rs.shfl_merge(1);
        const uint32_t nbw = (uint32_t)wave_sum_u64(below_cands);
        __syncthreads();  // the per-wave records' last readers are done
        if (lane == 0) {
            sm.red[wave][0] = rs.best;
            sm.red[wave][1] = rs.last;
            sm.red[wave][2] = ((uint64_t)rs.second << 32) | rs.nkept;
            sm.red[wave][3] = nbw;
        }
        __syncthreads();
        if (tid == 0) {
            RowRace all;
            all.best = sm.wrace[0];  // the wide race pass's survivors (wide rows), counted once
            all.second = (uint32_t)sm.wrace[1];
            all.last = sm.wrace[3];
            uint64_t nbelow = 0ull;
            for (int w = 0; w < kTpWaves; ++w) {
                RowRace o;
                o.best = sm.red[w][0];
                o.last = sm.red[w][1];
                o.second = (uint32_t)(sm.red[w][2] >> 32);
                o.nkept = (uint32_t)sm.red[w][2];
                all.merge(o);
                nbelow += sm.red[w][3];
            }
            // the first near-tie term counts when a survivor was removed: below the candidates,
            // among them, or in the boundary bucket
            const bool any_removed = any_below_nc || nbelow > 0ull || cpos > 0u;
            uint32_t f = 0u;
            if ((any_removed && (tflags & 1u)) || (tflags & 2u)) f |= VWS_FLAG_TOPP_NEAR_TIE;
            int32_t tok;
            if (all.best) {
                tok = (int32_t)(0x7FFFFFFF - (uint32_t)(all.best & 0xFFFFFFFFu));
                const float bk = u2f((uint32_t)(all.best >> 32));
                if (all.second) {
                    const float sk = u2f(all.second - 1u);
                    if ((double)sk >= (double)bk * (1.0 - 1e-6)) f |= VWS_FLAG_RACE_NEAR_TIE;
                }
            } else {
                tok = (int32_t)(uint32_t)(all.last & 0xFFFFFFFFu);
            }
            sm.bc[12] = (uint32_t)tok;
            sm.bc[13] = f;
            sm.bc[14] = all.nkept + (uint32_t)sm.wrace[2];
        }
        __syncthreads();
        token = (int32_t)tp_u(sm.bc[12]);
        flags |= tp_u(sm.bc[13]);
        nkept = (int32_t)tp_u(sm.bc[14]);
    }

    VWS_TRACE_MARK(a, VWS_TRACE_TP_RACE);
    // ---- raw logprobs: every element at or above the sampled one is a candidate
    float logS = 0.0f, xs = 0.0f;
    uint32_t rank = 0u;
    if (L >= 0) {
        const T* row = reinterpret_cast<const T*>(a.logits) + (size_t)r * a.lstride;
        xs = Elem<T>::load1(row + token);
        if (a.softcap > 0.0f) xs = softcap_out(xs, a.inv_softcap, a.softcap, a.softcap_f16 != 0);
        xs = tp_uf(xs);
        const uint32_t ks = key_of(xs);
        // a sampled token below the candidates (wide rows) is ranked by a pass over the row
        const bool rank_pass = ks < tauk;
        uint32_t rk = 0u;
        if (rank_pass) {
            pass(kTpPassRank, ks, 0);
            if (tp_u(sm.coop_fail)) return VWS_FALLBACK_COOP;
            rk = wave == 0 ? (uint32_t)tp_u64(sm.bc64[10]) : 0u;  // the per-wave records below add up
        } else {
            if (hist) {
                // raw values: the unmarked entries and the listed raw ones
                for (int i = lane; i < cnt; i += kWave)
                    rk += (sm.ck[wave][i] >= ks && !((uint32_t)sm.ci[wave][i] & kTpHist)) ? 1u : 0u;
                for (uint32_t j = (uint32_t)tid; j < tp_u(sm.rl_n); j += NT) rk += sm.rl_key[j] >= ks ? 1u : 0u;
            } else {
                for (int i = lane; i < cnt; i += kWave) rk += sm.ck[wave][i] >= ks ? 1u : 0u;
            }
            rk = (uint32_t)wave_sum_u64(rk);
        }
        uint32_t ncand = 0u;
        {
            // the L largest raw values lie in the buckets from the top that hold L candidates
            const int b0 = 2 * tid, b1 = 2 * tid + 1;
            const uint32_t c0 = sm.h.hcnt[b0], c1 = sm.h.hcnt[b1];
            uint64_t pre;                                                 // candidates in buckets < b0
            ncand = (uint32_t)tp_scan(c0 + c1, sm, 2, &pre);
            if (L > 0) {
                if (pre < (uint64_t)L && pre + c0 >= (uint64_t)L) sm.bc[15] = (uint32_t)b0;
                if (pre + c0 < (uint64_t)L && pre + c0 + c1 >= (uint64_t)L) sm.bc[15] = (uint32_t)b1;
            }
            if (lane == 0) sm.red[wave][3] = rk;
            if (wave == 0) {
                // log-sum-exp of the raw logits: the buffered part plus the stream's terms
                const bool u1 = greedy || Tt == 1.0f;
                const double sw = lane < kTpWaves ? ((u1 ? sm.wS[lane] : sm.wSR[lane]) -
                                                     (hist ? (u1 ? sm.wSub[lane] : sm.wSRsub[lane]) : 0.0)) : 0.0;
                const double s0 = sm.tot_s0b + tp_wave_sum_f64(sw) * exp((double)aw - (double)sm.xr);
                if (lane == 0) sm.bc64[8] = (uint64_t)__double_as_longlong(s0);
            }
        }
        __syncthreads();
        rank = (uint32_t)tp_sum16(sm, 3);
        logS = (float)log(__longlong_as_double((long long)tp_u64(sm.bc64[8])));
        if (L > 0) {
            if (ncand < (uint32_t)L) return VWS_FALLBACK_TOPL;  // the top-L reaches below the candidates
            const int bl = (int)tp_u(sm.bc[15]);
            const bool unitT = greedy || Tt == 1.0f;
            const float mr = unitT ? tp_uf(sm.xr) : tp_uf(sm.xr) / Tt;
            // history rows: raw values (unmarked entries and the listed raw ones) against the
            // threshold and the raw buckets
            auto raw_in = [&](uint32_t kr) __attribute__((always_inline)) {
                return kr >= tauk && tp_bucket((unitT ? val_of(kr) : val_of(kr) / Tt) - mr) <= bl;
            };
            auto gather = [&](auto hc) __attribute__((always_inline)) {
                for (int i = lane; i < cnt; i += kWave) {
                    const uint32_t c = (uint32_t)sm.ci[wave][i];
                    if (decltype(hc)::value ? ((c & kTpHist) || !raw_in(sm.ck[wave][i]))
                                            : ((c & kTpBelow) || tp_code_bucket(c) > bl))
                        continue;
                    const uint32_t pos = atomicAdd(&sm.bc[7], 1u);
                    if (pos < (uint32_t)kTpLpCap) {
                        sm.lp.key[pos] = sm.ck[wave][i];
                        sm.lp.idx[pos] = (int32_t)(c & imask);
                    }
                }
            };
            if (hist) gather(BoolC<true>{});
            else gather(BoolC<false>{});
            if (hist) {
                for (uint32_t j = (uint32_t)tid; j < tp_u(sm.rl_n); j += NT) {
                    if (!raw_in(sm.rl_key[j])) continue;
                    const uint32_t pos = atomicAdd(&sm.bc[7], 1u);
                    if (pos < (uint32_t)kTpLpCap) {
                        sm.lp.key[pos] = sm.rl_key[j];
                        sm.lp.idx[pos] = sm.rl_idx[j];
                    }
                }
            }
            __syncthreads();
            if (tp_u(sm.bc[7]) > (uint32_t)kTpLpCap) return VWS_FALLBACK_TOPL;
        }
    }

    VWS_TRACE_MARK(a, VWS_TRACE_TP_LOGPROBS);
    // ---- outputs (nothing was written before this point)
    if (tid == 0) {
        a.sampled[r] = token;
        if (a.flags) a.flags[r] = flags;
        if (a.nkept) a.nkept[r] = nkept;
    }
    if (L >= 0) {
        const int stride = L + 1;
        if (tid == 0) {
            a.lp_ids[(size_t)r * stride] = token;
            a.lp_vals[(size_t)r * stride] = (xs - sm.xr) - logS;
            a.lp_ranks[r] = (int32_t)rank;
        }
        if (L > 0) {
            const uint32_t n = tp_u(sm.bc[7]);
            for (uint32_t j = tid; j < n; j += NT) {
                const uint32_t kj = sm.lp.key[j];
                const int32_t ij = sm.lp.idx[j];
                int pos = 0;
                for (uint32_t i = 0; i < n; ++i) {
                    const uint32_t ki = sm.lp.key[i];
                    pos += (ki > kj || (ki == kj && sm.lp.idx[i] < ij)) ? 1 : 0;
                }
                if (pos < L) {
                    a.lp_ids[(size_t)r * stride + 1 + pos] = ij;
                    a.lp_vals[(size_t)r * stride + 1 + pos] = (val_of(kj) - tp_uf(sm.xr)) - logS;
                }
            }
        }
    }
    return 0;
}

}  // namespace vws
