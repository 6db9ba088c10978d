// vws_device.h -- device-side building blocks of the gfx950 sampler: the sampler arithmetic
// (bit-exact fp32 exp/log, order keys, integer masses), wave64 primitives and a wave-level
// radix select over LDS-resident keys.
//
// The arithmetic below is the project's definition of exp_det / log_det: fixed sequences of
// IEEE fp32 add/mul/fma that give the same bits on any IEEE machine.  The file must be
// compiled with -ffp-contract=off so that no multiply-add is fused behind our back.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vws {

constexpr int kWave = 64;
constexpr float kSamplingEps = 1e-5f;

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// Wave ballot of a condition.  HIP's __ballot takes an int, which makes the compiler materialise
// the condition in a register and compare it again; the builtin on a bool uses the compare's
// lane mask directly.
__device__ __forceinline__ uint64_t wave_ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// exp(d) for d in [-80, 80] (clamped above), 0 below -80 and for NaN.  Cody-Waite
// reduction n = rint(d * log2 e), r = d - n * ln2 with a 16-bit head of ln2 (n * head is
// exact) and an fp32 tail; exp(r) = 1 + r + r^2 Q(r) with Q of degree 4 fitted for this
// project on [-ln2/2, ln2/2]; exact scaling by 2^n.  Max error 1 ulp (checked on every fp32).
// Written without branches (special cases are selected at the end) so that it schedules freely
// in straight-line code.
__device__ __forceinline__ float exp_det(float d0) {
    const float d = __builtin_fminf(__builtin_fmaxf(d0, -80.0f), 80.0f);
    const float t = d * 0x1.715476p+0f;
    const float n = __builtin_rintf(t);
    float r = __builtin_fmaf(-n, 0x1.62e4p-1f, d);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = __builtin_fmaf(0x1.6d7532p-10f, r, 0x1.120b66p-7f);
    p = __builtin_fmaf(p, r, 0x1.5554b8p-5f);
    p = __builtin_fmaf(p, r, 0x1.5554dcp-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = (int)n;
    const float v = p * u2f((uint32_t)(ni + 127) << 23);
    const float v1 = __builtin_fabsf(d) < 0x1p-30f ? 1.0f : v;
    return (d0 >= -80.0f) ? v1 : 0.0f;  // below -80 and NaN: 0
}

// log(u) for u > 0: u = 2^e m with m in [sqrt(1/2), sqrt(2)], f = m - 1 (exact),
// log1p(f) = f + f^2 R(f) with R of degree 8 fitted for this project, log u = e ln2 + log1p(f).
// log(0) = -inf, log(+inf) = +inf, NaN otherwise.  Max error 1 ulp (checked on every fp32).
// Branch-free like exp_det: the special inputs are selected at the end.
__device__ __forceinline__ float log_det(float u) {
    const bool sub = f2u(u) < 0x00800000u;
    const uint32_t b = f2u(sub ? u * 0x1p23f : u);
    const bool hi = ((b & 0x007FFFFFu) | 0x3F800000u) > 0x3FB504F3u;
    const int e = (sub ? -23 : 0) + (int)((b >> 23) & 0xFFu) - 127 + (hi ? 1 : 0);
    const uint32_t mb = ((b & 0x007FFFFFu) | 0x3F800000u) - (hi ? 0x00800000u : 0u);
    const float f = u2f(mb) - 1.0f;
    const float f2 = f * f;
    float R = __builtin_fmaf(-0x1.4a5298p-4f, f, 0x1.088e82p-3f);
    R = __builtin_fmaf(R, f, -0x1.0bb9f2p-3f);
    R = __builtin_fmaf(R, f, 0x1.2245c6p-3f);
    R = __builtin_fmaf(R, f, -0x1.548f6ep-3f);
    R = __builtin_fmaf(R, f, 0x1.99a7bap-3f);
    R = __builtin_fmaf(R, f, -0x1.0001f8p-2f);
    R = __builtin_fmaf(R, f, 0x1.555548p-2f);
    R = __builtin_fmaf(R, f, -0x1.fffffep-2f);
    const float L = __builtin_fmaf(f2, R, f);
    const float ef = (float)e;
    const float v = e == 0 ? L : __builtin_fmaf(ef, 0x1.62e43p-1f, __builtin_fmaf(ef, -0x1.05c61p-29f, L));
    const float vi = u == __builtin_inff() ? u : v;
    return (u > 0.0f) ? vi : ((u == 0.0f) ? -__builtin_inff() : __builtin_nanf(""));
}

// Gemma's final-logit soft cap, cap * tanh(x / cap), with the reference's formula
// (vllm_webgpu/shaders/gemma/logit_softcap.wgsl:13-28): v = x * fl(1 / cap); tanh(v) = +-1 for
// |v| >= 20, else (e - 1) / (e + 1) with e = exp_det(2v); result t * cap in fp32.  NaN stays
// NaN.  Branch-free; the same operation sequence as the oracle's vwo_softcap.
__device__ __forceinline__ float softcap_det(float x, float inv_cap, float cap) {
    const float v = x * inv_cap;
    const float e = exp_det(2.0f * __builtin_fminf(__builtin_fmaxf(v, -20.0f), 20.0f));
    const float t0 = (e - 1.0f) / (e + 1.0f);
    const float t = v >= 20.0f ? 1.0f : (v <= -20.0f ? -1.0f : t0);
    return x != x ? x : t * cap;
}

// fp32 -> f16 (nearest, ties to even; overflow to +-inf) -> fp32: what an f16 store keeps.
__device__ __forceinline__ float round_f16(float v) { return (float)(_Float16)v; }

// The model's capped logit: softcap_det, rounded as an f16 store when the model stores the
// cap's output in f16 (vllm_webgpu/shaders/gemma/logit_softcap.wgsl:28).
__device__ __forceinline__ float softcap_out(float x, float inv_cap, float cap, bool f16) {
    const float c = softcap_det(x, inv_cap, cap);
    return f16 ? round_f16(c) : c;
}

// An upper bound on softcap_det(x') over every x' <= x (NaN excluded).  The fp32 tanh above is
// not monotone: over every fp32 v in [-20, 20] (it is constant outside), the largest drop
// max_{v' <= v} t(v') - t(v) is 2^-22.  v = x * (1 / cap) and t * cap round monotonically, so
// the capped values of x' <= x exceed softcap_det(x) by less than cap * 2^-21; this adds
// cap * 2^-20.
__device__ __forceinline__ float softcap_bound(float x, float inv_cap, float cap) {
    return softcap_det(x, inv_cap, cap) + cap * 0x1p-20f;
}

// A raw value below x whose capped value lies about twice softcap_bound's margin below x's:
// x - cap * 2^-19 / (1 - t^2), t = tanh(x / cap) (the cap's slope is 1 - t^2; near saturation
// the step stops growing at 1024 times its smallest value).  Any value works as a threshold;
// this one leaves x's capped value clear of the bound of everything below it.
__device__ __forceinline__ float softcap_lower(float x, float inv_cap, float cap) {
    const float t = softcap_det(x, inv_cap, cap) * inv_cap;
    return x - cap * 0x1p-19f / __builtin_fmaxf(1.0f - t * t, 0x1p-10f);
}

// A compile-time flag passed as a value (selects a specialisation of a generic lambda).
template <bool B>
struct BoolC {
    static constexpr bool value = B;
};

// floor(e * 2^44) for e in [0, 1]; 0 for e <= 0 or NaN.  Every step is exact in fp32:
// f = e * 2^44 (a power-of-two scaling, f <= 2^44), its high word floor(f / 2^32) and the rest
// f - hi * 2^32 (a multiple of f's ulp below 2^32, so the fma rounds nothing), each converted
// by truncation.  (Checked against the shift-based form on every fp32 up to 2^19.)
__device__ __forceinline__ uint64_t mass_of(float e) {
    const float f = __builtin_ldexpf(e > 0.0f ? e : 0.0f, 44);
    const float hf = __builtin_truncf(f * 0x1p-32f);
    const float lf = __builtin_fmaf(-hf, 0x1p32f, f);
    return ((uint64_t)(uint32_t)hf << 32) | (uint32_t)lf;
}

// Philox-4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as easy as 1, 2, 3",
// SC 2011): ten rounds, each multiplying counter words 0 and 2 by the round constants (32 x 32
// -> 64 bits) and mixing the halves with the other words and the key; the key advances by the
// Weyl constants after each round.  c: the counter (in), the four output words (out).
__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int i = 0; i < 10; ++i) {
        const uint64_t p0 = (uint64_t)c[0] * 0xD2511F53u;  // one 32 x 32 -> 64 multiply each
        const uint64_t p1 = (uint64_t)c[2] * 0xCD9E8D57u;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        c[0] = n0;
        c[1] = (uint32_t)p1;
        c[2] = n2;
        c[3] = (uint32_t)p0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

// A Philox word as the race's uniform: (2 floor(w / 2^9) + 1) 2^-24, an odd multiple of
// 2^-24 in (0, 1), exact in fp32.
__device__ __forceinline__ float philox_word_uniform(uint32_t w) {
    return (float)(2u * (w >> 9) + 1u) * 0x1p-24f;
}

// The generated uniforms of the N consecutive tokens t0 .. t0 + N - 1, t0 a multiple of 4 and
// N of 4: one Philox block per 4 tokens (philox_uniform of each).
template <int N>
__device__ __forceinline__ void philox_uniforms_aligned(uint64_t seed, uint64_t offset, uint32_t t0,
                                                        float (&u)[N]) {
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
        uint32_t c[4] = {(t0 >> 2) + (uint32_t)q, (uint32_t)offset, (uint32_t)(offset >> 32), 0u};
        philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
#pragma unroll
        for (int j = 0; j < 4; ++j) u[4 * q + j] = philox_word_uniform(c[j]);
    }
}

// The race's generated uniform of token t for a row with 64-bit key `seed` and `offset`: word
// t % 4 of Philox-4x32-10 at counter (t / 4, offset lo, offset hi, 0) with key (seed lo, seed
// hi), as (2 floor(w / 2^9) + 1) 2^-24, an odd multiple of 2^-24 in (0, 1).
__device__ __forceinline__ float philox_uniform(uint64_t seed, uint64_t offset, uint32_t t) {
    uint32_t c[4] = {t >> 2, (uint32_t)offset, (uint32_t)(offset >> 32), 0u};
    philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    const uint32_t j = t & 3u;
    const uint32_t w = j == 0u ? c[0] : (j == 1u ? c[1] : (j == 2u ? c[2] : c[3]));
    return philox_word_uniform(w);
}

// Order-preserving key: x < y <=> key(x) < key(y); -0 and +0 share a key; NaN -> 0.
__device__ __forceinline__ uint32_t key_of(float x) {
    uint32_t b = f2u(x);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0;
    if (b == 0x80000000u) b = 0;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Inverse of key_of on keys >= 1 (key 0 maps to a NaN).
__device__ __forceinline__ float val_of(uint32_t k) {
    return u2f((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// floor(q * W) for fp32 q in (0, 1) and W < 2^64, exact (128-bit product).
__device__ __forceinline__ uint64_t scale_floor(float q, uint64_t W) {
    const uint32_t b = f2u(q);
    const int ex = (int)(b >> 23);
    const uint64_t mq = ex ? ((b & 0x7FFFFFu) | 0x800000u) : (b & 0x7FFFFFu);
    const int sh = 150 - (ex ? ex : 1);
    const uint64_t lo = mq * W;
    const uint64_t hi = __umul64hi(mq, W);
    if (sh >= 128) return 0;
    if (sh >= 64) return hi >> (sh - 64);
    if (sh == 0) return lo;
    return (lo >> sh) | (hi << (64 - sh));
}

// vLLM-v1 penalty step: repetition on prompt|output tokens (x > 0: x * fl(1/r), else x * r),
// then x - f * count, then x - p * (count > 0).
__device__ __forceinline__ float apply_penalty(float x, bool in_prompt, uint32_t cnt, float rep,
                                               float inv_rep, float freq, float pres) {
    if (in_prompt || cnt > 0) x = (x > 0.0f) ? x * inv_rep : x * rep;
    x = x - freq * (float)cnt;
    x = x - pres * (cnt > 0 ? 1.0f : 0.0f);
    return x;
}

// History hash value word: output occurrences (bits 0-28), a logit bias present (bit 29),
// banned by a logits processor (bit 30), token in the prompt (bit 31).
constexpr uint32_t kHCount = 0x1FFFFFFFu;
// The bits of a token-state word (prompt flag, output count) the penalties read; the word has
// the hash value's layout without the processor flags.
constexpr uint32_t kStateMask = 0x80000000u | kHCount;
constexpr uint32_t kHBias = 1u << 29;
constexpr uint32_t kHBan = 1u << 30;
constexpr uint32_t kHPrompt = 1u << 31;

// A token of the row's hash: the logits processors (ban, else logit bias), then the penalties.
__device__ __forceinline__ float apply_hashed(float x, uint32_t hv, float bias, float rep,
                                              float inv_rep, float freq, float pres) {
    if (hv & kHBan) x = -__builtin_inff();
    else if (hv & kHBias) x = x + bias;
    return apply_penalty(x, (hv & kHPrompt) != 0u, hv & kHCount, rep, inv_rep, freq, pres);
}

// Greedy rows: temperature < 1e-5 or NaN.
__device__ __forceinline__ bool is_greedy(float T) { return !(T >= kSamplingEps); }

// ---- wave64 primitives ------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// Lane id computed at the point of use: the volatile asm is re-executed rather than kept live,
// so loops that need the lane's position do not hold a long-lived per-lane register for it.
__device__ __forceinline__ int lane_now() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

__device__ __forceinline__ int lane_prefix(uint64_t mask) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// v of lane (lane ^ s) for s in {1, 2, 4, 8, 16, 32}, on the VALU: DPP moves inside a row of
// 16 (xor 4 and xor 8 as compositions of mirrors), permlane swaps across rows and halves.
// Cheaper than an LDS-crossbar shuffle; s is a compile-time constant after unrolling.
__device__ __forceinline__ uint32_t lane_xor(uint32_t v, int s) {
    switch (s) {
    case 1: return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    case 2: return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    case 4:  // row_half_mirror (l ^ 7), then quad_perm [3,2,1,0] (l ^ 3)
        return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false), 0x1B,
                                        0xF, 0xF, false);
    case 8:  // row_mirror (l ^ 15), then row_half_mirror (l ^ 7)
        return __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false), 0x141,
                                        0xF, 0xF, false);
    case 16: {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane_id() & 16) ? p[0] : p[1];
    }
    default: {
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane_id() & 32) ? p[0] : p[1];
    }
    }
}
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v, int s) {
    return ((uint64_t)lane_xor((uint32_t)(v >> 32), s) << 32) | lane_xor((uint32_t)v, s);
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    const int l = lane_id();
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t t = __shfl_up(v, o, kWave);
        if (l >= o) v += t;
    }
    return v;
}

// Butterfly over the wave with op(a, b), strides 32 .. 1 written out (each stride is a
// constant, so lane_xor is a fixed DPP / permlane sequence).
#define VWS_BUTTERFLY(v, XOR, OP)          \
    do {                                   \
        v = OP(v, XOR(v, 32));             \
        v = OP(v, XOR(v, 16));             \
        v = OP(v, XOR(v, 8));              \
        v = OP(v, XOR(v, 4));              \
        v = OP(v, XOR(v, 2));              \
        v = OP(v, XOR(v, 1));              \
    } while (0)

__device__ __forceinline__ uint32_t vws_max32(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t vws_min32(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint64_t vws_max64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t vws_min64(uint64_t a, uint64_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint64_t vws_add64(uint64_t a, uint64_t b) { return a + b; }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    VWS_BUTTERFLY(v, lane_xor, vws_max32);
    return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    VWS_BUTTERFLY(v, lane_xor, vws_min32);
    return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
    VWS_BUTTERFLY(v, lane_xor64, vws_add64);
    return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    VWS_BUTTERFLY(v, lane_xor64, vws_max64);
    return v;
}

// Wave-aggregated LDS atomics, for per-element counters that many lanes of a wave may hit at
// once (elements that share a key or a bucket: the -inf elements of a masked row, a flat row's
// masses): LDS serialises the lanes of one atomic instruction that address one word, so such a
// wave costs 64 LDS cycles per instruction where one atomic of the sum would do.  Each helper
// may be called in divergent code; it covers the lanes active at the call.
//
// base[idx] += 1 for each active lane: one atomic when every active lane has the same idx.
__device__ __forceinline__ void agg_count(uint32_t* base, uint32_t idx) {
    const uint64_t act = wave_ballot(true);
    const uint32_t i0 = __builtin_amdgcn_readfirstlane(idx);
    if (wave_ballot(idx == i0) == act) {
        if (lane_id() == (int)__builtin_ctzll(act)) atomicAdd(&base[i0], (uint32_t)__popcll(act));
    } else {
        atomicAdd(&base[idx], 1u);
    }
}
// base[idx] += w for each active lane: one atomic of the wave's sum when all 64 lanes are
// active and share idx (the sum needs every lane's value).
__device__ __forceinline__ void agg_add64(uint64_t* base, uint32_t idx, uint64_t w) {
    const uint64_t act = wave_ballot(true);
    const uint32_t i0 = __builtin_amdgcn_readfirstlane(idx);
    if (act == ~0ull && wave_ballot(idx == i0) == act) {
        const uint64_t sum = wave_sum_u64(w);
        if (lane_id() == 0 && sum)
            atomicAdd(reinterpret_cast<unsigned long long*>(&base[i0]), (unsigned long long)sum);
    } else if (w) {
        atomicAdd(reinterpret_cast<unsigned long long*>(&base[idx]), (unsigned long long)w);
    }
}
// A slot of the counter *ctr for each active lane (ascending with the lane), one atomic per wave.
__device__ __forceinline__ uint32_t agg_reserve(uint32_t* ctr) {
    const uint64_t act = wave_ballot(true);
    uint32_t b = 0u;
    if (lane_id() == (int)__builtin_ctzll(act)) b = atomicAdd(ctr, (uint32_t)__popcll(act));
    return __builtin_amdgcn_readfirstlane(b) + (uint32_t)lane_prefix(act);
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
    VWS_BUTTERFLY(v, lane_xor64, vws_min64);
    return v;
}

// k-th largest key (1-based, counting multiplicity) among keys[0..n) in LDS, computed by one
// whole wave with a 4 x 8-bit radix select.  hist: 256 words of wave-private LDS.
// Requires 1 <= k <= n.
__device__ __forceinline__ uint32_t wave_kth_largest(const uint32_t* keys, int n, int k,
                                                     uint32_t* hist) {
    const int lane = lane_id();
    uint32_t prefix = 0, pmask = 0;
    uint32_t rem = (uint32_t)k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int b = lane; b < 256; b += kWave) hist[b] = 0;
        wave_sync();
        for (int i = lane; i < n; i += kWave) {
            const uint32_t kk = keys[i];
            if ((kk & pmask) == prefix) atomicAdd(&hist[(kk >> shift) & 255u], 1u);
        }
        wave_sync();
        // lane l owns bins 255-4l .. 252-4l (descending key order)
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

// The four largest keys of the wave (one key per lane, counted with multiplicity): lane i < 4
// receives the (i+1)-th largest, the other lanes 0.
__device__ __forceinline__ uint32_t wave_top4(uint32_t v) {
    const int lane = lane_id();
    uint32_t mine = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t mk = wave_max_u32(v);
        const uint64_t at = wave_ballot(v == mk);  // never empty: mk is some lane's key
        if (lane == (int)__builtin_ctzll(at)) v = 0u;
        if (lane == i) mine = mk;
    }
    return mine;
}

// The m-th largest of the wave's keys (one per lane, 1 <= m <= 64), in every lane: the largest
// x with at least m keys >= x, decided bit by bit from the top.
__device__ __forceinline__ uint32_t wave_mth_largest64(uint32_t v, int m) {
    uint32_t ans = 0u;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const uint32_t cand = ans | (1u << b);
        if (__popcll(wave_ballot(v >= cand)) >= m) ans = cand;
    }
    return ans;
}

// The same by counting, for one wave that selects for the workgroup: every lane counts the
// keys >= its own (64 lane reads, no dependent chain), and the answer is the largest key with
// at least m of them.
// N: the keys of lanes [0, N) take part (the others must hold 0).
template <int N = kWave>
__device__ __forceinline__ uint32_t wave_mth_largest64_count(uint32_t v, int m) {
    uint32_t cge = 0u;
#pragma unroll
    for (int j = 0; j < N; ++j) cge += __builtin_amdgcn_readlane(v, j) >= v ? 1u : 0u;
    return wave_max_u32(cge >= (uint32_t)m ? v : 0u);
}

// k-th largest key (1-based, with multiplicity) of at most 256 keys held 4 per lane by one
// whole wave (missing entries passed as 0): an in-register bitonic sort into descending order
// across the wave (element e = 4 * lane + i), then a read of element k - 1.
__device__ __forceinline__ uint32_t wave_kth_largest_256(uint32_t v0, uint32_t v1, uint32_t v2,
                                                         uint32_t v3, int k) {
    const int lane = lane_id();
    uint32_t v[4] = {v0, v1, v2, v3};
#pragma unroll
    for (int size = 2; size <= 256; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= 4) {
                const int lstride = stride >> 2;
                const bool upper = (lane & lstride) != 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int e = 4 * lane + i;
                    const bool desc = (e & size) == 0;
                    const uint32_t o = lane_xor(v[i], lstride);
                    const uint32_t hi = v[i] > o ? v[i] : o, lo = v[i] > o ? o : v[i];
                    // the lower element of a pair keeps the larger key in a descending block
                    v[i] = (upper != desc) ? hi : lo;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if ((i & stride) == 0) {
                        const int e = 4 * lane + i;
                        const bool desc = (e & size) == 0;
                        const uint32_t x = v[i], y = v[i + stride];
                        const bool swap = desc ? (x < y) : (x > y);
                        v[i] = swap ? y : x;
                        v[i + stride] = swap ? x : y;
                    }
                }
            }
        }
    }
    const int src = (k - 1) >> 2, sel = (k - 1) & 3;
    const uint32_t r0 = __builtin_amdgcn_readlane(v[0], src), r1 = __builtin_amdgcn_readlane(v[1], src);
    const uint32_t r2 = __builtin_amdgcn_readlane(v[2], src), r3 = __builtin_amdgcn_readlane(v[3], src);
    return sel == 0 ? r0 : sel == 1 ? r1 : sel == 2 ? r2 : r3;
}

// One key per lane sorted descending across the wave (bitonic network): lane i gets the i-th
// largest key.
__device__ __forceinline__ uint32_t wave_sort_desc64(uint32_t v) {
    const int lane = lane_id();
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint32_t o = lane_xor(v, stride);
            const bool desc = (lane & size) == 0;
            const bool upper = (lane & stride) != 0;
            const uint32_t hi = v > o ? v : o, lo = v > o ? o : v;
            v = (upper != desc) ? hi : lo;
        }
    }
    return v;
}

// Number of keys >= t among keys[0..n) (one whole wave).
__device__ __forceinline__ int wave_count_ge(const uint32_t* keys, int n, uint32_t t) {
    int c = 0;
    for (int i = lane_id(); i < n; i += kWave) c += (keys[i] >= t) ? 1 : 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) c += lane_xor(c, o);
    return c;
}

// ---- logits element access --------------------------------------------------------------

template <typename T> struct Elem;
template <> struct Elem<float> {
    static constexpr int kVec = 4;  // elements per 16-byte load
    __device__ __forceinline__ static float load1(const float* p) { return *p; }
    __device__ __forceinline__ static void load_vec(const float* p, float* out) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    }
    // the kVec elements of 16 loaded bytes
    __device__ __forceinline__ static void from_words(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                                      float* out) {
        out[0] = u2f(w0); out[1] = u2f(w1); out[2] = u2f(w2); out[3] = u2f(w3);
    }
};
template <> struct Elem<uint16_t> {  // bfloat16 bit patterns, widened exactly
    static constexpr int kVec = 8;
    __device__ __forceinline__ static float load1(const uint16_t* p) { return u2f((uint32_t)(*p) << 16); }
    __device__ __forceinline__ static void load_vec(const uint16_t* p, float* out) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = u2f(w[i] << 16);
            out[2 * i + 1] = u2f(w[i] & 0xFFFF0000u);
        }
    }
    __device__ __forceinline__ static void from_words(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                                      float* out) {
        const uint32_t w[4] = {w0, w1, w2, w3};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = u2f(w[i] << 16);
            out[2 * i + 1] = u2f(w[i] & 0xFFFF0000u);
        }
    }
};

template <> struct Elem<_Float16> {  // IEEE binary16, widened exactly
    static constexpr int kVec = 8;
    __device__ __forceinline__ static float lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)w); }
    __device__ __forceinline__ static float hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }
    __device__ __forceinline__ static float load1(const _Float16* p) { return (float)*p; }
    __device__ __forceinline__ static void load_vec(const _Float16* p, float* out) {
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        from_words(v.x, v.y, v.z, v.w, out);
    }
    __device__ __forceinline__ static void from_words(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                                      float* out) {
        const uint32_t w[4] = {w0, w1, w2, w3};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = lo(w[i]);
            out[2 * i + 1] = hi(w[i]);
        }
    }
};

// Data shared between the workgroups of one launch (which may run on different XCDs, whose L2
// caches are not coherent with each other): every access is an agent-scope atomic, which the
// memory model makes coherent across XCDs without whole-cache writeback or invalidation.  A
// workgroup publishes with stores_complete() (its own accesses have all completed) and a
// barrier before the single atomic that signals them; the reader issues its loads only after
// it has seen that signal.
__device__ __forceinline__ uint32_t ag_load32(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ag_load64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ag_store32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ag_store64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ag_add32(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ag_add64(uint64_t* p, uint64_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stores_complete() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Buffer resource over `bytes` bytes at p (raw addressing): a load whose vector offset (plus
// instruction offset) is at or past `bytes` returns zero and never faults.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// A row slice [lo, hi) seen as chunks of kVec elements: chunk 0 is the unaligned head
// (elements before the first 16-byte boundary), chunks 1..nbody are aligned vectors and chunk
// nbody+1 is the tail.  Elements outside the slice read as NaN, which every consumer ignores.
template <typename T> struct Slice {
    const T* row;
    int lo, hi;      // element range
    int a;           // first aligned element (>= lo, <= hi)
    int nbody;       // aligned vectors
    __device__ __forceinline__ void init(const T* row_, int lo_, int hi_) {
        row = row_; lo = lo_; hi = hi_;
        const uintptr_t addr = reinterpret_cast<uintptr_t>(row + lo);
        const int mis = (int)((addr & 15u) / sizeof(T));
        int head = mis ? (Elem<T>::kVec - mis) : 0;
        if (head > hi - lo) head = hi - lo;
        a = lo + head;
        nbody = (hi - a) / Elem<T>::kVec;
    }
    __device__ int nchunks() const { return nbody + 2; }
    // Aligned vector vi of the body with the index clamped into range (nbody >= 1), so the load
    // is unconditional and can stay in flight; vectors with vi >= nbody repeat the last vector
    // and must be discarded by the consumer (their element index is >= body_end()).
    __device__ __forceinline__ int load_body(int vi, float* out) const {
        constexpr int V = Elem<T>::kVec;
        const int vc = vi < nbody ? vi : nbody - 1;
        Elem<T>::load_vec(row + a + vc * V, out);
        return a + vi * V;
    }
    __device__ __forceinline__ int body_end() const { return a + nbody * Elem<T>::kVec; }
    // Unaligned head (which = 0) or tail (which = 1) elements as one NaN-padded chunk.
    __device__ __forceinline__ int load_edge(int which, float* out) const {
        constexpr int V = Elem<T>::kVec;
        const int i0 = which == 0 ? lo : a + nbody * V;
        const int end = which == 0 ? a : hi;
#pragma unroll
        for (int j = 0; j < V; ++j) out[j] = (i0 + j < end) ? Elem<T>::load1(row + i0 + j) : __builtin_nanf("");
        return i0;
    }
    // Loads chunk c into out[kVec]; returns the index of out[0].
    __device__ __forceinline__ int load(int c, float* out) const {
        constexpr int V = Elem<T>::kVec;
        const float nan = __builtin_nanf("");
        if (c >= 1 && c <= nbody) {
            const int i0 = a + (c - 1) * V;
            Elem<T>::load_vec(row + i0, out);
            return i0;
        }
        const int i0 = (c == 0) ? lo : a + nbody * V;
        const int end = (c == 0) ? a : hi;
#pragma unroll
        for (int j = 0; j < V; ++j) out[j] = (c <= nbody + 1 && i0 + j < end) ? Elem<T>::load1(row + i0 + j) : nan;
        return i0;
    }
};

}  // namespace vws
