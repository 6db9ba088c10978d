/*
 * vws_oracle.c -- CPU oracle for the MI355X token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  The product library (vllm_webgpu_amd/_vws.so) neither links nor
 * loads this file.  Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py
 * use it, and only as the checker.
 *
 * What it restates, one row at a time in plain sequential C:
 *   - greedy argmax, lowest index on ties: vllm_webgpu/v1/model_runner.py:145 (numpy argmax);
 *     the single-row WGSL kernel vllm_webgpu/shaders/generic/argmax.wgsl:1-60 has the same
 *     I/O contract; it never selects NaN (strict '>' at :28-31), and neither does this oracle.
 *   - top-k values/ids, descending: vllm_webgpu/shaders/generic/topk256.wgsl:1-70.
 *   - online max/normaliser softmax: vllm_webgpu/shaders/generic/softmax.wgsl:26-70.
 *   - the vLLM-v1 Sampler the plugin delegates sampling to
 *     (docs/superpowers/specs/2026-06-29-vllm-webgpu-design.md:451; pyproject.toml:10,
 *     vllm>=0.20, not vendored in the reference): logits processors (allowed-token mask,
 *     bans, logit bias) -> penalties -> temperature -> min-p -> top-k -> top-p ->
 *     exponential race, and raw logprobs.
 *
 * Sampler arithmetic (the definition that makes token ids reproducible bit for bit):
 *   exp_det / log_det are fixed fp32 operation sequences (Cody-Waite reduction and
 *   polynomials fitted for this project; every step is an IEEE add, mul or fma), so any
 *   IEEE-754 machine that runs the same sequence gets the same bits.  Compile with
 *   -ffp-contract=off.
 *   top-p uses exact integer masses w = floor(e * 2^44) and exact 64/128-bit sums, so the
 *   cumulative sum does not depend on summation order.
 *   min-p keeps a token iff fl(y - max) >= log_det(min_p) (the logit-space form of
 *   p >= max_p * min_p).
 *   The exponential race key is e / (0 - log_det(u)); the largest key wins, lowest index on
 *   equal keys.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define VWO_FLAG_TOPP_NEAR_TIE 0x1u
#define VWO_FLAG_RACE_NEAR_TIE 0x2u
#define VWO_FLAG_DEGENERATE 0x4u
#define VWO_FLAG_GREEDY 0x8u

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- sampler arithmetic --------------------------------------------------------------- */

/* exp(d) on [-80, 80]; 0 below -80 and for NaN.  Cody-Waite: n = rint(d*log2e),
 * r = d - n*ln2 with ln2 split into a 16-bit head (n*head is exact) and an fp32 tail,
 * exp(r) = 1 + r + r^2*Q(r), Q of degree 4 fitted on [-ln2/2, ln2/2] (max rel err 7.5e-9),
 * then an exact scale by 2^n. */
float vwo_exp(float d) {
    if (!(d >= -80.0f)) return 0.0f;
    if (d > 80.0f) d = 80.0f;
    if (fabsf(d) < 0x1p-30f) return 1.0f;
    const float t = d * 0x1.715476p+0f;
    const float n = rintf(t);
    float r = fmaf(-n, 0x1.62e4p-1f, d);
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = fmaf(0x1.6d7532p-10f, r, 0x1.120b66p-7f);
    p = fmaf(p, r, 0x1.5554b8p-5f);
    p = fmaf(p, r, 0x1.5554dcp-3f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n;
    return p * u2f((uint32_t)(ni + 127) << 23);
}

/* log(u) for u > 0: u = 2^e * m, m in [sqrt(1/2), sqrt(2)], f = m - 1 (exact),
 * log1p(f) = f + f^2*R(f), R of degree 8 fitted on [sqrt(1/2)-1, sqrt(2)-1] (rel err 1e-8),
 * log(u) = e*ln2 + log1p(f).  log(0) = -inf, log(+inf) = +inf, NaN for u < 0 or NaN. */
float vwo_log(float u) {
    if (!(u > 0.0f)) return (u == 0.0f) ? -INFINITY : NAN;
    if (u == INFINITY) return INFINITY;
    uint32_t b = f2u(u);
    int e = 0;
    if (b < 0x00800000u) { b = f2u(u * 0x1p23f); e = -23; }
    e += (int)(b >> 23) - 127;
    uint32_t mb = (b & 0x007FFFFFu) | 0x3F800000u;
    if (mb > 0x3FB504F3u) { mb -= 0x00800000u; e += 1; }
    const float f = u2f(mb) - 1.0f;
    const float f2 = f * f;
    float R = fmaf(-0x1.4a5298p-4f, f, 0x1.088e82p-3f);
    R = fmaf(R, f, -0x1.0bb9f2p-3f);
    R = fmaf(R, f, 0x1.2245c6p-3f);
    R = fmaf(R, f, -0x1.548f6ep-3f);
    R = fmaf(R, f, 0x1.99a7bap-3f);
    R = fmaf(R, f, -0x1.0001f8p-2f);
    R = fmaf(R, f, 0x1.555548p-2f);
    R = fmaf(R, f, -0x1.fffffep-2f);
    const float L = fmaf(f2, R, f);
    if (e == 0) return L;
    const float ef = (float)e;
    return fmaf(ef, 0x1.62e43p-1f, fmaf(ef, -0x1.05c61p-29f, L));
}

/* Gemma's final-logit soft cap, cap * tanh(x / cap), as the reference computes it
 * (vllm_webgpu/shaders/gemma/logit_softcap.wgsl:13-28): v = x * fl(1 / cap); tanh(v) = +-1 for
 * |v| >= 20, else (e - 1) / (e + 1) with e = exp(2v), here e = vwo_exp(2v); the result is t * cap
 * in fp32 (the reference stores it as f16; this library keeps fp32).  NaN stays NaN. */
float vwo_softcap(float x, float inv_cap, float cap) {
    if (x != x) return x;
    const float v = x * inv_cap;
    float t;
    if (v >= 20.0f) {
        t = 1.0f;
    } else if (v <= -20.0f) {
        t = -1.0f;
    } else {
        const float e = vwo_exp(2.0f * v);
        t = (e - 1.0f) / (e + 1.0f);
    }
    return t * cap;
}

/* Philox-4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as easy as 1, 2, 3",
 * SC 2011): ten rounds, each multiplying counter words 0 and 2 by the round constants (32 x 32
 * -> 64 bits) and mixing the halves with the other words and the key; the key advances by
 * the Weyl constants after each round.  c: the counter (in), the four output words (out). */
void vwo_philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
    for (int i = 0; i < 10; ++i) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
        const uint32_t n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
        const uint32_t n3 = (uint32_t)p0;
        c[0] = n0; c[1] = n1; c[2] = n2; c[3] = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

/* The sampler's generated uniform of token t for a row with 64-bit key `seed` and 64-bit
 * `offset`: word t % 4 of Philox-4x32-10 at counter (t / 4, offset lo, offset hi, 0) with key
 * (seed lo, seed hi), mapped to (2 floor(w / 2^9) + 1) 2^-24, an odd multiple of 2^-24 in
 * (0, 1) (exact in fp32, never 0 or 1). */
float vwo_philox_uniform(uint64_t seed, uint64_t offset, uint32_t t) {
    uint32_t c[4] = {t >> 2, (uint32_t)offset, (uint32_t)(offset >> 32), 0u};
    vwo_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    return (float)(2u * (c[t & 3u] >> 9) + 1u) * 0x1p-24f;
}

/* Every row's uniforms [B, V] from per-row seeds and offsets (offsets may be NULL: 0). */
void vwo_philox_uniforms(const uint64_t* seeds, const uint64_t* offsets, int B, int V, float* out) {
#pragma omp parallel for schedule(static)
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < V; ++t)
            out[(size_t)b * V + t] = vwo_philox_uniform(seeds[b], offsets ? offsets[b] : 0u, (uint32_t)t);
}

/* fp32 -> binary16 (round to nearest, ties to even; overflow to +-inf, underflow through the
 * subnormals to +-0) -> fp32: the value an f16 store keeps, widened back exactly.  The
 * reference's soft-cap shader writes its fp32 result t * cap into an f16 buffer
 * (vllm_webgpu/shaders/gemma/logit_softcap.wgsl:28). */
float vwo_round_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t ax = x & 0x7FFFFFFFu;
    const int neg = (x >> 31) != 0u;
    if (ax > 0x7F800000u) return f;                      /* NaN */
    if (ax >= 0x477FF000u) return neg ? -INFINITY : INFINITY;  /* >= 65520: rounds to inf */
    if (ax <= 0x33000000u) return neg ? -0.0f : 0.0f;    /* <= 2^-25: ties to 0 (even) */
    const int e = (int)(ax >> 23) - 127;                 /* -25 <= e <= 15 */
    const int shift = e < -14 ? 13 + (-14 - e) : 13;     /* mantissa bits an f16 drops */
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    m >>= shift;
    if (rem > half || (rem == half && (m & 1u))) m += 1u;
    const float r = ldexpf((float)m, e - 23 + shift);   /* exact: m <= 2^11 */
    return neg ? -r : r;
}

/* The soft cap of a row; round_f16: each result as an f16 store keeps it. */
void vwo_softcap_row(const float* x, int V, float cap, int round_f16, float* out) {
    const float inv = 1.0f / cap;
    for (int i = 0; i < V; ++i) {
        const float c = vwo_softcap(x[i], inv, cap);
        out[i] = round_f16 ? vwo_round_f16(c) : c;
    }
}

/* floor(e * 2^44) for e in [0, 1] (0 for e <= 0 or NaN). */
uint64_t vwo_mass(float e) {
    if (!(e > 0.0f)) return 0;
    const uint32_t b = f2u(e);
    const int ex = (int)(b >> 23);
    const uint64_t mant = ex ? ((b & 0x7FFFFFu) | 0x800000u) : (b & 0x7FFFFFu);
    const int sh = (ex ? ex : 1) - 106;
    if (sh >= 0) return mant << sh;
    if (sh <= -64) return 0;
    return mant >> (-sh);
}

/* Order-preserving key: x < y  <=>  key(x) < key(y); -0 and +0 share a key; NaN -> 0,
 * below -inf (whose key is 0x007FFFFF). */
uint32_t vwo_key(float x) {
    uint32_t b = f2u(x);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0;
    if (b == 0x80000000u) b = 0;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* floor(q * W) exactly, for fp32 q in (0, 1) and W < 2^64. */
uint64_t vwo_scale_floor(float q, uint64_t W) {
    const uint32_t b = f2u(q);
    const int ex = (int)(b >> 23);
    const uint64_t mq = ex ? ((b & 0x7FFFFFu) | 0x800000u) : (b & 0x7FFFFFu);
    const int sh = 150 - (ex ? ex : 1); /* q = mq * 2^-sh, sh >= 24 for q < 1 */
    const unsigned __int128 prod = (unsigned __int128)mq * (unsigned __int128)W;
    if (sh >= 128) return 0;
    return (uint64_t)(prod >> sh);
}

/* One repetition/frequency/presence penalty step, vLLM-v1 order: repetition on
 * prompt|output tokens (x>0: x*fl(1/r), else x*r -- the torch fallback form), then
 * x - f*count, then x - p*(count>0). */
static inline float apply_pen(float x, int in_prompt, uint32_t cnt, float rep, float inv_rep,
                              float freq, float pres) {
    if (in_prompt || cnt > 0) x = (x > 0.0f) ? x * inv_rep : x * rep;
    x = x - freq * (float)cnt;
    x = x - pres * (cnt > 0 ? 1.0f : 0.0f);
    return x;
}

/* ---- per-row sampler ------------------------------------------------------------------ */

typedef struct {
    float temperature, top_p, min_p, rep, pres, freq;
    int32_t top_k, _pad;
} vwo_params;

typedef struct {
    int32_t token;
    uint32_t flags;
    int32_t n_kept;        /* |S|: tokens with non-zero probability after all truncation */
    int32_t n_topk;        /* tokens surviving temperature + min-p + top-k */
    uint64_t mass_total;   /* W over the top-k/min-p survivors */
    uint64_t threshold;    /* floor(q32 * W) when top-p is active, else 0 */
    float row_max;         /* m = max y */
    float kth_y;           /* k-th largest y (or -inf when top-k is off) */
} vwo_row_out;

static int cmp_u64(const void* a, const void* b) {
    const uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return (x > y) - (x < y);
}

/* k-th largest key (with multiplicity) among keys[0..n), 1 <= k <= n. */
static uint32_t kth_largest_key(const uint32_t* keys, int n, int k) {
    uint32_t* tmp = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
    memcpy(tmp, keys, sizeof(uint32_t) * (size_t)n);
    /* two-level 16-bit radix select, from the top */
    uint32_t* hist = (uint32_t*)calloc(65536, sizeof(uint32_t));
    for (int i = 0; i < n; ++i) hist[tmp[i] >> 16]++;
    int rem = k, hi = 65535;
    for (; hi >= 0; --hi) { if ((int)hist[hi] >= rem) break; rem -= (int)hist[hi]; }
    memset(hist, 0, 65536 * sizeof(uint32_t));
    for (int i = 0; i < n; ++i) if ((tmp[i] >> 16) == (uint32_t)hi) hist[tmp[i] & 0xFFFF]++;
    int lo = 65535;
    for (; lo >= 0; --lo) { if ((int)hist[lo] >= rem) break; rem -= (int)hist[lo]; }
    free(hist);
    free(tmp);
    return ((uint32_t)hi << 16) | (uint32_t)lo;
}

/* vLLM-v1's logits processors that run before the penalties, in place on x (length V):
 * tokens whose bit is clear in `allowed` (V bits, NULL = all allowed) and tokens listed with
 * value -inf (bad words, min-tokens stop ids) become -inf; a token listed with a finite value
 * gets x + value (logit bias; at most one finite entry per token).  Ids outside [0, V) are
 * padding. */
void vwo_apply_adjustments_row(float* x, int V, const uint32_t* allowed, const int32_t* ids,
                               const float* vals, int n) {
    if (allowed)
        for (int i = 0; i < V; ++i)
            if (!((allowed[i >> 5] >> (i & 31)) & 1u)) x[i] = -INFINITY;
    uint8_t* ban = n > 0 ? (uint8_t*)calloc((size_t)V, 1) : NULL;
    for (int j = 0; j < n; ++j)
        if (ids[j] >= 0 && ids[j] < V && vals[j] == -INFINITY) ban[ids[j]] = 1;
    for (int j = 0; j < n; ++j) {
        const int t = ids[j];
        if (t < 0 || t >= V || ban[t] || vals[j] == -INFINITY) continue;
        x[t] = x[t] + vals[j];
    }
    for (int t = 0; n > 0 && t < V; ++t) if (ban[t]) x[t] = -INFINITY;
    free(ban);
}

/* Applies penalties to x (length V) in place.  Token ids outside [0, V) are padding. */
void vwo_apply_penalties_row(float* x, int V, const int32_t* prompt, int np, const int32_t* output,
                             int no, float rep, float pres, float freq) {
    uint32_t* cnt = (uint32_t*)calloc((size_t)V, sizeof(uint32_t));
    uint8_t* inp = (uint8_t*)calloc((size_t)V, 1);
    for (int i = 0; i < np; ++i) if (prompt[i] >= 0 && prompt[i] < V) inp[prompt[i]] = 1;
    for (int i = 0; i < no; ++i) if (output[i] >= 0 && output[i] < V) cnt[output[i]]++;
    const float inv_rep = 1.0f / rep;
    for (int i = 0; i < V; ++i)
        if (inp[i] || cnt[i]) x[i] = apply_pen(x[i], inp[i], cnt[i], rep, inv_rep, freq, pres);
    free(cnt);
    free(inp);
}

int32_t vwo_argmax_row(const float* x, int V) {
    int32_t best = 0;
    uint32_t bk = 0;
    for (int i = 0; i < V; ++i) {
        const uint32_t k = vwo_key(x[i]);
        if (k > bk) { bk = k; best = i; }
    }
    return best;
}

/* Full sampler on one row.  x0: raw fp32 logits (bf16 inputs are widened exactly by the
 * caller).  u: uniforms [V] in (0,1).  Logprob outputs (optional, L >= 0): lp_ids/lp_vals have
 * L+1 entries: [sampled, top1..topL]; *rank = #{j : x0_j >= x0_sampled}. */
int vwo_sample_row(const float* x0, int V, const int32_t* prompt, int np, const int32_t* output,
                   int no, const uint32_t* allowed, const int32_t* adj_ids, const float* adj_vals,
                   int na, const vwo_params* prm, const float* u, int L, int32_t* lp_ids,
                   float* lp_vals, int32_t* rank, vwo_row_out* out) {
    memset(out, 0, sizeof(*out));
    out->kth_y = -INFINITY;
    float* x = (float*)malloc(sizeof(float) * (size_t)V);
    memcpy(x, x0, sizeof(float) * (size_t)V);
    if (allowed || na > 0) vwo_apply_adjustments_row(x, V, allowed, adj_ids, adj_vals, na);
    const int has_hist = (np > 0 || no > 0);
    if (has_hist) vwo_apply_penalties_row(x, V, prompt, np, output, no, prm->rep, prm->pres, prm->freq);

    const float T = prm->temperature;
    if (!(T >= 1e-5f)) { /* greedy row: argmax of penalised, pre-temperature logits */
        out->token = vwo_argmax_row(x, V);
        out->flags = VWO_FLAG_GREEDY;
        out->n_kept = 1;
        out->n_topk = 1;
        goto logprobs;
    }
    {
        float* y = (float*)malloc(sizeof(float) * (size_t)V);
        uint32_t* ky = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)V);
        float m = -INFINITY;
        uint32_t mk = 0;
        int32_t mi = 0;
        int nvalid = 0;
        for (int i = 0; i < V; ++i) {
            y[i] = x[i] / T;
            ky[i] = vwo_key(y[i]);
            if (ky[i]) nvalid++;
            if (ky[i] > mk) { mk = ky[i]; mi = i; m = y[i]; }
        }
        out->row_max = m;
        if (!(m > -INFINITY && m < INFINITY)) { /* degenerate row: greedy over y */
            out->token = mi;
            out->flags = VWO_FLAG_DEGENERATE;
            out->n_kept = 1;
            out->n_topk = 1;
            free(y); free(ky);
            goto logprobs;
        }
        /* min-p (logit-space form) */
        float lp_min = -INFINITY;
        if (prm->min_p > 0.0f) lp_min = vwo_log(prm->min_p < 1.0f ? prm->min_p : 1.0f);
        /* top-k: keep y >= k-th largest y */
        uint32_t kth = 0;
        const int k = prm->top_k;
        if (k > 0 && k < V && k <= nvalid) kth = kth_largest_key(ky, V, k);
        /* gather survivors of top-k and min-p as packed (key << 32 | idx) */
        uint64_t* s = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
        int ns = 0;
        for (int i = 0; i < V; ++i) {
            if (!ky[i] || ky[i] < kth) continue;
            if (!((y[i] - m) >= lp_min)) continue;
            s[ns++] = ((uint64_t)ky[i] << 32) | (uint32_t)i;
        }
        if (kth) { for (int i = 0; i < V; ++i) if (ky[i] == kth) { out->kth_y = y[i]; break; } }
        out->n_topk = ns;
        qsort(s, (size_t)ns, sizeof(uint64_t), cmp_u64); /* (y asc, idx asc) */
        uint64_t* w = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(ns ? ns : 1));
        float* e = (float*)malloc(sizeof(float) * (size_t)(ns ? ns : 1));
        uint64_t W = 0;
        for (int j = 0; j < ns; ++j) {
            const int i = (int)(uint32_t)s[j];
            e[j] = vwo_exp(y[i] - m);
            w[j] = vwo_mass(e[j]);
            W += w[j];
        }
        out->mass_total = W;
        int first = 0; /* first kept position in ascending order */
        const float q32 = 1.0f - prm->top_p;
        if (q32 > 0.0f && ns > 0) {
            const uint64_t thr = vwo_scale_floor(q32 < 1.0f ? q32 : 0x1.fffffep-1f, W);
            /* q32 >= 1 means top_p <= 0: every token but the last is removed */
            const int all_but_last = !(q32 < 1.0f);
            out->threshold = thr;
            uint64_t C = 0, Cprev = 0;
            for (first = 0; first < ns - 1; ++first) {
                const uint64_t Cn = C + w[first];
                if (!all_but_last && Cn > thr) break;
                Cprev = Cn;
                C = Cn;
            }
            if (!all_but_last) {
                const uint64_t tol = (uint64_t)((double)W * 1e-6);
                const uint64_t Cat = C + w[first];
                if ((first > 0 && thr - Cprev <= tol) || (Cat > thr && Cat - thr <= tol))
                    out->flags |= VWO_FLAG_TOPP_NEAR_TIE;
            }
        }
        out->n_kept = ns - first;
        /* exponential race over the kept tail s[first..ns) */
        int32_t best = -1;
        float bkey = 0.0f, skey = -1.0f;
        for (int j = first; j < ns; ++j) {
            const int i = (int)(uint32_t)s[j];
            const float q = 0.0f - vwo_log(u[i]);
            const float key = e[j] / q;
            if (!(key >= 0.0f)) continue; /* NaN keys never win */
            if (best < 0 || key > bkey || (key == bkey && i < best)) {
                if (best >= 0) skey = (bkey > skey) ? bkey : skey;
                best = i;
                bkey = key;
            } else if (key > skey) {
                skey = key;
            }
        }
        if (best < 0) best = (int32_t)(uint32_t)s[ns - 1]; /* no valid key: most probable */
        else if (skey >= 0.0f && (double)skey >= (double)bkey * (1.0 - 1e-6))
            out->flags |= VWO_FLAG_RACE_NEAR_TIE;
        out->token = best;
        free(w); free(e); free(s); free(y); free(ky);
    }
logprobs:
    if (L >= 0 && lp_ids) {
        double m0 = -INFINITY;
        for (int i = 0; i < V; ++i) if (x0[i] == x0[i] && x0[i] > m0) m0 = x0[i];
        double S0 = 0.0;
        for (int i = 0; i < V; ++i) if (x0[i] == x0[i]) S0 += exp((double)x0[i] - m0);
        const double lse = m0 + log(S0);
        const int32_t s = out->token;
        lp_ids[0] = s;
        lp_vals[0] = (float)((double)x0[s] - lse);
        const uint32_t ks = vwo_key(x0[s]);
        int32_t r = 0;
        for (int i = 0; i < V; ++i) { const uint32_t kk = vwo_key(x0[i]); if (kk && kk >= ks) r++; }
        *rank = r;
        if (L > 0) {
            /* top-L by (x0 desc, idx asc): sort packed (~key << 32 | idx) ascending */
            uint64_t* t = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
            for (int i = 0; i < V; ++i) t[i] = ((uint64_t)(~vwo_key(x0[i])) << 32) | (uint32_t)i;
            qsort(t, (size_t)V, sizeof(uint64_t), cmp_u64);
            for (int j = 0; j < L && j < V; ++j) {
                const int i = (int)(uint32_t)t[j];
                lp_ids[1 + j] = i;
                lp_vals[1 + j] = (float)((double)x0[i] - lse);
            }
            free(t);
        }
    }
    free(x);
    return 0;
}

/* Batched driver (rows are independent; OpenMP over rows when built with -fopenmp).
 * prompt/output: padded [B, *_stride] with ids outside [0, V) ignored; lens may be NULL.
 * softcap > 0: the logits are first mapped through vwo_softcap (they are the model's output
 * then: processors, penalties and the raw logprobs all see the capped values); softcap_f16:
 * each capped value rounded as an f16 store (vwo_round_f16). */
int vwo_sample_batch(const float* logits, int B, int V, const int32_t* prompt, int prompt_stride,
                     const int32_t* prompt_lens, const int32_t* output, int output_stride,
                     const int32_t* output_lens, const uint32_t* allowed, int allowed_stride,
                     const int32_t* adj_ids, const float* adj_vals, int adj_stride,
                     const int32_t* adj_lens, const vwo_params* prm, const float* uniforms,
                     int L, int32_t* lp_ids, float* lp_vals, int32_t* ranks, vwo_row_out* outs,
                     float softcap, int softcap_f16) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int b = 0; b < B; ++b) {
        float* capped = NULL;
        if (softcap > 0.0f) {
            capped = (float*)malloc(sizeof(float) * (size_t)V);
            vwo_softcap_row(logits + (size_t)b * V, V, softcap, softcap_f16, capped);
        }
        const int np = prompt ? (prompt_lens ? prompt_lens[b] : prompt_stride) : 0;
        const int no = output ? (output_lens ? output_lens[b] : output_stride) : 0;
        const int na = adj_ids ? (adj_lens ? adj_lens[b] : adj_stride) : 0;
        vwo_sample_row(capped ? capped : logits + (size_t)b * V, V,
                       prompt ? prompt + (size_t)b * prompt_stride : NULL, np,
                       output ? output + (size_t)b * output_stride : NULL, no,
                       allowed ? allowed + (size_t)b * allowed_stride : NULL,
                       adj_ids ? adj_ids + (size_t)b * adj_stride : NULL,
                       adj_vals ? adj_vals + (size_t)b * adj_stride : NULL, na, &prm[b],
                       uniforms ? uniforms + (size_t)b * V : NULL, L,
                       lp_ids ? lp_ids + (size_t)b * (L + 1) : NULL,
                       lp_vals ? lp_vals + (size_t)b * (L + 1) : NULL, ranks ? ranks + b : NULL,
                       &outs[b]);
        free(capped);
    }
    return 0;
}

/* Top-k values/ids of one row, (value desc, index asc); the topk256.wgsl contract. */
void vwo_topk_row(const float* x, int V, int k, float* vals, int32_t* ids) {
    uint64_t* t = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
    for (int i = 0; i < V; ++i) t[i] = ((uint64_t)(~vwo_key(x[i])) << 32) | (uint32_t)i;
    qsort(t, (size_t)V, sizeof(uint64_t), cmp_u64);
    for (int j = 0; j < k && j < V; ++j) { ids[j] = (int32_t)(uint32_t)t[j]; vals[j] = x[ids[j]]; }
    free(t);
}

/* softmax(x / T) of one row with the sampler's exp: p_i = exp_det(fl(x_i/T) - m) / S,
 * S accumulated in double.  Also returns m and log(S) (so log-sum-exp = m + log S). */
void vwo_softmax_row(const float* x, int V, float T, float* probs, float* row_max, double* log_sum) {
    float m = -INFINITY;
    for (int i = 0; i < V; ++i) { const float y = x[i] / T; if (y > m) m = y; }
    double S = 0.0;
    for (int i = 0; i < V; ++i) S += (double)vwo_exp(x[i] / T - m);
    for (int i = 0; i < V; ++i) probs[i] = (float)((double)vwo_exp(x[i] / T - m) / S);
    *row_max = m;
    *log_sum = log(S);
}

/* ---- exhaustive checks of the arithmetic (pins exp_det/log_det against libm double) --- */

static int64_t ulp_diff(float a, float b) {
    const int64_t ka = (int64_t)vwo_key(a), kb = (int64_t)vwo_key(b);
    return ka > kb ? ka - kb : kb - ka;
}

/* Walks every fp32 d in [lo, hi] with the given bit stride; reports the max ulp error of
 * exp_det against double exp rounded to fp32, and a 64-bit hash of all outputs. */
void vwo_check_exp(float lo, float hi, uint32_t stride, int64_t* max_ulp, float* worst,
                   uint64_t* hash, uint64_t* count) {
    int64_t mu = 0; float wd = 0.0f; uint64_t h = 0, c = 0;
    const uint32_t klo = vwo_key(lo), khi = vwo_key(hi);
#pragma omp parallel
    {
        int64_t lmu = 0; float lwd = 0.0f; uint64_t lh = 0, lc = 0;
#pragma omp for schedule(static)
        for (int64_t kk = klo; kk <= (int64_t)khi; kk += stride) {
            const uint32_t key = (uint32_t)kk;
            const uint32_t bits = (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
            const float d = u2f(bits);
            const float got = vwo_exp(d);
            const float want = (d >= -80.0f) ? (float)exp((double)d) : 0.0f;
            const int64_t du = ulp_diff(got, want);
            if (du > lmu) { lmu = du; lwd = d; }
            lh += (uint64_t)f2u(got) * 0x9E3779B97F4A7C15ull ^ (uint64_t)bits;
            lc++;
        }
#pragma omp critical
        {
            if (lmu > mu) { mu = lmu; wd = lwd; }
            h += lh; c += lc;
        }
    }
    *max_ulp = mu; *worst = wd; *hash = h; *count = c;
}

/* vwo_round_f16 on every fp32 of [lo, hi] (bit stride): the same hash as vwo_check_exp, to
 * compare with the device's fp32 -> f16 -> fp32 conversion. */
void vwo_check_round_f16(float lo, float hi, uint32_t stride, uint64_t* hash, uint64_t* count) {
    uint64_t h = 0, c = 0;
    const uint32_t klo = vwo_key(lo), khi = vwo_key(hi);
#pragma omp parallel
    {
        uint64_t lh = 0, lc = 0;
#pragma omp for schedule(static)
        for (int64_t kk = klo; kk <= (int64_t)khi; kk += stride) {
            const uint32_t key = (uint32_t)kk;
            const uint32_t bits = (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
            lh += (uint64_t)f2u(vwo_round_f16(u2f(bits))) * 0x9E3779B97F4A7C15ull ^ (uint64_t)bits;
            lc++;
        }
#pragma omp critical
        {
            h += lh; c += lc;
        }
    }
    *hash = h; *count = c;
}

/* vwo_softcap at cap 1 (t(x), the cap's tanh) on every fp32 x whose key lies in [lo, hi]: the
 * largest absolute error against tanh in double, the same hash as vwo_check_exp (comparable
 * with the device self-test) and the largest drop max_{x' <= x} t(x') - t(x).  t is not
 * monotone in fp32: the device sampler's single pass thresholds raw logits and relies on this
 * drop bound to decide when a capped row is settled.  The drop uses two passes over fixed
 * chunks (chunk maxima, then each chunk with the running maximum of the chunks before it). */
void vwo_check_softcap(float lo, float hi, double* max_err, float* worst, uint64_t* hash,
                       uint64_t* count, double* max_drop) {
    const uint32_t klo = vwo_key(lo), khi = vwo_key(hi);
    const int64_t n = (int64_t)khi - klo + 1, nch = 256, per = (n + nch - 1) / nch;
    float cmax[256];
    double me = 0.0; float wd = 0.0f; uint64_t h = 0, c = 0;
#pragma omp parallel
    {
        double lme = 0.0; float lwd = 0.0f; uint64_t lh = 0, lc = 0;
#pragma omp for schedule(dynamic)
        for (int64_t ch = 0; ch < nch; ++ch) {
            float m = -2.0f;
            for (int64_t i = ch * per; i < (ch + 1) * per && i < n; ++i) {
                const uint32_t key = klo + (uint32_t)i;
                const uint32_t bits = (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
                const float x = u2f(bits);
                const float t = vwo_softcap(x, 1.0f, 1.0f);
                const double err = fabs((double)t - tanh((double)x));
                if (err > lme) { lme = err; lwd = x; }
                lh += (uint64_t)f2u(t) * 0x9E3779B97F4A7C15ull ^ (uint64_t)bits;
                lc++;
                if (t > m) m = t;
            }
            cmax[ch] = m;
        }
#pragma omp critical
        {
            if (lme > me) { me = lme; wd = lwd; }
            h += lh; c += lc;
        }
    }
    double drop = 0.0;
#pragma omp parallel
    {
        double ld = 0.0;
#pragma omp for schedule(dynamic)
        for (int64_t ch = 0; ch < nch; ++ch) {
            float run = -2.0f;
            for (int64_t j = 0; j < ch; ++j) run = cmax[j] > run ? cmax[j] : run;
            for (int64_t i = ch * per; i < (ch + 1) * per && i < n; ++i) {
                const uint32_t key = klo + (uint32_t)i;
                const uint32_t bits = (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
                const float t = vwo_softcap(u2f(bits), 1.0f, 1.0f);
                if (t > run) run = t;
                const double d = (double)run - (double)t;
                if (d > ld) ld = d;
            }
        }
#pragma omp critical
        if (ld > drop) drop = ld;
    }
    *max_err = me; *worst = wd; *hash = h; *count = c; *max_drop = drop;
}

void vwo_check_log(float lo, float hi, uint32_t stride, int64_t* max_ulp, float* worst,
                   uint64_t* hash, uint64_t* count) {
    int64_t mu = 0; float wd = 0.0f; uint64_t h = 0, c = 0;
    const uint32_t klo = vwo_key(lo), khi = vwo_key(hi);
#pragma omp parallel
    {
        int64_t lmu = 0; float lwd = 0.0f; uint64_t lh = 0, lc = 0;
#pragma omp for schedule(static)
        for (int64_t kk = klo; kk <= (int64_t)khi; kk += stride) {
            const uint32_t key = (uint32_t)kk;
            const uint32_t bits = (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
            const float uu = u2f(bits);
            const float got = vwo_log(uu);
            const float want = (float)log((double)uu);
            const int64_t du = ulp_diff(got, want);
            if (du > lmu) { lmu = du; lwd = uu; }
            lh += (uint64_t)f2u(got) * 0x9E3779B97F4A7C15ull ^ (uint64_t)bits;
            lc++;
        }
#pragma omp critical
        {
            if (lmu > mu) { mu = lmu; wd = lwd; }
            h += lh; c += lc;
        }
    }
    *max_ulp = mu; *worst = wd; *hash = h; *count = c;
}
