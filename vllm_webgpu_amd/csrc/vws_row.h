// vws_row.h -- per-row sampling parameters as the kernels see them, and the rule that sends a
// row to the single-pass kernel or to the general kernel.
#pragma once

#include "vws_device.h"
#include "vws_internal.h"
#include "vws_sampler.h"

namespace vws {

struct RowP {
    float T, top_p, min_p, rep, pres, freq, inv_rep;
    int k, np, no;
    int na;          // logits-processor entries (bans, logit bias) of the row
    bool greedy;
    bool has_hist;   // penalties apply: a history and not every penalty the identity
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
    p.np = a.prompt ? (a.plens ? min(max(a.plens[r], 0), a.pwidth) : a.pwidth) : 0;
    p.no = a.output ? (a.olens ? min(max(a.olens[r], 0), a.owidth) : a.owidth) : 0;
    // vLLM skips the penalty step when every penalty is the identity; the result is the same
    const bool identity = (p.rep == 1.0f && p.pres == 0.0f && p.freq == 0.0f);
    p.has_hist = (p.np > 0 || p.no > 0) && !identity;
    p.na = a.adj_ids ? (a.adjlens ? min(max(a.adjlens[r], 0), a.adjwidth) : a.adjwidth) : 0;
    if (a.mode == kModeTopK) {
        p.greedy = false;
        p.has_hist = false;
        p.na = 0;
        p.k = a.topk_k;
    }
    p.need_hash = p.has_hist || p.na > 0;
    return p;
}

// k served by the single-pass kernel for this row, or 0 when the row needs the general kernel.
__device__ __forceinline__ int fast_k(const KArgs& a, const RowP& p) {
    if (a.mode == kModeTopK) return a.topk_k;
    if (a.L >= 0 || a.allowed) return 0;
    if (p.greedy) return 1;
    if (p.k > 0 && p.k < a.V && p.k <= kKMax) return p.k;
    return 0;
}

}  // namespace vws
