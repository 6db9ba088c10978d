// vws_internal.h -- kernel argument block and workspace layout shared by the launchers
// (vws_capi.hip) and the kernels (vws_sample_row.hip, vws_topk.hip, vws_ops.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vws {

// Split-row top-k operation (vws_topk.hip): shape constants.
constexpr int kFastThreads = 256;                 // 4 waves per part
constexpr int kFastWaves = kFastThreads / 64;
constexpr int kCapW = 512;                        // candidate slots per wave (LDS)
constexpr int kKMax = 256;                        // largest k of the top-k operation and of the
                                                  // sampling kernel's single pass
constexpr int kPartCap = 512;                     // list entries a part may publish
constexpr int kMergeCap = kFastWaves * kCapW;     // entries the last part can merge
constexpr int kPartMax = 32768;                   // elements per part
constexpr int kMaxParts = 16;                    // parts per row: VWS_MAX_VOCAB / kPartMax

// General path (one workgroup per row, multi-pass).
constexpr int kGenThreads = 1024;
constexpr int kGenWaves = kGenThreads / 64;
constexpr int kBuckets = 4096;                    // d-buckets of width 1/128 over d in [0, 32)
constexpr int kGatherCap = 2048;                  // boundary-bucket entries resolved in LDS
constexpr int kLpCapW = 192;                      // per-wave top-L candidate slots

// The sampling kernel's instantiations by what the top-p path does to each logit as it loads it
// (the single pass caps candidates only and masks as it streams): nothing, the launch's allowed
// mask (masked elements become -inf), or the launch's soft cap (cap * tanh(x / cap), with its
// f16 store when asked); the same in every pass over a row.
constexpr int kXfNone = 0;
constexpr int kXfMask = 1;
constexpr int kXfCap = 2;

// Row states written by the fast path for the general path.
constexpr uint32_t kRowNeedsGeneral = 1u;

// Cooperative passes (vws_topp.h).  A top-p row whose decision needs a further pass over its
// logits hands the pass out in chunks of kCoopChunkVecs 16-byte vectors through a slot here;
// workgroups whose own row is done take chunks and add their results into the slot.  The
// region sits at the start of every workspace; each launch leaves it ready for the next one.
constexpr int kCoopSlots = 16;
constexpr int kCoopMaxChunks = 64;
constexpr int kCoopBuckets = 2048;                // the top-p path's exact-mass buckets
constexpr int kCoopGather = 2048;                 // boundary-bucket members a slot gathers
constexpr int kCoopChunkVecs = 4 * kGenThreads;   // vectors per chunk (a multiple of this)
constexpr int kCoopWaitPolls = 1 << 20;           // default bound of the owner's wait for helpers
// An owner that stops waiting adds kCoopAbandon - (chunks helpers still owe) to the slot's done
// count; the completion that brings it to exactly kCoopAbandon (the owner's own add when every
// chunk was already done, or the last late helper's increment) frees the slot.
constexpr uint32_t kCoopAbandon = 1u << 30;

struct CoopSlot {
    uint64_t claim;    // generation (bits 40-63) | chunks of the pass (32-39) | next chunk (0-31)
    uint64_t sw, n, nrem;                  // totals added by the workgroups that helped
    uint32_t done;     // chunks finished by workgroups other than the owner
    uint32_t owner;    // row + 1 while a row holds the slot, 0 when free
    uint32_t ngather;  // boundary-bucket members appended to gkey
    int32_t kind, r, bstar;                // the pass (read once the chunk is claimed)
    uint32_t key, ksv, kkeep, kmem;
    float Tt, m, lp_min;
    int32_t cvecs;     // vectors per chunk
    uint32_t pad[4];
    uint64_t race[kCoopMaxChunks][3];      // wide race per chunk: best, second << 32 | kept, last
    uint64_t hmass[kCoopBuckets];          // exact pass: bucket masses
    uint64_t gkey[kCoopGather];            // wide race: boundary-bucket members
};

// wgs: workgroups started (bits 0-19) and finished (bits 20-39), counted only when the grid is
// larger than the device holds at once (coop_count); rows holding a slot (bits 40-51); top-p
// rows in progress, which may still open a pass (bits 52-63).
constexpr uint64_t kCoopStarted = 1ull;
constexpr uint64_t kCoopFinished = 1ull << 20;
constexpr uint64_t kCoopActive = 1ull << 40;
constexpr uint64_t kCoopPending = 1ull << 52;
constexpr int kCoopMaxGrid = (1 << 20) - 1;
// Largest counted batch whose rows are served longest first (each workgroup of such a launch
// reads every row's parameters twice to find its row, O(B^2) in all); larger batches run in
// index order.
constexpr int kRowOrderMaxBatch = 16384;
inline __host__ __device__ uint32_t coop_started(uint64_t w) { return (uint32_t)(w & 0xFFFFFu); }
inline __host__ __device__ uint32_t coop_finished(uint64_t w) { return (uint32_t)((w >> 20) & 0xFFFFFu); }
inline __host__ __device__ uint32_t coop_active(uint64_t w) { return (uint32_t)((w >> 40) & 0xFFFu); }
inline __host__ __device__ uint32_t coop_pending(uint64_t w) { return (uint32_t)(w >> 52); }

struct CoopState {
    uint64_t wgs;
    uint32_t pad[62];
    CoopSlot slot[kCoopSlots];
};

struct KArgs {
    const void* logits;
    int64_t lstride;
    int B, V;
    const float* temperature;
    const int32_t* top_k;
    const float* top_p;
    const float* min_p;
    const float* rep;
    const float* pres;
    const float* freq;
    const int32_t* prompt;
    int64_t pstride;
    int pwidth;
    const int32_t* plens;
    const int32_t* output;
    int64_t ostride;
    int owidth;
    const int32_t* olens;
    // per-request token state instead of the history lists (or null): word t of table row
    // trows[r] (r when trows is null) = prompt flag (bit 31) | output occurrences of token t
    const uint32_t* tstate;
    int64_t tstride;
    const int32_t* trows;
    const uint32_t* tbits;     // bitmap of the table's non-zero words (same rows), or null
    int64_t tbstride;
    const uint32_t* allowed;   // [B, astride] words, bit set = token allowed (or null)
    int64_t astride;
    const int32_t* adj_ids;    // [B, adjstride] sparse processor list (or null)
    const float* adj_vals;
    int64_t adjstride;
    int adjwidth;
    const int32_t* adjlens;
    const float* u;
    int64_t ustride;
    const uint64_t* rng_seed;   // [B] keys of the generated uniforms (when u is NULL)
    const uint64_t* rng_offset; // [B] their counter offsets, or NULL (0)
    int32_t* sampled;
    uint32_t* flags;
    int32_t* nkept;
    int L;
    int32_t* lp_ids;
    float* lp_vals;
    int32_t* lp_ranks;
    // workspace views
    uint32_t* row_counter;  // [B]
    uint32_t* row_state;    // [B]
    uint32_t* part_meta;    // [B * kMaxParts * 4]: count, kth key, status, 0
    uint2* part_list;       // [B * kMaxParts * kPartCap]: (key, index)
    uint32_t* hist_hash;    // [B * hs_row * 4]: token+1, count | flags, penalised bits, bias
    int hs_row;             // history hash slots per row (power of two) or 0
    int S;                  // parts per row
    int part_len;           // elements per part (multiple of 64)
    int nofast;             // no row takes the single pass (vws_set_single_pass(0))
    int topk_k;             // k of the top-k operation
    float softcap;          // > 0: Gemma's soft cap applied to every logit first
    float inv_softcap;      // fl(1 / softcap)
    int softcap_f16;        // capped values rounded as an f16 store
    float* topk_vals;       // [B, k]
    int32_t* topk_ids;      // [B, k]
    CoopState* coop;        // cooperative passes (sampling workspace), or null
    int coop_count;         // B exceeds the workgroups resident at once: count them in coop->wgs
    int coop_wait_polls;    // bound of an owner's wait for the chunks helpers run (>= 0)
    uint64_t* trace;        // trace build: [trace_wgs][VWS_TRACE_SLOTS] phase stamps, or null
    int trace_wgs;
    uint64_t rng_key;       // launch-wide key (u and rng_seed NULL): row r's offset is r
};

// Workspace layout (bytes, 256-aligned sections).
struct WsLayout {
    size_t counter, state, meta, list, coop, hash, total;
    int hs_row;
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

inline int hash_slots_for(int history_width) {
    if (history_width <= 0) return 0;
    int s = 64;
    while (s < 2 * history_width) s <<= 1;
    return s;
}

// Workspace sections.  Every layout starts with the cooperative-pass region at offset 0, so that
// one workspace can serve every operation in turn (the region keeps its state between sampling
// calls; the other operations leave it alone).  Then: sampling and the penalty op, the history
// hash of the multi-pass path (B x hs_row x 4 words); the split top-k op (parts = true), its
// per-row counters, row states and part lists.
inline WsLayout ws_layout(int B, int V, int history_width, bool parts) {
    (void)V;
    WsLayout w{};
    size_t off = 0;
    w.coop = off;    off = align256(off + sizeof(CoopState));
    if (parts) {
        w.counter = off; off = align256(off + sizeof(uint32_t) * (size_t)B);
        w.state = off;   off = align256(off + sizeof(uint32_t) * (size_t)B);
        w.meta = off;    off = align256(off + sizeof(uint32_t) * 4 * (size_t)B * kMaxParts);
        w.list = off;    off = align256(off + sizeof(uint2) * (size_t)B * kMaxParts * kPartCap);
    }
    w.hs_row = parts ? 0 : hash_slots_for(history_width);
    w.hash = off;    off = align256(off + sizeof(uint32_t) * 4 * (size_t)B * (size_t)w.hs_row);
    w.total = off;
    return w;
}

}  // namespace vws
