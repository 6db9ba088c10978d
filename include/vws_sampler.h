/*
 * vws_sampler.h -- C ABI of the MI355X (gfx950) token-sampling library
 * (vllm_webgpu_amd/_vws.so).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed as void*.
 * Nothing here allocates device memory: callers own every buffer, including the workspace.
 * Work is enqueued on the given stream with no host synchronisation; the return value only
 * reports argument errors and launch failures.  On error, vws_last_error() gives a
 * thread-local message.
 *
 * Reference interfaces each entry point replaces (paths under the vllm_webgpu reference):
 *   vws_sample   <- vllm_webgpu/v1/model_runner.py:139-166 (execute_model's host argmax at :145
 *                   and the sample_tokens() stub at :164-166) and run_inference.py:383-390
 *                   (greedy / temperature sampling in the CLI); semantics of the vLLM-v1
 *                   Sampler the plugin delegates to (docs/.../2026-06-29-vllm-webgpu-design.md:451)
 *   vws_argmax   <- vllm_webgpu/shaders/generic/argmax.wgsl:1-60, dispatched as in
 *                   tests/test_kernels_sample.py:8-43 (batched here: [B, V] -> [B])
 *   vws_topk     <- vllm_webgpu/shaders/generic/topk256.wgsl:1-70, dispatched as in
 *                   tests/test_kernels_sample.py:46-101 (batched, K <= 256 as in topk256, no mask buffer)
 *   vws_softmax  <- vllm_webgpu/shaders/generic/softmax.wgsl:1-71 (row softmax; here with a
 *                   per-row temperature as in run_inference.py:386-389, plus max and log-sum)
 *   vws_apply_penalties <- the vLLM-v1 penalty step the plugin inherits (no WGSL counterpart)
 */
#ifndef VWS_SAMPLER_H
#define VWS_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VWS_ABI_VERSION 8

/* status codes */
#define VWS_OK 0
#define VWS_ERR_INVALID_ARGUMENT 1
#define VWS_ERR_UNSUPPORTED_DTYPE 2
#define VWS_ERR_WORKSPACE_TOO_SMALL 3
#define VWS_ERR_HIP 4
#define VWS_ERR_LIMIT 5
#define VWS_ERR_UNSUPPORTED 6   /* a call only the trace build serves (vws_trace_set) */

/* logits element types */
#define VWS_DTYPE_F32 0
#define VWS_DTYPE_BF16 1
#define VWS_DTYPE_F16 2  /* IEEE binary16 (the reference's f16 logits), widened exactly */

/* per-row result flags (vws_sample_args.row_flags) */
#define VWS_FLAG_TOPP_NEAR_TIE 0x1u  /* top-p cumulative mass within 1e-6 of the threshold */
#define VWS_FLAG_RACE_NEAR_TIE 0x2u  /* best and second race keys within 1e-6 (relative) */
#define VWS_FLAG_DEGENERATE 0x4u     /* row maximum not finite: greedy over y = x / T */
#define VWS_FLAG_GREEDY 0x8u         /* temperature < 1e-5 (or NaN): argmax of penalised x */
#define VWS_FLAG_GENERAL_PATH 0x100u /* served by the multi-pass kernel (diagnostic only) */
#define VWS_FLAG_STREAM_TOPP 0x200u  /* served by the single-pass top-p path (diagnostic only) */
#define VWS_FLAG_TOPP_RECOUNT 0x400u /* ... after an exact pass over its tail (diagnostic only) */
#define VWS_FLAG_TOPP_WIDE 0x800u    /* ... with its nucleus reaching below the candidates: one
                                        more pass races them (diagnostic only) */
/* Bits 16-23 (diagnostic only): why a row left the single-pass top-p path for the multi-pass
 * kernel (1 candidate overflow, 2 non-finite sum, 3 no finite maximum, 6 ambiguous after the
 * exact pass, 7 boundary bucket too large, 8 top-L below the candidates, 9 a pass shared with
 * other workgroups not completed in time; 4 and 5 are no longer used). */

#define VWS_MAX_VOCAB (1 << 19)       /* masses are floor(e * 2^44) summed in 64 bits */
#define VWS_MAX_LOGPROBS 64

typedef struct vws_sample_args {
    uint32_t struct_size; /* sizeof(vws_sample_args): ABI guard */
    int32_t batch;        /* B >= 1 */
    int32_t vocab;        /* 1 <= V <= VWS_MAX_VOCAB */
    int32_t dtype;        /* VWS_DTYPE_* */
    const void* logits;   /* [B, V] with row stride below; read only */
    int64_t logits_row_stride; /* elements */
    /* > 0: the logits are the lm_head output before Gemma's final soft cap, applied here as
     * cap * tanh(x / cap) (vllm_webgpu/models/gemma4.py:158-163, shaders/gemma/
     * logit_softcap.wgsl:13-28; tanh(v) = +-1 for |v| >= 20, else (e - 1) / (e + 1) with
     * e = exp(2v), fp32).  Everything downstream -- processors, penalties, raw logprobs --
     * sees the capped values.  0 = off. */
    float logit_softcap;
    /* Non-zero: each capped value is rounded to f16 (nearest, ties to even) and widened back,
     * as the reference's shader stores it into an f16 buffer (logit_softcap.wgsl:28). */
    int32_t logit_softcap_f16;

    /* Per-row parameters, device arrays of length B.  NULL selects the default:
     * temperature NULL = every row greedy; top_k NULL/<=0/>=V = off; top_p NULL/>=1 = off;
     * min_p NULL/0 = off; repetition NULL = 1; presence/frequency NULL = 0. */
    const float* temperature;
    const int32_t* top_k;
    const float* top_p;
    const float* min_p;
    const float* repetition_penalty;
    const float* presence_penalty;
    const float* frequency_penalty;

    /* Token histories for the penalties: padded int32 [B, width] with the given row stride.
     * Ids outside [0, V) are padding (vLLM pads with V).  *_lens (device, [B]) may be NULL,
     * meaning the full width.  Prompt tokens take the repetition penalty only; output tokens
     * take repetition, frequency (per occurrence) and presence. */
    const int32_t* prompt_ids;
    int64_t prompt_row_stride;
    int32_t prompt_width;
    const int32_t* prompt_lens;
    const int32_t* output_ids;
    int64_t output_row_stride;
    int32_t output_width;
    const int32_t* output_lens;

    /* Per-request token state, instead of the two lists above (optional; prompt_ids and
     * output_ids must then be NULL): uint32 [rows, >= V] with the given row stride (elements);
     * logits row r uses table row token_state_rows[r] (device int32 [B]; NULL = row r).  Word t
     * of a row = 0x80000000 when token t is in the request's prompt, plus the number of times t
     * occurs in its output (< 2^29; bits 29-30 are ignored) -- the prompt mask and output bin
     * counts vLLM-v1 rebuilds from the histories every step (apply_penalties), kept on the
     * device instead (vws_token_state_update).  The single-pass paths read only the words of
     * the tokens that reach a row's candidates, so a history of any length costs the same; the
     * multi-pass path scans the row's words once. */
    const uint32_t* token_state;
    int64_t token_state_row_stride;
    const int32_t* token_state_rows;
    /* Optional with token_state: uint32 [rows, >= ceil(V/32)] (row stride in words, rows as
     * for the table), bit (t & 31) of word t >> 5 set when word t of the table row is non-zero;
     * vws_token_state_update keeps it with the table.  With it, rows whose survivors top-p
     * alone cuts (top-k off) keep the single-pass top-p path with their penalties when
     * V <= 196608 (the bitmap is staged in LDS); without it such rows take the multi-pass
     * path.  NULL otherwise. */
    const uint32_t* token_state_bits;
    int64_t token_state_bits_stride;

    /* vLLM-v1 logits processors, applied before the penalties (raw logprobs never see them).
     * allowed_mask: uint32 [B, ceil(V/32)] words with the given row stride, bit (t & 31) of word
     * t >> 5 set = token t allowed, others become -inf (allowed_token_ids); NULL = all allowed.
     * adjust_ids / adjust_vals: padded [B, width] (shared row stride) sparse per-row list:
     * value -inf bans the token (bad words, min-tokens stop ids), a finite value is added to
     * its logit (logit bias; at most one finite entry per token and row).  Ids outside [0, V)
     * are padding; adjust_lens (device [B]) may be NULL, meaning the full width.  With an
     * allowed mask and no raw logprobs every row is masked as its logits stream in (top-k,
     * greedy and top-p rows alike; rows that do not start 16-byte aligned take the multi-pass
     * path); with raw logprobs (of the unmasked logits) top-k and greedy rows mask their
     * candidates and top-p rows take the multi-pass path. */
    const uint32_t* allowed_mask;
    int64_t allowed_row_stride;
    const int32_t* adjust_ids;
    const float* adjust_vals;
    int64_t adjust_row_stride;
    int32_t adjust_width;
    const int32_t* adjust_lens;

    /* Uniforms in (0, 1), fp32 [B, V] (row stride in elements); read only at surviving
     * tokens.  Required when temperature is non-NULL, unless rng_seeds or rng_key_set is
     * given. */
    const float* uniforms;
    int64_t uniforms_row_stride;
    /* Generated uniforms instead (when uniforms is NULL): device u64 [B] keys and offsets
     * (rng_offsets NULL = 0).  Token t of row r draws word t % 4 of Philox-4x32-10 (Salmon et
     * al., SC 2011) at counter (t / 4, offset lo, offset hi, 0) with key (seed lo, seed hi),
     * as (2 floor(w / 2^9) + 1) 2^-24, evaluated only at the tokens that race.  No [B, V]
     * buffer is read or needs to be written. */
    const uint64_t* rng_seeds;
    const uint64_t* rng_offsets;
    /* Or one key for the whole launch (uniforms and rng_seeds NULL, rng_key_set non-zero): row
     * r generates as with seed rng_key and offset r.  A by-value key: a sampling step needs no
     * upload of per-row keys (no extra copy ahead of the kernel on the stream). */
    uint64_t rng_key;
    int32_t rng_key_set;

    /* Outputs */
    int32_t* sampled;    /* [B] token ids */
    uint32_t* row_flags; /* [B] VWS_FLAG_* or NULL */
    int32_t* num_kept;   /* [B] tokens left with non-zero probability, or NULL */
    int32_t num_logprobs;   /* -1: none.  L >= 0: raw (pre-penalty) logprobs */
    int32_t* logprob_ids;   /* [B, L+1]: sampled id, then top-L ids (value desc, id asc) */
    float* logprob_vals;    /* [B, L+1] */
    int32_t* logprob_ranks; /* [B]: #{j : logprob_j >= logprob_sampled} */

    /* Device scratch, >= vws_sample_workspace_size(); see vws_workspace_init.  Without any
     * history (prompt, output and processor lists all absent or of width 0) it may be NULL or
     * smaller: the launch then runs without the cooperative passes (same results). */
    void* workspace;
    size_t workspace_bytes;
    void* stream; /* hipStream_t */
} vws_sample_args;

/* ABI version (VWS_ABI_VERSION of the built library). */
int32_t vws_abi_version(void);

/* Thread-local description of the last error returned on this thread ("" if none). */
const char* vws_last_error(void);

/* Bytes of workspace vws_sample needs for this shape and history width
 * (prompt_width + output_width + adjust_width): a fixed region (about 530 KiB, first) through
 * which the workgroups of one launch share the extra passes over a row's logits that some
 * top-p rows need, and through which a batch larger than the device's resident workgroups
 * gets its rows handed out; then the history hash of rows served by the multi-pass path,
 * B x (power of two >= 2 x history_width, at least 64) x 16 bytes.  Every operation's
 * workspace starts with that same region (the others leave it alone), so one buffer can serve
 * them all in stream order. */
size_t vws_sample_workspace_size(int32_t batch, int32_t vocab, int32_t history_width);

/* Clears a workspace on `stream` (a fill kernel, safe under graph capture).  Required once
 * after allocation; vws_sample leaves it clean again for the next call. */
int vws_workspace_init(void* workspace, size_t workspace_bytes, void* stream);

/* Host-only argument check (no device access): the status vws_sample would return before
 * launching anything. */
int vws_validate_sample_args(const vws_sample_args* args);

/* Full sampler: penalties -> temperature -> min-p -> top-k -> top-p -> exponential race,
 * plus greedy rows and raw logprobs.  Results are identical, bit for bit, to the CPU oracle
 * in oracle/ for the same inputs. */
int vws_sample(const vws_sample_args* args);

/* vws_sample without a caller workspace, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart
 * in the reference.  `workspace` and `workspace_bytes` are ignored: the scratch is a static
 * device array of VWS_NOALLOC_SCRATCH_BYTES per GPU, looked up and cleared on the first call on
 * each device and held until the process ends.  Batches whose vws_sample_workspace_size exceeds
 * it are rejected with VWS_ERR_LIMIT.  Every call on one GPU shares that GPU's scratch: calls
 * that overlap on one GPU (different streams, no ordering between them) race; calls ordered on
 * one stream do not.  Nothing is allocated, on the host or the device. */
#define VWS_NOALLOC_SCRATCH_BYTES (16 << 20)
int vws_sample_noalloc(const vws_sample_args* args);

/* Token-state table maintenance on `stream` (no counterpart in the reference, which has no
 * sampler state; vLLM-v1 rebuilds the same counts from the histories every step).  For each
 * i < n with 0 <= tokens[i] < vocab: VWS_STATE_OUTPUT adds one output occurrence to word
 * tokens[i] of table row rows[i], VWS_STATE_PROMPT sets that word's prompt flag (atomics: ids and
 * rows may repeat).  rows and tokens are device int32 [n]; rows NULL sends every id to table
 * row `row`.  Ids outside [0, vocab) and negative rows are padding and skipped.  `bits` (or
 * NULL): the table's bitmap of non-zero words (vws_sample_args::token_state_bits, row stride
 * bits_stride >= ceil(vocab/32) words), whose bit of every id updated is set.  A row is cleared
 * by zeroing its words and its bitmap row (the caller's memory). */
#define VWS_STATE_OUTPUT 0
#define VWS_STATE_PROMPT 1
int vws_token_state_update(uint32_t* state, int64_t row_stride, uint32_t* bits,
                           int64_t bits_stride, int32_t vocab, int32_t n, const int32_t* rows,
                           int32_t row, const int32_t* tokens, int32_t kind, void* stream);

/* Greedy argmax of each row (lowest index on ties; NaN never selected). */
int vws_argmax(const void* logits, int32_t dtype, int32_t batch, int32_t vocab,
               int64_t row_stride, int32_t* out_ids, void* stream);

/* Top-k values (as fp32) and ids of each row, ordered (value desc, id asc); 1 <= k <= 256.
 * Needs vws_topk_workspace_size() bytes of workspace (initialised with vws_workspace_init). */
size_t vws_topk_workspace_size(int32_t batch, int32_t vocab, int32_t k);
int vws_topk(const void* logits, int32_t dtype, int32_t batch, int32_t vocab, int64_t row_stride,
             int32_t k, float* out_vals, int32_t* out_ids, void* workspace,
             size_t workspace_bytes, void* stream);

/* probs = softmax(x / T) per row with the sampler's exp; temperature [B] (NULL = 1).
 * row_max [B] (= max x / T) and log_sum [B] (= log sum exp(x/T - max)) may be NULL. */
int vws_softmax(const void* logits, int32_t dtype, int32_t batch, int32_t vocab,
                int64_t row_stride, const float* temperature, float* probs, float* row_max,
                float* log_sum, void* stream);

/* In-place penalties on fp32 logits [B, V] (vLLM-v1 order and arithmetic); history arrays as
 * in vws_sample_args.  Needs vws_sample_workspace_size(B, V, prompt_width + output_width). */
int vws_apply_penalties(float* logits, int32_t batch, int32_t vocab, int64_t row_stride,
                        const float* repetition, const float* presence, const float* frequency,
                        const int32_t* prompt_ids, int64_t prompt_row_stride, int32_t prompt_width,
                        const int32_t* prompt_lens, const int32_t* output_ids,
                        int64_t output_row_stride, int32_t output_width,
                        const int32_t* output_lens, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Test hook (no counterpart in the reference): the bound, in polls of a few dozen cycles each,
 * of a top-p row's wait for the chunks of its shared passes that other workgroups run (default
 * 2^20; process-wide, read by each vws_sample launch).  A row that stops waiting takes the
 * multi-pass path (same results) and leaves its slot to the last of those chunks to finish,
 * which frees it.  0 gives every shared pass up as soon as the row's own chunks are done,
 * finished elsewhere or not, so that tests reach that path whatever the timing.  Returns the
 * previous bound, or -1 (with vws_last_error) for polls < 0. */
int32_t vws_set_coop_wait_polls(int32_t polls);

/* Test hook (no counterpart in the reference): 0 keeps every row of later vws_sample launches
 * off the single pass (greedy and top-k rows take the multi-pass path, top-p rows still the
 * single-pass top-p path), 1 (the default) lets rows take it again; process-wide, read by each
 * launch.  Both paths give the same results, which tests compare.  Returns the previous
 * setting, or -1 (with vws_last_error) for any other value. */
int32_t vws_set_single_pass(int32_t enabled);

/* Per-kernel timing.  vws_profile_begin(n) makes the next n kernel launches of this library
 * (on any stream) carry a hipEvent pair that the runtime stamps when the kernel itself begins
 * and ends (hipExtLaunchKernel; no marker packets between launches, so the sum is the kernels'
 * own durations, as a kernel trace reports them); vws_profile_end() waits for those events,
 * writes the summed milliseconds and launch counts per kernel kind into
 * ms[VWS_KERNEL_KINDS] / count[VWS_KERNEL_KINDS] and turns recording off. */
#define VWS_KERNEL_SAMPLE 0    /* the sampling kernel of vws_sample (one workgroup per row) */
#define VWS_KERNEL_TOPK 1      /* the kernels of vws_topk */
#define VWS_KERNEL_ARGMAX 2
#define VWS_KERNEL_SOFTMAX 3
#define VWS_KERNEL_PENALTIES 4
#define VWS_KERNEL_OTHER 5     /* workspace fill, self-test */
#define VWS_KERNEL_KINDS 6
int vws_profile_begin(int32_t max_launches);
int vws_profile_end(double* ms, int32_t* count);

/* Phase trace of the sampling kernel (no counterpart in the reference: a diagnostic for the
 * people who tune this library).  Only the trace build records (vllm_webgpu_amd/_vws_trace.so,
 * `make -C vllm_webgpu_amd/csrc trace`, the same kernels compiled with -DVWS_TRACE); this build
 * returns VWS_ERR_UNSUPPORTED.  vws_trace_set(buf, max_workgroups) makes every later vws_sample
 * launch of the process write, for each of its first max_workgroups workgroups, the
 * VWS_TRACE_SLOTS 64-bit words buf[wg * VWS_TRACE_SLOTS + slot] (device memory the caller owns
 * and keeps alive): s_memrealtime stamps (a 100 MHz device clock) at the phase boundaries
 * below, by the first thread of the workgroup's last wave, and the XCD and row the workgroup
 * ran.  Each stamp delays the stamping wave by the clock read (the trace build's launches take
 * a few percent longer than the product build's).  A phase a
 * row does not reach keeps whatever the buffer held (clear it first).  vws_trace_set(NULL, 0)
 * turns it off.  Launches that overlap on one buffer overwrite each other's records. */
#define VWS_TRACE_SLOTS 16
#define VWS_TRACE_ENTRY 0    /* the workgroup's first instruction */
#define VWS_TRACE_PARAMS 1   /* single pass: the row's parameters are read (last wave) */
#define VWS_TRACE_FIRST 2    /* single pass: the last wave holds its first iteration */
#define VWS_TRACE_SEED 3     /* the seed threshold is published to every wave */
#define VWS_TRACE_STREAM 4   /* every wave has streamed the row (single pass: and packed its
                                candidates) */
#define VWS_TRACE_ROW 5      /* the row is done (results written, or handed to another path) */
#define VWS_TRACE_EXIT 6     /* the workgroup is done, after any help with other rows' passes */
#define VWS_TRACE_WAVE_LOOP 7 /* single pass: the last wave has examined its share */
#define VWS_TRACE_WAVE_PACK 8 /* single pass: the last wave has packed its candidates */
#define VWS_TRACE_TP_HIST 9   /* top-p path, history rows: every history token is buffered */
#define VWS_TRACE_TP_MASS 10  /* top-p path: the candidates' exact masses are in */
#define VWS_TRACE_TP_CUT 11   /* top-p path: the cut is decided (any further pass run) */
#define VWS_TRACE_TP_RACE 12  /* top-p path: the race is done */
#define VWS_TRACE_TP_LOGPROBS 13 /* top-p path: the raw logprobs are done */
#define VWS_TRACE_XCC 14     /* value: the XCD (XCC id) the workgroup ran on */
#define VWS_TRACE_ROWID 15   /* value: the row the workgroup served */
int vws_trace_set(uint64_t* buf, int32_t max_workgroups);

/* Device self-test of the sampler arithmetic: evaluates fn (0 = exp_det, 1 = log_det,
 * 2 = the logit soft cap at cap 1, i.e. its tanh, 3 = fp32 -> f16 -> fp32 rounding) at
 * every fp32 whose order key lies in [key_lo, key_hi] and accumulates the same 64-bit hash
 * as the CPU oracle's checker into out2[0] and the count into out2[1] (device u64[2],
 * zeroed by this call). */
int vws_math_selftest(int32_t fn, uint32_t key_lo, uint32_t key_hi, uint64_t* out2, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VWS_SAMPLER_H */
