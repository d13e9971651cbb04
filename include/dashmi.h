/* dashmi: the MI355X (gfx950) attention and gated-delta-rule hot path behind a C ABI.
 *
 * Each entry point replaces one operation of dash-ops' backend-extension traits, which the
 * reference's callers (dash-mag's Arm, dash-conformance's Adapter) reach through:
 *
 *   dm_attention_fwd     AttentionBackend::attention_forward   crates/dash-ops/src/attention.rs:289-352
 *                        (public fn attention_with_lse          crates/dash-ops/src/attention.rs:660)
 *   dm_attention_bwd     AttentionBackend::attention_backward   crates/dash-ops/src/attention.rs:689
 *   dm_attention_decode  AttentionBackend::attention_decode     crates/dash-ops/src/attention.rs:732
 *   dm_attention_decode_paged  (none: the decode over a paged cache)
 *   dm_gdr_chunk_fwd     ChunkGatedDeltaBackend::chunk_gated_delta_forward
 *                                                               crates/dash-ops/src/gated_delta/chunk.rs:340-425, :856
 *   dm_gdr_chunk_bwd     ChunkGatedDeltaBackend::chunk_gated_delta_backward (the Autodiff node's
 *                        backward, chunk.rs:542-767, as an explicit entry point)
 *   dm_gdr_step          GatedDeltaStepBackend::gated_delta_step crates/dash-ops/src/gated_delta/recurrent.rs:52-81, :158
 *   dm_gdr_step_bwd      the tracked step's gradients (recurrent.rs:89-130: the reference under
 *                        autodiff), as an explicit entry point
 *   dm_causal_conv1d_fwd     CausalConv1dBackend::causal_conv1d  crates/dash-ops/src/conv1d.rs:198-300, :690
 *   dm_causal_conv1d_bwd     CausalConv1dBackend::causal_conv1d_backward
 *                                                               crates/dash-ops/src/conv1d.rs:300-329
 *   dm_causal_conv1d_update  CausalConv1dBackend::causal_conv1d_update
 *                                                               crates/dash-ops/src/conv1d.rs:331-360, :750
 *   dm_chosen_logprob    ChosenLogprobBackend::chosen_logprob{,_with_grad}
 *                                                               crates/dash-ops/src/logprob.rs:127-160
 *   dm_linear_cross_entropy_fwd  LinearCrossEntropyBackend::linear_cross_entropy
 *                                                               crates/dash-ops/src/loss.rs:134-160
 *   dm_linear_cross_entropy_bwd  LinearCrossEntropyBackend::linear_cross_entropy_backward
 *                                                               crates/dash-ops/src/loss.rs:157-200
 *
 * Conventions (crates/dash-contract/src/lib.rs:38-91):
 *   - Every tensor is a device pointer to an array in the contract's layout: [B, T, H, D] for
 *     queries/keys/values/outputs, [B, T, H] for lse, g and beta, [S, H, Dk, Dv] f32 for
 *     states. Outputs are contiguous (freshly allocated by the caller, as the reference's are).
 *     The attention, decode and chunked gated-delta-rule inputs may be strided views (a slice
 *     of one fused projection, a [B, H, T, D] tensor seen through a permutation): with
 *     `strided` set in the descriptor, each such input's (batch, time, head) strides in
 *     elements are given and its last dimension is contiguous; the kernels read it in place
 *     (crates/dash-ops/src/attention.rs:85-93, attention/cube.rs:428-461). The fast kernels
 *     take strides that are multiples of 16 bytes and 16-byte aligned bases (other calls run
 *     the generic kernels, which take any), except the chunked gated delta rule: a bf16/f16
 *     call whose heads are multiples of 8 wide (up to 128) is refused unless q, k, v, d_out
 *     and its 16-bit outputs are 16-byte aligned. Without `strided`, every input is contiguous.
 *   - Floating inputs of a call share one dtype (dm_dtype); lse and states are f32; g and beta
 *     of the gated delta rule may each be f32 or the inputs' dtype.
 *   - Sequence boundaries (cu_seqlens) and cache lengths are int32 device arrays.
 *   - A call outside the contract is refused before any launch: the call returns
 *     DM_ERR_REFUSED and dm_last_error() holds "<operation>: <reason>" (thread-local).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL for the default stream) and nothing
 *     synchronises the host, except where stated.
 *   - Scratch memory is the caller's: each entry point that needs any has a *_workspace query
 *     returning the bytes it needs, and takes that buffer (device memory, 256-byte aligned).
 */
#ifndef DASHMI_H
#define DASHMI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DM_OK 0
#define DM_ERR_REFUSED 1 /* outside the contract, or an input this library does not take */
#define DM_ERR_HIP 2     /* a HIP runtime error */

#define DM_UNBOUNDED UINT64_MAX /* a window side that does not bind (usize::MAX) */

typedef enum { DM_F32 = 0, DM_BF16 = 1, DM_F16 = 2 } dm_dtype;

typedef enum {
    DM_MASK_NONE = 0,        /* every key */
    DM_MASK_KEY_PADDING = 1, /* uint8 [B, Tk], nonzero where a key is left out */
    DM_MASK_PACKED = 2       /* cu_seqlens_q, cu_seqlens_k int32 [nseq + 1], B = 1 */
} dm_mask_kind;

/* AttentionOptions (crates/dash-contract/src/attention.rs:83-115). */
typedef struct {
    int32_t causal;
    int32_t has_scale; /* 0: scale = 1/sqrt(D) */
    float scale;
    int32_t has_window;
    uint64_t window_left, window_right; /* DM_UNBOUNDED for an open side */
    int32_t deterministic;              /* 1: the query gradient in a fixed summation order */
} dm_attention_options;

/* An input's strides in elements along (batch, time, head); its last dimension is contiguous. */
typedef struct {
    int64_t b, t, h;
} dm_strides;

/* One attention call's shapes, dtype and mask (check_shapes, attention.rs:551-590). */
typedef struct {
    int64_t b, tq, tk, hq, hkv, d;
    int32_t dtype; /* dm_dtype of q, k, v, o, d_o and the gradients */
    int32_t mask_kind;
    const uint8_t *key_padding;
    const int32_t *cu_seqlens_q, *cu_seqlens_k;
    int64_t nseq;
    dm_attention_options options;
    /* 0: every input contiguous. 1: the strides below (each >= 0). Decode reads sq.b and sq.h
     * of q [B, Hq, D], and of the cache sk/sv: dense [B, S, Hkv, D] (b, t, h); packed
     * [N, Hkv, D] (t, h; b unused); paged [P, page_size, Hkv, D] (b = the page stride). */
    int32_t strided;
    dm_strides sq, sk, sv, so, sdo; /* q, k, v; the backward's o and d_o */
} dm_attention_desc;

/* The gated delta rule's shapes and options (chunk.rs:771 check_inputs, recurrent.rs:258). */
typedef struct {
    int64_t b, t, h, dk, dv;  /* step: b = rows (tokens), t = 1 */
    int32_t dtype;            /* q, k, v, the output and their gradients */
    int32_t g_dtype;          /* DM_F32 or dtype */
    int32_t beta_dtype;       /* DM_F32 or dtype */
    const int32_t *cu_seqlens; /* packed: [nseq + 1] over a batch of one; NULL: a sequence per row */
    int64_t nseq;
    int32_t qk_l2norm;
    int32_t has_scale;
    float scale;
    /* 0: every input contiguous. 1: the strides below (elements, each >= 0) along (batch, time,
     * head) of q, k, v [B, T, H, D] (the step: [B, H, D], t unused), g and beta [B, T, H], and
     * the backward's d_out. The kernels index tokens as the flattened b * T + t, so each b
     * stride must be T times the t stride (or B = 1); calls whose strides are not of that form
     * are refused (the caller copies them). */
    int32_t strided;
    dm_strides sq, sk, sv, sg, sbeta, sdo;
} dm_gdr_desc;

/* The causal conv1d's activation (crates/dash-contract/src/conv1d.rs:81-90). */
typedef enum { DM_ACT_NONE = 0, DM_ACT_SILU = 1 } dm_activation;
/* One causal conv1d call's shapes and options (conv1d.rs:774-820 check_parameters/check_state;
 * the contract's CausalConv1dOptions, crates/dash-contract/src/conv1d.rs:92-140): x [B, T, C],
 * weight [C, K], bias [C], states [S, W, C] f32. The step: x [B, C], state [B, w, C]. */
typedef struct {
    int64_t b, t, c, k;
    int32_t dtype;             /* x, weight, bias, the output and their gradients */
    const int32_t *cu_seqlens; /* packed: [nseq + 1] over a batch of one; NULL: a sequence per row */
    int64_t nseq;
    int32_t has_bias;
    int32_t activation;        /* dm_activation */
    int32_t has_initial;       /* initial states of w steps (w >= K - 1); the step's state length */
    int64_t w;
    int32_t has_final;         /* final states of w_out steps */
    int64_t w_out;
} dm_conv1d_desc;

/* One chosen-token log-probability call (crates/dash-contract/src/logprob.rs:17-56): hidden
 * [n, D], weight [V, D], each DM_BF16 or DM_F32 (bf16 arithmetic where both are bf16, else both
 * taken as f32); LogprobOptions (logprob.rs:33-56): vocab_chunk tokens per chunk (0: this
 * implementation's own choice, 8192; dash-ops' is 4096 below 2304 rows,
 * crates/dash-ops/src/logprob.rs:90-101), row_chunk the most rows per block (at least 1;
 * dash-ops' default 3072). A vocab_chunk above 8192 is walked 8192 tokens at a time (the
 * statistics kernel holds one chunk's logits in registers), so the order of the online sums is
 * that of 8192-token chunks; results stay within the contract's bounds either way. */
typedef struct {
    int64_t n, v, d;
    int32_t hidden_dtype, weight_dtype;
    int64_t vocab_chunk, row_chunk;
} dm_logprob_desc;

/* One fused linear cross-entropy call (crates/dash-contract/src/loss.rs:52-95): the
 * log-probability's shapes and chunks (hidden and weight of one dtype: f32, bf16 or f16) and
 * CrossEntropyOptions but the reduction and the masked ids: ignore_index (torch's -100 by
 * default), label_smoothing eps in 0..=1, z_loss lambda >= 0, entropy (whether the entropy takes
 * a gradient). */
typedef struct {
    dm_logprob_desc lp;
    int64_t ignore_index;
    float label_smoothing, z_loss;
    int32_t entropy;
} dm_lce_desc;

/* The message of this thread's last refusal or error. */
const char *dm_last_error(void);

/* Device buffers and copies, for a caller that binds no HIP API of its own (the uploads and
 * read-backs of the reference's adapter, crates/dash-ops/tests/common/adapter.rs:140-154, which a
 * Rust -sys crate would otherwise take from a HIP binding). dm_device_alloc returns 256-byte
 * aligned device memory (*ptr = NULL for bytes = 0); the copies are enqueued on `stream` (NULL:
 * the default stream) and have completed when they return; dm_stream_synchronize waits for
 * every launch enqueued on `stream`. */
int dm_device_alloc(size_t bytes, void **ptr);
int dm_device_free(void *ptr);
int dm_copy_to_device(void *dst, const void *src, size_t bytes, void *stream);
int dm_copy_to_host(void *dst, const void *src, size_t bytes, void *stream);
int dm_stream_synchronize(void *stream);

/* Library and device facts: "gfx950, 256 CUs, ..." (the capability probe of
 * crates/dash-ops/src/cube.rs:27-151). Returns DM_OK, or DM_ERR_REFUSED on a device the kernels
 * are not built for. */
int dm_describe(char *buf, size_t len);

/* Launch counters, the probes of attention.rs:158-221, chunk.rs:119-163 and recurrent.rs:41-50:
 * how many kernels of each kind this process launched. */
typedef enum {
    DM_PROBE_ATTN_FWD_MFMA = 0,
    DM_PROBE_ATTN_FWD_GENERIC,
    DM_PROBE_ATTN_BWD_MFMA,
    DM_PROBE_ATTN_BWD_GENERIC,
    DM_PROBE_DECODE_SPLIT,
    DM_PROBE_DECODE_MERGE,
    DM_PROBE_GDR_CHUNK_FWD,
    DM_PROBE_GDR_CHUNK_BWD,
    DM_PROBE_GDR_STEP,
    DM_PROBE_CONV1D_FWD,
    DM_PROBE_CONV1D_BWD,
    DM_PROBE_CONV1D_UPDATE,
    DM_PROBE_LOGPROB,
    DM_PROBE_LCE_FWD,
    DM_PROBE_LCE_BWD,
    DM_PROBE_GDR_CHUNK_FWD_MFMA, /* the MFMA kernels of the chunked forward (a subset of the above) */
    DM_PROBE_GDR_CHUNK_BWD_MFMA, /* the MFMA kernels of the chunked backward */
    DM_PROBE_GDR_STEP_BWD,       /* the recurrent step's backward */
    DM_PROBE_COUNT
} dm_probe;
uint64_t dm_probe_count(int probe);
void dm_probe_reset(void);

/* Kernel timers (no counterpart in the reference; a measurement hook for benchmarks and
 * profilers): while enabled, the library records a HIP event pair around each launch of the
 * kernels below, on the stream it launches them on. dm_kernel_time waits for the recorded events
 * and returns the summed duration in ms and the launch count since timing was last enabled. */
typedef enum {
    DM_KERNEL_ATTN_FWD = 0,   /* MFMA attention forward */
    DM_KERNEL_ATTN_BWD_DKDV,  /* MFMA attention backward, dk and dv */
    DM_KERNEL_ATTN_BWD_DQ,    /* MFMA attention backward, dq */
    DM_KERNEL_DECODE_SPLIT,   /* decode, pass 1 */
    DM_KERNEL_GDR_PREP,       /* chunked gated delta rule: per-chunk preparation */
    DM_KERNEL_GDR_STATE,      /* chunked gated delta rule: the state pass */
    DM_KERNEL_GDR_OUTPUT,     /* chunked gated delta rule: the output (generic f32 kernels) */
    DM_KERNEL_GDR_STEP,       /* gated delta rule step */
    DM_KERNEL_GDR_BWD_PRE,    /* chunked gated delta rule backward: per-chunk state-gradient terms */
    DM_KERNEL_GDR_BWD_STATE,  /* chunked gated delta rule backward: the state-gradient pass */
    DM_KERNEL_GDR_BWD_GRADS,  /* chunked gated delta rule backward: per-chunk gradients */
    DM_KERNEL_CONV1D_FWD,     /* causal conv1d forward */
    DM_KERNEL_CONV1D_BWD,     /* causal conv1d backward: the input gradient and the partial sums */
    DM_KERNEL_CONV1D_UPDATE,  /* causal conv1d decoding step */
    DM_KERNEL_LOGPROB_STATS,  /* chosen-token log-probability: the per-chunk statistics */
    DM_KERNEL_DECODE_MERGE,   /* decode, pass 2: the splits merged by log-sum-exp */
    DM_KERNEL_GDR_STEP_BWD,   /* gated delta rule step backward (both of its kernels) */
    DM_KERNEL_COUNT
} dm_kernel;
int dm_kernel_timing(int enable);
int dm_kernel_time(int kernel, double *ms, uint64_t *launches);

/* The keys query `i` of batch row `b` sees, as the half-open interval [*lo, *hi) of key indices
 * (empty when *lo >= *hi), before key padding, which is per key: the closed form of
 * crates/dash-ops/src/attention/kernels.rs:416-523 (row_bounds, query_range) and of the
 * reference's materialised mask, reference.rs:163-272. Host-only; reads host copies of the
 * offsets (desc->cu_seqlens_* must point to host memory for this call). */
int dm_attention_row_bounds(const dm_attention_desc *desc, int64_t b, int64_t i, int64_t *lo,
                            int64_t *hi);

/* Attention forward: o [B, Tq, Hq, D] in dtype, lse [B, Tq, Hq] f32 (natural log, -inf for a
 * query that sees no key, whose output is 0). Replaces attention.rs:660 / cube.rs:562. */
size_t dm_attention_fwd_workspace(const dm_attention_desc *desc);
int dm_attention_fwd(const dm_attention_desc *desc, const void *q, const void *k, const void *v,
                     void *o, float *lse, void *workspace, size_t workspace_bytes, void *stream);

/* Attention backward from the forward's o and lse and the output's gradient d_o: dq, dk, dv in
 * dtype (dk, dv summed over each key-value head's group). Replaces attention.rs:689 /
 * cube.rs:850. */
size_t dm_attention_bwd_workspace(const dm_attention_desc *desc);
int dm_attention_bwd(const dm_attention_desc *desc, const void *q, const void *k, const void *v,
                     const void *o, const float *lse, const void *d_o, void *dq, void *dk,
                     void *dv, void *workspace, size_t workspace_bytes, void *stream);

/* Decoding: q [B, Hq, D] against the cache k, v [B, S, Hkv, D], sequence b holding its first
 * lengths[b] keys (all S when lengths is NULL); the options' scale and window left apply.
 * o [B, Hq, D] in dtype. Replaces attention.rs:732 / cube.rs:1126. `desc->tq` is unused,
 * desc->tk is S.
 * A packed cache (desc->cu_seqlens_k set, desc->nseq = B): k, v [N, Hkv, D], sequence b's keys in
 * rows cu_seqlens_k[b] .. cu_seqlens_k[b + 1] - 1, the first lengths[b] of them (all when
 * lengths is NULL), at most desc->tk = S of them (S bounds every sequence's span). The contract
 * has only the dense form (crates/dash-contract/src/attention.rs:61-71); the packed form is the
 * same operation over a cache that keeps each sequence's rows at an offset, and a dense cache is
 * the packed one with offsets b * S. */
size_t dm_attention_decode_workspace(const dm_attention_desc *desc);
int dm_attention_decode(const dm_attention_desc *desc, const void *q, const void *k,
                        const void *v, const int32_t *lengths, void *o, void *workspace,
                        size_t workspace_bytes, void *stream);

/* dm_attention_decode without a workspace and without allocating (no counterpart in the
 * reference): for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The split pass's partials go to a
 * static device array of 16 MiB per GPU, held until the process ends; a call whose
 * dm_attention_decode_workspace exceeds 16 MiB is refused (about 64 sequences x 32 query heads
 * x 16 splits at D = 128). Every call on one GPU shares that array: calls that overlap on one GPU
 * (concurrent streams or threads) race, and so do replays of graphs that captured it. The
 * first call on a device looks up that device's array (hipGetSymbolAddress): make it outside
 * graph capture. Same arguments, results and refusals as dm_attention_decode otherwise (dense
 * or packed cache). */
int dm_attention_decode_noalloc(const dm_attention_desc *desc, const void *q, const void *k,
                                const void *v, const int32_t *lengths, void *o, void *stream);

/* Decoding against a paged cache (no counterpart in the reference, whose decode takes the dense
 * cache of crates/dash-contract/src/attention.rs:61-71; this is the same operation, with the
 * dense cache's key j of sequence b stored at row j % page_size of page
 * block_table[b * max_pages + j / page_size]): k_pages, v_pages [num_pages, page_size, Hkv, D],
 * block_table [B, max_pages] int32, lengths [B] int32 or NULL (all max_pages * page_size keys).
 * desc->tk must be max_pages * page_size; desc->cu_seqlens_k must be NULL. Only the pages that
 * hold visible keys are read. A page index outside [0, num_pages) for a visible key reads as
 * zeros (a wrong result, never an access outside the pages). D = 128 with pages of a multiple of
 * 16 keys runs the split pass on MFMA; other shapes run the generic kernel. */
size_t dm_attention_decode_paged_workspace(const dm_attention_desc *desc, int64_t page_size);
int dm_attention_decode_paged(const dm_attention_desc *desc, const void *q, const void *k_pages,
                              const void *v_pages, int64_t num_pages, int64_t page_size,
                              const int32_t *block_table, int64_t max_pages,
                              const int32_t *lengths, void *o, void *workspace,
                              size_t workspace_bytes, void *stream);

/* The chunked gated delta rule forward: out [B, T, H, Dv] in dtype and, if final_state is not
 * NULL, each sequence's final state [S, H, Dk, Dv] f32; h0 [S, H, Dk, Dv] f32 or NULL (zeros).
 * Replaces chunk.rs:856 / chunk/cube.rs:4757. */
size_t dm_gdr_chunk_fwd_workspace(const dm_gdr_desc *desc);
int dm_gdr_chunk_fwd(const dm_gdr_desc *desc, const void *q, const void *k, const void *v,
                     const void *g, const void *beta, const float *h0, void *out,
                     float *final_state, void *workspace, size_t workspace_bytes, void *stream);

/* Its backward: from d_out [B, T, H, Dv] (dtype) and d_final [S, H, Dk, Dv] f32 (NULL: zeros),
 * the gradients dq, dk [B, T, H, Dk], dv (dtype), dg (g_dtype), dbeta (beta_dtype) and
 * dh0 [S, H, Dk, Dv] f32 (NULL: not wanted). Replaces chunk.rs:545 / chunk/cube.rs:3623. */
size_t dm_gdr_chunk_bwd_workspace(const dm_gdr_desc *desc);
int dm_gdr_chunk_bwd(const dm_gdr_desc *desc, const void *q, const void *k, const void *v,
                     const void *g, const void *beta, const float *h0, const void *d_out,
                     const float *d_final, void *dq, void *dk, void *dv, void *dg, void *dbeta,
                     float *dh0, void *workspace, size_t workspace_bytes, void *stream);

/* The recurrent step: rows q, k [B, H, Dk], v [B, H, Dv], g, beta [B, H] advance the states
 * [S, H, Dk, Dv] f32 (S = B, or cu_seqlens' sequences token by token); out [B, H, Dv] in
 * dtype. state_out may equal state_in (in place). Replaces recurrent.rs:158 /
 * recurrent/kernel.rs:294. */
int dm_gdr_step(const dm_gdr_desc *desc, const void *q, const void *k, const void *v,
                const void *g, const void *beta, const float *state_in, float *state_out,
                void *out, void *stream);

/* The step's backward: from d_out [B, H, Dv] (dtype; NULL: zeros) and d_state, the new states'
 * gradient [S, H, Dk, Dv] f32 (NULL: zeros), the gradients dq, dk [B, H, Dk], dv [B, H, Dv]
 * (dtype), dg (g_dtype), dbeta (beta_dtype) [B, H] and d_state_in [S, H, Dk, Dv] f32 (NULL: not
 * wanted), all contiguous. The reference's tracked step runs its reference under autodiff
 * (recurrent.rs:89-130, the operations of :362-404); dash-conformance holds the gradients to
 * torch's (crates/dash-conformance/src/gated_delta_recurrent.rs:229-269,
 * gated_delta_packed.rs:419-517). The workspace holds, with cu_seqlens, the state before every
 * token ([B, H, Dk, Dv] f32: packed tokens are walked in reverse), plus per-token partial sums. */
size_t dm_gdr_step_bwd_workspace(const dm_gdr_desc *desc);
int dm_gdr_step_bwd(const dm_gdr_desc *desc, const void *q, const void *k, const void *v,
                    const void *g, const void *beta, const float *state_in, const void *d_out,
                    const float *d_state, void *dq, void *dk, void *dv, void *dg, void *dbeta,
                    float *d_state_in, void *workspace, size_t workspace_bytes, void *stream);

/* The causal depthwise conv1d over sequences: out [B, T, C] in dtype and, with has_final, each
 * sequence's final state (the last w_out steps of its history) [S, w_out, C] f32; with
 * has_initial, each sequence continues from initial_state [S, w, C] f32. Replaces
 * conv1d.rs:690 / CausalConv1dBackend::causal_conv1d. Kernel widths up to 16. */
int dm_causal_conv1d_fwd(const dm_conv1d_desc *desc, const void *x, const void *weight,
                         const void *bias, const float *initial_state, void *out,
                         float *final_state, void *stream);
/* Its gradients from the output's (grad_out [B, T, C], grad_out_dtype f32 or dtype) and, with
 * has_final, the final states' (grad_final_state [S, w_out, C] f32, or NULL for zeros): grad_x
 * [B, T, C] and grad_weight [C, K] in dtype, grad_bias [C] in dtype with has_bias,
 * grad_initial_state [S, w, C] f32 with has_initial. The weight's and the bias's gradients are
 * summed in a fixed order (deterministic). Replaces CausalConv1dBackend::causal_conv1d_backward
 * (conv1d.rs:300-329), the Autodiff node's backward as an explicit entry point. */
size_t dm_causal_conv1d_bwd_workspace(const dm_conv1d_desc *desc);
int dm_causal_conv1d_bwd(const dm_conv1d_desc *desc, const void *x, const void *weight,
                         const void *bias, const float *initial_state, const void *grad_out,
                         int grad_out_dtype, const float *grad_final_state, void *grad_x,
                         void *grad_weight, void *grad_bias, float *grad_initial_state,
                         void *workspace, size_t workspace_bytes, void *stream);
/* One decoding step: x [B, C] (desc->b = B, desc->w = the state's steps W >= K - 1) and state
 * [B, W, C] f32 to out [B, C] in dtype and next_state [B, W, C] f32 (the state without its oldest
 * step, then x; next_state may be state itself). Replaces conv1d.rs:750 /
 * CausalConv1dBackend::causal_conv1d_update. */
int dm_causal_conv1d_update(const dm_conv1d_desc *desc, const void *x, const void *weight,
                            const void *bias, const float *state, void *out, float *next_state,
                            void *stream);

/* The chosen-token log-probability and entropy (crates/dash-contract/src/logprob.rs:4-15):
 * logits z = hidden weight^T over the vocabulary minus the masked ids, never all held;
 * logprob [n] f32 = z[t] - logsumexp z (-inf where the target is masked or outside [0, V)),
 * entropy [n] f32; with grad (not NULL), grad [n, D] f32 = d logprob[i] / d hidden[i], which the
 * caller scales by the upstream gradient (the backward of logprob.rs:160-190). targets [n] int64
 * on the device; masked: n_masked token ids on the HOST (the reference's Vec<u32>), any order,
 * each below V, at least one token left unmasked. Replaces ChosenLogprobBackend::chosen_logprob
 * and chosen_logprob_with_grad (logprob.rs:127-160). The logits' and the gradient's products
 * run as hipBLASLt GEMMs on the stream; the online log-sum-exp between them as this library's
 * kernels. vocab_chunk 0 walks 8192 tokens a chunk, and wider chunks are walked 8192 tokens at a
 * time. D must be a multiple of 8. */
size_t dm_chosen_logprob_workspace(const dm_logprob_desc *desc, int with_grad);
int dm_chosen_logprob(const dm_logprob_desc *desc, const void *hidden, const void *weight,
                      const int64_t *targets, const uint32_t *masked, int64_t n_masked,
                      float *logprob, float *entropy, float *grad, void *workspace,
                      size_t workspace_bytes, void *stream);

/* The fused linear cross-entropy (crates/dash-contract/src/loss.rs:1-50), forward: rows [8, n]
 * f32 per row = loss, logprob, entropy (each 0 on an ignored row; loss +inf and logprob -inf
 * where the target is masked or outside [0, V)), lse, q = 1 - p(target) summed over the other
 * tokens, s, counted, found (crates/dash-ops/src/loss.rs:96-116). The caller reduces the loss row
 * (mean over the counted rows, sum, or none, loss.rs:872-877). targets [n] int64 on the device;
 * masked: n_masked ids on the HOST, any order, each below V, at least one token left. Replaces
 * LinearCrossEntropyBackend::linear_cross_entropy (loss.rs:134-160; the written-out backward is
 * always taken, as with a weight that trains). The workspace query's `backward`: 0 for the
 * forward, 1 for a backward with both gradients, 2 for a backward without grad_weight (a frozen
 * output weight: no V x D f32 accumulator is reserved; the backward then refuses a non-NULL
 * grad_weight with that smaller workspace). */
size_t dm_linear_cross_entropy_workspace(const dm_lce_desc *desc, int backward);
int dm_linear_cross_entropy_fwd(const dm_lce_desc *desc, const void *hidden, const void *weight,
                                const int64_t *targets, const uint32_t *masked, int64_t n_masked,
                                float *rows, void *workspace, size_t workspace_bytes,
                                void *stream);
/* Its backward from the forward's rows and upstream [3, n] f32 (the gradients of the loss,
 * logprob and entropy rows; the entropy's is read only with desc->entropy): grad_hidden [n, D]
 * and grad_weight [V, D] in the inputs' dtype, either NULL when not wanted. A second pass over
 * the vocabulary recomputes each chunk's logits; the logits' gradient is rounded to bf16 for the
 * products from bf16 inputs. Replaces LinearCrossEntropyBackend::linear_cross_entropy_backward
 * (loss.rs:157-200). */
int dm_linear_cross_entropy_bwd(const dm_lce_desc *desc, const void *hidden, const void *weight,
                                const int64_t *targets, const uint32_t *masked, int64_t n_masked,
                                const float *rows, const float *upstream, void *grad_hidden,
                                void *grad_weight, void *workspace, size_t workspace_bytes,
                                void *stream);

#ifdef __cplusplus
}
#endif
#endif
