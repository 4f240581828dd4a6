/*
 * sa.h -- C ABI of the MI355X (gfx950) Selective Attention kernels.
 *
 * Selective Attention (Leviathan, Kalman, Matias, ICLR 2025): causal softmax attention whose
 * logits, for every head h, have the running selection F subtracted:
 *
 *     L_h[i,j] = s q_h[i].k_h[j]                     s = 1/sqrt(D), key j <= query i
 *     S[r,j]   = relu(L_0[r,j])   if E <= j < r, else 0      (head 0 of the sequence selects)
 *     F[i,j]   = sum_{r<i} S[r,j]
 *     O_h      = softmax_j(L_h - F) V_h
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t (passed as void*),
 * never allocates, never throws, and returns an int status (0 = ok, < 0 = error; see
 * sa_status_string). The caller owns every buffer. Launches are asynchronous on `stream`.
 *
 * Tensor layouts (row-major, contiguous):
 *   q, k, v, dout            (nseq*heads, T, D)      storage dtype SA_DTYPE_BF16 or SA_DTYPE_F32
 *                                                   (sa_forward's k, v: heads kv_stride apart)
 *   out                      (nseq*heads, Tq, D)     fp32
 *   rmax, rden               (nseq*heads, Tq)        fp32   row max (log2 domain) / denominator
 *   carry                    (nseq, ceil(Tq/32), Tk) fp32   per-key selection on entry to every
 *                                                           32-query block (the reference's CARRY)
 *   state_in / state_out     (nseq, state_ld)        fp32   per-key selection before / after
 * The operand precision follows the storage dtype: bf16 storage runs bf16 MFMA with fp32
 * accumulation; fp32 storage runs fp32 MFMA. Selection, F, softmax statistics and every
 * accumulator are fp32.
 *
 * Per-head selection (every head its own selector) is the caller reshaping (B, H, T, D) to
 * nseq = B*H sequences of heads = 1, as the reference's module does (mixers.py:76-84).
 */
#ifndef SA_H
#define SA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SA_DTYPE_BF16 0
#define SA_DTYPE_F32 1

#define SA_OK 0
#define SA_ERR_ARGUMENT -1      /* a size, pointer or option is invalid */
#define SA_ERR_HEAD_DIM -2      /* head_dim not in {32, 64, 128} */
#define SA_ERR_DTYPE -3         /* dtype code unknown */
#define SA_ERR_WORKSPACE -4     /* workspace smaller than the *_workspace_bytes figure */
#define SA_ERR_LAUNCH -5        /* a kernel launch failed (hipGetLastError) */
#define SA_ERR_SCRATCH -6       /* sa_decode_noalloc: the step needs more than its fixed scratch */

/* ABI revision of this header; bumps when a signature changes or an entry point is added. */
int sa_abi_version(void);

/* Human-readable text for a status code (static storage). */
const char* sa_status_string(int status);

/*
 * Kernel timing for measurement tools; no counterpart in the reference (which times whole calls
 * with perf_counter, scripts/bench_kernels.py:36-58). While enabled, sa_forward and sa_backward
 * record a pair of HIP events on their stream around each of their main kernels (sa_decode too).
 * sa_timing_enable(on) discards what was recorded and switches recording on (1) or off (0).
 * sa_timing_read waits for the recorded events of one kernel and returns the summed duration in
 * milliseconds and the number of launches. Not meant for production paths: the events cost a
 * little time per launch.
 */
#define SA_KERNEL_FORWARD 0     /* the attention forward kernel */
#define SA_KERNEL_BACKWARD 1    /* the key-parallel backward kernel (dK, dV) */
#define SA_KERNEL_SELECTION 2   /* head 0's selection column sums + scan */
#define SA_KERNEL_BACKWARD_DQ 3 /* the query-parallel backward kernel (dQ) */
#define SA_KERNEL_DECODE 4      /* the decode step's cache-reading kernel */
#define SA_KERNEL_COUNT 5
int sa_timing_enable(int on);
int sa_timing_read(int kernel, double* total_ms, int64_t* launches);

/* Leading dimension (elements) of the transposed copies held in the workspaces. */
int64_t sa_transposed_ld(int64_t t);

/* Bytes of scratch sa_forward needs for the same `group` argument: the transposed value copy, or 0
 * for bf16 at head dim 64 with one or two heads per wavefront (the default there), whose kernel
 * reads the value rows themselves (workspace may then be NULL). */
int64_t sa_forward_workspace_bytes(int64_t nseq, int64_t heads, int64_t tk, int64_t head_dim, int dtype, int group);

/*
 * Forward pass, and one chunk of a chunked prefill.
 *
 * Replaces selective_attention_forward's two Triton launches (_selective_carry and
 * _selective_forward[_grouped]), reference src/selective_attention/kernels.py:526-605, and
 * adds the chunk form the reference lacks: queries are the absolute positions
 * [q_offset, q_offset + tq) of a sequence whose keys/values are [0, tk), tk = q_offset + tq.
 * state_in (may be NULL when q_offset == 0) holds, for every key j < q_offset, the selection
 * sum over all queries before q_offset; state_out receives the same sum over all queries
 * before q_offset + tq (for q_offset == 0 it is the reference's `selected_total`,
 * kernels.py:547-549). state_in and state_out may alias.
 *
 * kv_stride: elements between consecutive heads of k and v (0 = tk * head_dim, the contiguous
 * layout); a prefill over a preallocated (nseq, heads, capacity, head_dim) cache passes
 * capacity * head_dim, so no prefix is copied. A multiple of 8.
 * scale: the logit scale s (the reference uses 1/sqrt(D); a caller that zero-pads D passes the
 * unpadded value). group: heads per wavefront (0 = automatic: at bf16 head dim 64 two, or one when
 * the two-head grid would fill the CUs only once; both give the same bits there); damp_mode 0 none, 1 linear, 2 sqrt scales F of
 * query i by min(1, train_len/(i+1)) (or its square root), reference kernels.py:179-182.
 * Limits (all entry points): one head's rows below 2 GiB ((t + 64) * row stride * element size
 * < 2^31; the row stride is head_dim here).
 */
int sa_forward(const void* q, const void* k, const void* v,
               float* out, float* rmax, float* rden, float* carry,
               const float* state_in, float* state_out, int64_t state_ld,
               void* workspace, int64_t workspace_bytes,
               int64_t nseq, int64_t heads, int64_t tq, int64_t tk, int64_t q_offset,
               int64_t kv_stride, int64_t head_dim, float scale, int dtype, int exempt, int group,
               int damp_mode, int64_t train_len, void* stream);

/*
 * Element strides of a view of a (nseq, heads, rows, head_dim) tensor whose head_dim elements per
 * row are contiguous: element (b, h, r, d) sits at p + b * seq + h * head + r * row + d.
 * Strides are multiples of 8 (bf16) or 4 (fp32) elements, row >= head_dim.
 */
typedef struct sa_view_strides {
  int64_t seq, head, row;
} sa_view_strides;

/*
 * sa_forward on views: q, k and v may be any (sequence, head, row) views, e.g. slices of one
 * packed projection (B, T, 3, heads, head_dim) read in place -- the split and transpose of the
 * reference's model (model.py:59-67) then cost nothing. y (may be NULL) receives the output
 * again, in the storage dtype, through its own view (e.g. (B, T, heads, head_dim), the layout
 * the output projection reads, mixers.py:94's cast included); `out` stays the fp32
 * (nseq, heads, tq, head_dim) output the backward needs. Layer-boundary fusion; no reference
 * counterpart (the reference copies). kv_stride of sa_forward corresponds to
 * k_strides = v_strides = {heads * kv_stride, kv_stride, head_dim}. Pointers 16-byte aligned.
 */
int sa_forward_strided(const void* q, const sa_view_strides* q_strides,
                       const void* k, const sa_view_strides* k_strides,
                       const void* v, const sa_view_strides* v_strides,
                       float* out, void* y, const sa_view_strides* y_strides,
                       float* rmax, float* rden, float* carry,
                       const float* state_in, float* state_out, int64_t state_ld,
                       void* workspace, int64_t workspace_bytes,
                       int64_t nseq, int64_t heads, int64_t tq, int64_t tk, int64_t q_offset,
                       int64_t head_dim, float scale, int dtype, int exempt, int group,
                       int damp_mode, int64_t train_len, void* stream);

/* Bytes of scratch sa_backward needs for the same `group` argument (-1 for invalid sizes). */
int64_t sa_backward_workspace_bytes(int64_t nseq, int64_t heads, int64_t t, int64_t head_dim, int dtype, int group);

/*
 * Full backward pass: replaces _SelectiveAttentionFn.backward (dbar, zeroing, the
 * _selective_backward[_pair] launch and the head-0 merge), reference
 * src/selective_attention/kernels.py:621-666. Inputs are those of a full forward
 * (q_offset 0, tq == tk == t) plus its out, rmax, rden and carry, and dout in the storage
 * dtype. dq, dk, dv receive the gradients, head 0's selection path included, in grad_dtype
 * (SA_DTYPE_BF16 or SA_DTYPE_F32; the reference accumulates in fp32 and casts to the input
 * dtype, kernels.py:664-666, so fp32 inputs run with bf16 operands get fp32 gradients).
 * group: heads per wavefront of the backward kernels (0 = automatic); the workspace size depends
 * on it. Two kernels replace the reference's one: a key-parallel pass (dK, dV) and a
 * query-parallel pass (dQ), so no gradient element is accumulated with per-tile atomics.
 * The kernels write dq, dk, dv of every head but 0 directly; head 0's dq, dk are its own sums
 * plus the other head groups' shares (one workspace slot per group), added in a fixed order by a
 * finishing pass: no atomics anywhere, so repeated calls give the same bits. q, k, v, dout, dq,
 * dk, dv 16-byte aligned.
 */
int sa_backward(const void* q, const void* k, const void* v, const float* out, const void* dout,
                const float* rmax, const float* rden, const float* carry,
                void* dq, void* dk, void* dv,
                void* workspace, int64_t workspace_bytes,
                int64_t nseq, int64_t heads, int64_t t, int64_t head_dim, float scale, int dtype,
                int grad_dtype, int exempt, int group, void* stream);

/*
 * sa_backward on views: q, k, v and dout read through their views, dq, dk, dv written through
 * theirs (e.g. straight into the gradient of a packed (B, T, 3, heads, head_dim) projection, so
 * no gradient is assembled from slices). `out` is sa_forward(_strided)'s fp32 output.
 * Layer-boundary fusion; no reference counterpart (reference kernels.py:621-666 copies).
 */
int sa_backward_strided(const void* q, const sa_view_strides* q_strides,
                        const void* k, const sa_view_strides* k_strides,
                        const void* v, const sa_view_strides* v_strides,
                        const float* out, const void* dout, const sa_view_strides* dout_strides,
                        const float* rmax, const float* rden, const float* carry,
                        void* dq, const sa_view_strides* dq_strides,
                        void* dk, const sa_view_strides* dk_strides,
                        void* dv, const sa_view_strides* dv_strides,
                        void* workspace, int64_t workspace_bytes,
                        int64_t nseq, int64_t heads, int64_t t, int64_t head_dim, float scale, int dtype,
                        int grad_dtype, int exempt, int group, void* stream);

/* Bytes of scratch sa_decode needs (per-chunk partial softmax sums, the new state rows) for t keys. */
int64_t sa_decode_workspace_bytes(int64_t nseq, int64_t heads, int64_t t, int64_t head_dim);

/*
 * One cached decode step; replaces the PyTorch step of the reference's attention slot
 * (src/selective_attention/mixers.py:115-130, `SelectiveAttention.step_cache`). The newest query
 * of every head (position t-1) attends over the t cached keys, its own included, with the carried
 * selection subtracted from its logits; then the selector head of every group adds this query's
 * own selection relu(s q.k_j) to the state, for exempt <= j < t-1:
 *   q          (nseq*heads, D)             this step's queries (storage dtype)
 *   k, v       (nseq*heads, ., D)          the caches, heads kv_stride elements apart; keys 0..t-1
 *   out        (nseq*heads, D)             fp32
 *   selected   (nseq*groups, state_ld)     fp32 per-key selection, read, then updated in place
 *   groups     selector groups per sequence: 1 = head 0 selects for every head (the shared
 *              variant), heads = every head selects for itself; heads % groups == 0
 * Logits, softmax and sums are fp32 on the upcast operands, as the reference's step.
 * Limits: head_dim 32, 64 or 128; kv_stride (0 = t * head_dim) a multiple of 8; one head's t rows
 * below 2 GiB (t * head_dim * element size < 2^31); q, k, v 16-byte aligned. Successive calls on
 * one stream may share one workspace.
 */
int sa_decode(const void* q, const void* k, const void* v, float* out, float* selected, int64_t state_ld,
              void* workspace, int64_t workspace_bytes, int64_t nseq, int64_t heads, int64_t groups, int64_t t,
              int64_t kv_stride, int64_t head_dim, float scale, int dtype, int exempt, void* stream);

/*
 * sa_decode without a workspace: the same step, arguments (less the workspace pair), results and
 * errors, for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. It allocates
 * nothing and records no timing events: the step's scratch (sa_decode_workspace_bytes of it) lives
 * in a fixed device array of SA_DECODE_SCRATCH_BYTES that the library holds on every GPU it runs
 * on until the process ends; a step needing more returns SA_ERR_SCRATCH (64 MiB takes, e.g.,
 * t = 800K keys at nseq 1, heads 16, head_dim 64, or t = 100K at nseq 8). The first call on a
 * device looks up the array's address there (with that device current). Nothing in the array
 * needs to start at zero. Every call on one GPU shares that GPU's array, which keeps the last
 * call's contents: calls that overlap on one GPU (on different streams, or from threads without
 * ordering between them) race; calls in order on one stream do not.
 */
#define SA_DECODE_SCRATCH_BYTES ((int64_t)64 << 20)
int sa_decode_noalloc(const void* q, const void* k, const void* v, float* out, float* selected, int64_t state_ld,
                      int64_t nseq, int64_t heads, int64_t groups, int64_t t, int64_t kv_stride, int64_t head_dim,
                      float scale, int dtype, int exempt, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SA_H */
