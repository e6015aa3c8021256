/*
 * C ABI of the MI355X (gfx950) dilution-attention library, libdilution_hip.so.
 *
 * The reference (Royer-Research-Labs/Dilution-Attention) has no native code:
 * its hot path is Triton kernels launched from Python.  Each entry point below
 * replaces one reference host routine and the kernel launches it makes; the
 * Python module dilution/kernels.py binds them with ctypes and keeps the
 * reference's Python signatures.
 *
 * Conventions
 *   - All tensor arguments are device pointers.  Slices are the flattened
 *     (batch * heads) dimension n; rows within a slice are contiguous with
 *     head_dim elements each.
 *   - dtype:     0 = float32, 1 = bfloat16, 2 = float16 (storage type of
 *                q / k / v / dout / outputs where stated).
 *   - precision: 0 = "ieee" (fp32 MFMA operands), 1 = "tf32" (gfx950 has no
 *                tf32 MFMA: fp32 values split into bf16 hi + lo operands,
 *                hi*hi + hi*lo + lo*hi on bf16 MFMA, about 16 bits kept per
 *                operand; the *_variant entry points run it as "ieee"),
 *                2 = "bf16" (bf16 MFMA operands).  fp32 accumulation and
 *                fp32 demand/share math in every mode.
 *   - head_dim in {16, 32, 64, 128}, and 256 with bf16 operands (precision 2)
 *     for the forward, prefill and backward and with every cache dtype for the
 *     decode steps; the *_variant entry points take 16-128.  Other widths are
 *     an argument error (-1).
 *   - Every launch is asynchronous on `stream` (a hipStream_t); no entry point
 *     synchronises or allocates device memory.  Scratch memory is
 *     caller-provided (`workspace`, at least the size the matching
 *     *_workspace_bytes query returns, 256-byte aligned).  The library's only
 *     state is the optional kernel-timing records (dil_timing_*) and, for
 *     dil_decode_step_noalloc alone, one static scratch array per GPU.
 *   - The key-parallel forward's workspace holds at most 24 GiB of output
 *     partials; a call whose slices need more runs over them in batches, so
 *     the forward workspace stays bounded at any batch size.
 *   - Return value: 0 on success, a positive hipError_t from the launch, or a
 *     negative argument error (see dil_status_string).  A NULL pointer where
 *     an argument is required is an argument error (-4); only `pk` of
 *     dil_forward may be NULL, and `carry` of dil_forward and
 *     dil_prefill_chunk on calls that take the key pass.  Argument errors are
 *     returned before any launch.
 */
#ifndef DILUTION_HIP_H
#define DILUTION_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of this ABI (bumped on any signature change). */
int dil_abi_version(void);

/* Human-readable text for a status code returned by the entry points. */
const char* dil_status_string(int status);

/*
 * Whether a dil_forward call (start = 0, chunk = seq) or a dil_prefill_chunk
 * call of this shape takes the key-parallel output pass: 1 or 0.  Its demand
 * checkpoints are an output only, so such a call may pass carry = NULL (an
 * inference forward or a prefill chunk that keeps no aux); the three-pass
 * forward reads the checkpoints it writes and needs the array.  No reference
 * counterpart: the reference's forward always writes its carry
 * (src/dilution/kernels.py:349-355).  Reads DILUTION_FORWARD_KEY_PASS as the
 * entry points do.
 */
int dil_forward_key_pass(int64_t chunk, int64_t start, int head_dim, int dtype, int precision);

/*
 * Forward over a whole sequence, with everything the backward needs.
 * Replaces dilution_attention_forward (src/dilution/kernels.py:328-455) and
 * the launches it makes (_dilution_k1 :137-198, _dilution_scan :251-264,
 * _dilution_k2 :267-315).
 *
 * q, k, v:   (n, seq, head_dim) in `dtype`.
 * out:       (n, seq, head_dim) float32.
 * rmax/rden: (n, seq) float32 row statistics: p_ij = 2^(a_ij - rmax_i) / rden_i
 *            with a_ij = log2(e) * q_i.k_j / sqrt(head_dim).
 * ssum:      (n, seq) float32 row sums of the shares.
 * carry:     (n, ceil(seq/32), seq) float32; carry[:, b, j] = sum of p_ij over
 *            rows i < 32*b (the demand checkpoint at every 32-row block),
 *            written for the block's causal keys j < 32*(b+1) only: the
 *            future triangle is left unwritten and never read (as the
 *            reference leaves it, kernels.py:353-354, test_kernels.py:143-149).
 *            May be NULL when dil_forward_key_pass(seq, 0, ...) is 1: then no
 *            checkpoint is written (outputs, statistics and totals are the
 *            same bits).
 * committed_total: (n, seq) float32 column totals of p (the decode demand).
 * pk:        (n, seq, head_dim) float32 (p @ k)/sqrt(head_dim), or NULL.
 */
int64_t dil_forward_workspace_bytes(int64_t n, int64_t seq, int head_dim, int dtype,
                                    int precision, int want_pk);
int dil_forward(const void* q, const void* k, const void* v, int64_t n, int64_t seq,
                int head_dim, int dtype, int precision, float* out, float* rmax, float* rden,
                float* ssum, float* carry, float* committed_total, float* pk, void* workspace,
                int64_t workspace_bytes, void* stream);

/*
 * Chunked prefill: rows [start, start + chunk) of the operator against the
 * cached keys [0, start + chunk), carrying the demand vector across chunks.
 * No reference counterpart: the reference prefills the whole prompt at once
 * (src/dilution/model.py:198-229, kernels.py:328-455 with return_aux=True);
 * this entry point is the same forward with an incoming demand.
 *
 * q_chunk:   (n, chunk, head_dim) in `dtype`.
 * k_cache, v_cache: (n, capacity, head_dim) in `dtype`, rows [0, start+chunk)
 *            valid.
 * committed: (n, capacity) float32.  On entry [0, start) holds the demand of
 *            rows < start and [start, start+chunk) is zero; on return
 *            [0, start+chunk) holds the demand of rows < start+chunk.  Entries
 *            at and beyond start+chunk are not touched.
 * out:       (n, chunk, head_dim) float32.
 * rmax, rden, ssum: (n, chunk) float32; carry: (n, ceil(chunk/32), start+chunk),
 *            written for keys j < start + 32*(b+1) of block b only, or NULL
 *            when dil_forward_key_pass(chunk, start, ...) is 1.
 */
int64_t dil_prefill_workspace_bytes(int64_t n, int64_t chunk, int64_t start, int head_dim,
                                    int dtype, int precision);
int dil_prefill_chunk(const void* q_chunk, const void* k_cache, const void* v_cache, int64_t n,
                      int64_t chunk, int64_t start, int64_t capacity, int head_dim, int dtype,
                      int precision, float* committed, float* out, float* rmax, float* rden,
                      float* ssum, float* carry, void* workspace, int64_t workspace_bytes,
                      void* stream);

/*
 * Backward.  Replaces _DilutionAttentionFn.backward
 * (src/dilution/kernels.py:851-903) and its launches (_dilution_ba :678-775,
 * _dilution_bc :778-809, _dilution_dq_epilogue :815-826, and the torch dbar
 * glue at :866).
 *
 * q, k, v:   (n, seq, head_dim) in `dtype` (the forward inputs).
 * dout:      (n, seq, head_dim) in `dout_dtype`.
 * out, rmax, rden, ssum, carry, pk: the forward's outputs (pk required).
 * dq, dk, dv: (n, seq, head_dim) in `grad_dtype`.
 */
int64_t dil_backward_workspace_bytes(int64_t n, int64_t seq, int head_dim, int dtype,
                                     int precision);
int dil_backward(const void* q, const void* k, const void* v, const void* dout,
                 const float* out, const float* rmax, const float* rden, const float* ssum,
                 const float* carry, const float* pk, int64_t n, int64_t seq, int head_dim,
                 int dtype, int dout_dtype, int grad_dtype, int precision, void* dq, void* dk,
                 void* dv, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Cached decode step.  Replaces dilution_decode_step
 * (src/dilution/kernels.py:994-1038) and _dilution_decode (:937-991).
 *
 * q1:        (n, head_dim) in `q_dtype` (the new row), read as fp32.
 * k_cache, v_cache: (n, capacity, head_dim) in `dtype`; rows [0, length) valid,
 *            the new token written at length-1.
 * committed: (n, capacity) float32 column totals of p over earlier rows, with
 *            committed[:, length-1] == 0.  Advanced in place over [0, length)
 *            to include this row; [length, capacity) is never touched.
 * out:       (n, head_dim) in `q_dtype` (kernels.py:953, 1029: q1 loaded in
 *            its own dtype, the output stored in it).
 */
int64_t dil_decode_workspace_bytes(int64_t n, int64_t length, int head_dim);
int dil_decode_step(const void* q1, const void* k_cache, const void* v_cache, float* committed,
                    void* out, int64_t n, int64_t capacity, int64_t length, int head_dim,
                    int dtype, int q_dtype, void* workspace, int64_t workspace_bytes,
                    void* stream);

/*
 * Cached decode step with the length in device memory.  No counterpart in
 * the reference: it is for callers that replay one captured HIP graph for
 * every decode step (the length changes each step; a kernel argument would
 * be frozen into the graph).
 *
 * Arguments as dil_decode_step, except `length`: a device pointer to the
 * live length (int64), read by the kernels when they run, and `max_length`
 * (<= capacity), which sizes the grid and the workspace
 * (dil_decode_workspace_bytes(n, max_length, head_dim)).  A live length
 * outside [0, max_length] is clamped to it.  The results are those of
 * dil_decode_step with the live length (bitwise: the same key chunks, summed
 * in the same order).
 */
int dil_decode_step_dlen(const void* q1, const void* k_cache, const void* v_cache, float* committed,
                         void* out, int64_t n, int64_t capacity, const int64_t* length,
                         int64_t max_length, int head_dim, int dtype, int q_dtype, void* workspace,
                         int64_t workspace_bytes, void* stream);

/*
 * Allocation-free cached decode step.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).
 *
 * Arguments and results as dil_decode_step, without the workspace: the
 * kernels' scratch lives in a static device array of
 * DIL_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until the
 * process ends.  A call needing more than that, i.e.
 * dil_decode_workspace_bytes(n, length, head_dim) > DIL_NOALLOC_SCRATCH_BYTES
 * (about n * length <= 16.7M at head_dim 64), returns -7 before any launch.
 * No allocation of any kind is made.  All calls on one GPU share its array:
 * calls that overlap on one GPU (two streams, two host threads) race.  The
 * array's device address is looked up on the first call per device and kept
 * for the process: a hipDeviceReset() invalidates it, so a process that
 * resets a device must not call this entry point on that device afterwards.
 */
#define DIL_NOALLOC_SCRATCH_BYTES (64LL << 20)
int dil_decode_step_noalloc(const void* q1, const void* k_cache, const void* v_cache,
                            float* committed, void* out, int64_t n, int64_t capacity,
                            int64_t length, int head_dim, int dtype, int q_dtype, void* stream);

/*
 * Operator variants: the bid and share ablations.  Replace the entry points of
 * src/dilution/kernels_bid.py -- dilution_attention_forward (:424-489, its
 * _dilution_k1 :280-360 and _dilution_k2 :362-411), _DilutionAttentionFn.
 * backward (:756-815, _dilution_b1-_b4 :513-729) and dilution_decode_step
 * (:962-1010, _dilution_decode :853-960).
 *
 * Arguments as for dil_forward / dil_backward / dil_decode_step, plus
 *   bid:    0 softmax, 1 relu, 2 relu2, 3 softplus, 4 minshift, 5 sigmoid,
 *           6 expshift, 7 sigshift (kernels_bid.py:4-42);
 *   share:  1 dilution p/(committed+p+eps), 2 exclusive p/(committed+eps),
 *           0 none (kernels_bid.py:123-127);
 *   shift:  SHIFT of expshift / sigshift (> 0).
 * (bid, share) = (0, 1) is the production operator; every variant takes the
 * head dims of the base entry points.  rmax / rden follow kernels_bid: the
 * row minimum (minshift) or 0 and the row sum of the bid numerators for the
 * ratio bids (1-4); 0 and 1 (SHIFT for expshift) for the elementwise bids;
 * pk holds scale * jac @ k, jac = dp/da (p for the softmax bids).  The
 * workspace sizes are those of the matching base entry point.
 */
int dil_forward_variant(const void* q, const void* k, const void* v, int64_t n, int64_t seq,
                        int head_dim, int dtype, int precision, int bid, int share, float shift,
                        float* out, float* rmax, float* rden, float* ssum, float* carry,
                        float* committed_total, float* pk, void* workspace, int64_t workspace_bytes,
                        void* stream);
int dil_backward_variant(const void* q, const void* k, const void* v, const void* dout,
                         const float* out, const float* rmax, const float* rden,
                         const float* ssum, const float* carry, const float* pk, int64_t n,
                         int64_t seq, int head_dim, int dtype, int dout_dtype, int grad_dtype,
                         int precision, int bid, int share, float shift, void* dq, void* dk,
                         void* dv, void* workspace, int64_t workspace_bytes, void* stream);
int dil_decode_step_variant(const void* q1, const void* k_cache, const void* v_cache,
                            float* committed, void* out, int64_t n, int64_t capacity,
                            int64_t length, int head_dim, int dtype, int q_dtype, int bid,
                            int share, float shift, void* workspace, int64_t workspace_bytes,
                            void* stream);

/*
 * Few-row projections of the LM's decode step.  No counterpart in the
 * reference, whose model runs these projections through torch.nn.Linear
 * (model.py:41-93) with the norms and the MLP activation as separate ops: at
 * M = the decode batch (at most 8 rows) each product streams its weight once,
 * and a library GEMM tiled for large M reads it at a fraction of HBM speed.
 *
 *   mode 0:  out = x W1^T
 *   mode 1:  out = resid + x W1^T
 *   mode 2:  out = rmsnorm(x) W1^T,               rmsnorm(x) = x / sqrt(mean(x^2) + eps) * g
 *   mode 3:  out = silu(r W1^T) * (r W2^T),        r = rmsnorm(x)
 *
 * x (rows, k), W1 / W2 (n, k) (nn.Linear weights), g (k), resid and out
 * (rows, n): row-major, contiguous, dtype bf16 only (dtype code 1; others
 * return -2).  1 <= rows <= 8, k a multiple of 256 up to 4096, eps >= 0.
 * Intermediates are rounded to bf16 where the unfused torch ops round them.
 * Asynchronous on `stream`; no workspace; out must not alias x or resid.
 */
int dil_rows_linear(const void* x, const void* w1, const void* w2, const void* g, const void* resid,
                    void* out, int64_t rows, int64_t n, int64_t k, int mode, int dtype, float eps,
                    void* stream);

/*
 * The decode step's norm + q/k/v projection with the cache append folded in.
 * No counterpart in the reference, whose attention block projects with
 * c_attn (model.py:41-93) and then writes k and v into its cache
 * (model.py:86-93) as separate ops.  w is c_attn's weight (3 heads head_dim,
 * k) with the q, k and v rows in that order; g the RMSNorm weight:
 *
 *   [q | k | v] = rmsnorm(x) w^T              (rows, 3 heads head_dim)
 *   q_out[m, :]                  = q[m, :]     (rows, heads * head_dim)
 *   k_cache[m, h, pos, :]        = k[m, h * head_dim : (h + 1) * head_dim]
 *   v_cache[m, h, pos, :]        = v[m, ...]   likewise
 *
 * The caches are (rows, heads, capacity, head_dim) contiguous.  pos is read
 * from device memory when pos_dev is not null (graph replay), else taken
 * from `pos` (0 <= pos < capacity, checked); a device position outside
 * [0, capacity) stores no cache row.  Same dtype, rows and k rules as
 * dil_rows_linear.
 */
int dil_rows_linear_qkv(const void* x, const void* w, const void* g, void* q_out, void* k_cache,
                        void* v_cache, int64_t rows, int64_t heads, int64_t head_dim, int64_t capacity,
                        const int64_t* pos_dev, int64_t pos, int64_t k, int dtype, float eps, void* stream);

/*
 * Greedy token selection for the decode step.  No counterpart in the
 * reference, whose sampler takes torch.argmax of the last position's logits
 * (model.py:473-509).  out[r] (int64) = the index of the largest of
 * logits[r, 0:limit] for r < rows, with torch.argmax's choice: a NaN counts
 * as the largest value, and among equal values the smallest index wins.
 * logits are bf16 (dtype code 1; others return -2), row r at
 * logits + r * row_stride elements; 1 <= rows <= 65535,
 * 1 <= limit <= row_stride, limit < 2^31.  Asynchronous on `stream`.
 */
int dil_rows_argmax(const void* logits, int64_t rows, int64_t row_stride, int64_t limit, void* out, int dtype,
                    void* stream);

/*
 * Kernel timing for measurement harnesses.  No reference counterpart (the
 * reference times its Triton launches with torch.profiler and CUDA events in
 * scripts/step_profile.py:29-47 and scripts/profile_kernels.py:115-144).
 *
 * dil_timing_enable(1) makes every later launch of the entry points above
 * record a pair of hipEvents on its stream; dil_timing_count() /
 * dil_timing_read() wait for those events and report, per kernel name, the
 * number of launches and the summed event-to-event milliseconds since the
 * last dil_timing_reset().  Off by default.
 */
int dil_timing_enable(int on);
int dil_timing_reset(void);
int dil_timing_count(void);
int dil_timing_read(int index, char* name, int name_capacity, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* DILUTION_HIP_H */
