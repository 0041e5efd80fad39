/*
 * tasft_amd — C ABI of the MI355X (gfx950) block-sparse attention hot path.
 *
 * Every function launches asynchronously on `stream` (a hipStream_t; pass the
 * caller's current stream) and never synchronises the device, allocates, frees or
 * retains a pointer beyond the call. Device buffers — inputs, outputs and
 * workspaces — are owned by the caller. Q, K, V and outputs of attention are 16-bit
 * (raw words) of the type named by the call's `dtype` argument: TASFT_DTYPE_BF16 or
 * TASFT_DTYPE_F16 (scores, softmax and accumulation are fp32 either way); other tensors
 * are as stated. Each 4-D tensor is described by element strides for its dims
 * (b, h, s, d); the d stride must be 1 and no stride may be negative (a negative one is
 * rejected with TASFT_ERR_INVALID_ARGUMENT). Return value: 0 on success, a negative
 * status on error, with the message available from tasft_last_error() on the
 * calling thread.
 *
 * Layouts: Q [B, Hq, S, D]; K and V [B, Hkv, S, D] (GQA-native: query head h uses
 * KV head h / (Hq / Hkv)); block masks are one byte per block, non-zero = attend.
 */
#ifndef TASFT_AMD_H_
#define TASFT_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define TASFT_OK 0
#define TASFT_ERR_INVALID_ARGUMENT (-1)
#define TASFT_ERR_UNSUPPORTED (-2)
#define TASFT_ERR_LAUNCH (-3)
#define TASFT_ERR_WORKSPACE (-4)

/* Message of the last error on this thread ("" if none). */
const char* tasft_last_error(void);

/* ABI version of this library (9). */
int tasft_abi_version(void);

/* Element types of the 16-bit tensors (the `dtype` argument). The reference kernel takes
 * fp16 or bf16 (tasft/kernels/block_sparse_fa.py:228, :252 are dtype-generic) and its gate
 * module fp16, bf16 or fp32 (tasft/modules/attn_gate.py:59). */
#define TASFT_DTYPE_BF16 0
#define TASFT_DTYPE_F16 1

/*
 * Block-sparse flash-attention prefill.
 * Replaces BlockSparseFlashAttention._triton_forward and the Triton kernel
 * _block_sparse_attn_fwd_kernel (reference tasft/kernels/block_sparse_fa.py:454-552
 * and :108-269), and makes the GQA expansion of K/V at
 * tasft/modules/tasft_attention.py:725-729 unnecessary.
 *
 * out[b,h,i,:] = softmax_j(q[b,h,i,:] . k[b,h/G,j,:] * scale + M[i,j]) v[b,h/G,j,:]
 * with M = 0 where block_mask[b,h,i/bs,j/bs] != 0 (AND j/bs <= i/bs when causal;
 * AND j <= i inside the diagonal block when causal) and j < seq_len, else -inf.
 * Rows with no admissible key are 0. P is rounded to `dtype` before the PV product.
 * block_mask: [B, Hq, ceil(S/bs), ceil(S/bs)] bytes, strides in mask_strides (bytes).
 * head_dim in {64, 128}; block_size in {32, 64, 128}; strides of b/h/s multiples of 8.
 * Block size 128 runs on the block-64 kernels, each 128-token block as its four 64-token
 * quarters (the same tokens attend to the same keys).
 * workspace: NULL (one workgroup per query-block row), or >=
 * tasft_bsfa_prefill_workspace_bytes(...) bytes, 16-byte aligned: then (block size 64 or
 * 128, head_dim 64) a persistent launch keeps every CU slot busy, pulling rows from ticket
 * counters kept in the workspace (zeroed on `stream` by the call itself). head_dim 128
 * always runs one workgroup per row (its two-wave kernel fills four slots per CU) and
 * leaves the workspace untouched. The output does not depend on it.
 * Calls that share one workspace must be ordered on one stream.
 */
int tasft_bsfa_prefill_fwd(const void* q, const void* k, const void* v, void* out,
                           const uint8_t* block_mask, void* workspace, size_t workspace_bytes,
                           int64_t batch, int64_t num_q_heads,
                           int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                           int64_t block_size, const int64_t* q_strides, const int64_t* k_strides,
                           const int64_t* v_strides, const int64_t* o_strides,
                           const int64_t* mask_strides, float scale, int causal, int dtype,
                           void* stream);

/*
 * Block-sparse prefill of a packed batch of variable-length sequences, in one launch.
 * Stands in for the flat-token prefill of TASFTvLLMAttentionBackend.forward
 * (reference tasft/inference/vllm_patch.py:172-176 and :199-203), which views all
 * num_tokens tokens as one sequence (B = 1) and so lets a request attend to the tokens of
 * the requests packed before it; here sequence n is tokens cu_seqlens[n] ..
 * cu_seqlens[n+1]-1 and attends only within itself, with the semantics of
 * tasft_bsfa_prefill_fwd applied per sequence (positions and blocks counted from its
 * first token).
 *
 * q, out [T, Hq, D]; k, v [T, Hkv, D] (strides of token, head, dim in elements, dim
 * contiguous, token and head strides multiples of 8). cu_seqlens: device int32
 * [num_seqs + 1], cu_seqlens[0] = 0, non-decreasing, every length <= max_seqlen.
 * block_mask: [num_seqs, Hq, NB, NB] bytes with NB = ceil(max_seqlen / bs); sequence n
 * uses its leading ceil(len_n / bs) x ceil(len_n / bs) corner. Lengths are clamped to
 * [0, max_seqlen]; the caller guarantees the tokens exist. No workspace.
 */
int tasft_bsfa_prefill_varlen_fwd(const void* q, const void* k, const void* v, void* out,
                                  const uint8_t* block_mask, const int32_t* cu_seqlens,
                                  int64_t num_seqs, int64_t num_q_heads, int64_t num_kv_heads,
                                  int64_t max_seqlen, int64_t head_dim, int64_t block_size,
                                  const int64_t* q_strides, const int64_t* k_strides,
                                  const int64_t* v_strides, const int64_t* o_strides,
                                  const int64_t* mask_strides, float scale, int causal,
                                  int dtype, void* stream);

/*
 * Zeroes the rows of out [T, H, D] (strides of token, head, dim in elements, dim
 * contiguous) for the tokens at or after cu_seqlens[num_seqs], reading that offset from
 * device memory, so a caller holding cu_seqlens on the device gets the zero rows of
 * tasft_bsfa_prefill_varlen_fwd's contract without a host round trip. Launch it on the
 * same stream as the prefill; the two write disjoint rows. No reference counterpart: the
 * reference's flat-token prefill has no uncovered rows (tasft/inference/vllm_patch.py:172-176).
 */
int tasft_bsfa_varlen_zero_tail(void* out, const int32_t* cu_seqlens, int64_t num_seqs,
                                int64_t tokens, int64_t num_heads, int64_t head_dim,
                                const int64_t* o_strides, void* stream);

/*
 * Bytes of the optional workspace of tasft_bsfa_prefill_fwd (work-queue counters).
 * No reference counterpart: the reference launches one program per query block in
 * grid order (tasft/kernels/block_sparse_fa.py:517-550).
 */
size_t tasft_bsfa_prefill_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t seq_len,
                                          int64_t block_size);

/*
 * Bytes of workspace tasft_bsfa_decode_fwd needs for `num_splits` splits.
 * No reference counterpart: the reference has no sparse decode
 * (tasft/inference/vllm_patch.py:189-196 routes decode to dense PagedAttention).
 */
size_t tasft_bsfa_decode_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim,
                                         int64_t num_splits);

/*
 * Split-K block-sparse decode: one new query token per sequence.
 * Stands in for the dense decode branch at tasft/inference/vllm_patch.py:189-196 and
 * :215-252 (and the S_q != S_k rejection at tasft/modules/attn_gate.py:216-221); its
 * result equals the last query row of tasft_bsfa_prefill_fwd under the same mask row.
 *
 * q [B, Hq, 1, D]; k_cache, v_cache [B, Hkv, kv_len_max, D]; out [B, Hq, 1, D];
 * block_mask [B, Hq, 1, ceil(kv_len_max/bs)] bytes; kv_lens [B] int32 valid lengths
 * (NULL = kv_len_max). Every KV block selected by any query head of a KV head is read
 * once for that KV head. workspace: >= tasft_bsfa_decode_workspace_bytes(...) bytes,
 * 16-byte aligned. At most 16 query heads per KV head. A 128-key block is read as its
 * two 64-key halves, and num_blocks below counts those halves. num_splits >=
 * ceil(num_blocks / 1024); the splits of a (b, KV head) share its selected blocks
 * equally, and with num_splits == 1 the output is written without a combine pass.
 * Results differ between split counts only by float rounding. One launch runs
 * batch * num_kv_heads * num_splits workgroups (two fit per CU); about one per CU
 * measured fastest.
 */
int tasft_bsfa_decode_fwd(const void* q, const void* k_cache, const void* v_cache, void* out,
                          const uint8_t* block_mask, const int32_t* kv_lens, void* workspace,
                          size_t workspace_bytes, int64_t batch, int64_t num_q_heads,
                          int64_t num_kv_heads, int64_t kv_len_max, int64_t head_dim,
                          int64_t block_size, int64_t num_splits, const int64_t* q_strides,
                          const int64_t* k_strides, const int64_t* v_strides,
                          const int64_t* o_strides, const int64_t* mask_strides, float scale,
                          int dtype, void* stream);

/*
 * tasft_bsfa_decode_fwd without a workspace: the variant that allocates nothing.
 * No counterpart in the reference. It is for callers that cannot allocate device memory
 * or take a caller-sized workspace: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.
 *
 * Arguments and results are those of tasft_bsfa_decode_fwd minus the workspace. The split
 * partials go to a static device array of TASFT_DECODE_NOALLOC_MAX_BYTES bytes inside the
 * library (one per GPU, held until the process ends; its address is looked up on the
 * first call on each device, with the stream's device current). A call whose
 * tasft_bsfa_decode_workspace_bytes(batch, num_q_heads, head_dim, num_splits) exceeds it
 * returns TASFT_ERR_WORKSPACE without launching. With num_splits == 1 the array is not
 * touched. Every call on one GPU shares the array: calls that overlap on one GPU (on
 * different streams, or from different threads without ordering) race and give wrong
 * results; calls ordered on one stream are safe.
 */
#define TASFT_DECODE_NOALLOC_MAX_BYTES ((size_t)16 << 20)
int tasft_bsfa_decode_fwd_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                  void* out, const uint8_t* block_mask, const int32_t* kv_lens,
                                  int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                  int64_t kv_len_max, int64_t head_dim, int64_t block_size,
                                  int64_t num_splits, const int64_t* q_strides,
                                  const int64_t* k_strides, const int64_t* v_strides,
                                  const int64_t* o_strides, const int64_t* mask_strides,
                                  float scale, int dtype, void* stream);

/*
 * Split-K block-sparse decode over a paged KV cache (vLLM's block-table layout).
 * Stands in for the paged dense decode that tasft/inference/vllm_patch.py:189-196 and
 * :215-252 hand to vLLM's PagedAttention; its result equals tasft_bsfa_decode_fwd on the
 * contiguous cache holding the same tokens.
 *
 * k_pages, v_pages [num_pages, page_size, Hkv, D] (strides of page, token, head, dim in
 * elements, dim contiguous); token t of sequence b is row t % page_size of page
 * block_table[b * block_table_stride + t / page_size] (device int32; only the pages that
 * hold a token below kv_lens[b] are read). num_pages: the number of pages in each pool;
 * a table entry outside [0, num_pages) is clamped into it, so a corrupt table gives wrong
 * values but never reads outside the pools. kv_lens: device int32 [B], required.
 * kv_len_max bounds every kv_lens[b]; block_mask [B, Hq, 1, ceil(kv_len_max/bs)].
 * block_size 32, 64 or 128 (vLLM's per-layer block size, tasft/inference/vllm_patch.py:522-525;
 * a 128-key block is read as its two 64-key halves, and num_splits then counts 64-key
 * blocks: ceil(kv_len_max/64) / num_splits <= 1024); page_size a power of two >= 8.
 * Other arguments as in tasft_bsfa_decode_fwd (same workspace size).
 */
int tasft_bsfa_decode_paged_fwd(const void* q, const void* k_pages, const void* v_pages,
                                void* out, const uint8_t* block_mask,
                                const int32_t* block_table, const int32_t* kv_lens,
                                void* workspace, size_t workspace_bytes, int64_t batch,
                                int64_t num_q_heads, int64_t num_kv_heads, int64_t kv_len_max,
                                int64_t head_dim, int64_t block_size, int64_t page_size,
                                int64_t num_pages, int64_t num_splits, const int64_t* q_strides,
                                const int64_t* k_strides, const int64_t* v_strides,
                                const int64_t* o_strides, const int64_t* mask_strides,
                                int64_t block_table_stride, float scale, int dtype,
                                void* stream);

/* Bytes of workspace tasft_gate_fwd needs (projected block features; head_dim is checked
 * but does not change the size). */
size_t tasft_gate_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                  int64_t seq_len, int64_t head_dim, int64_t block_size,
                                  int64_t hidden);

/*
 * Fused AttnGate forward.
 * Replaces AttnGate._pool_to_blocks + AttnGate.forward (reference
 * tasft/modules/attn_gate.py:151-285) for inference, without the [B,H,NB,NB,2D]
 * concat tensor of :250-257.
 *
 * w_in [hidden, 2*D] fp32 (columns [:D] act on pooled Q, [D:] on pooled K), b_in [hidden],
 * w_out [hidden], thresholds [Hq] fp32 per-head tau. Outputs, all [B, Hq, NB, NB]
 * contiguous: soft_scores fp32 (sigmoid of the logit, exactly 0 above the block
 * diagonal when causal), logits fp32 (may be NULL), hard_mask bytes (soft >= tau).
 * active_count: one uint64 in device memory receiving the number of set mask bytes.
 * q_means [B, Hq, NB, D], k_means [B, Hkv, NB, D] fp32 (each may be NULL) receive the
 * zero-padded block means (what tasft_gate_bwd's caller needs for the W_in gradient).
 * The workspace afterwards holds u = W_q qbar + b_in [B, Hq, NB, hidden] followed by
 * v = W_k kbar [B, Hkv, NB, hidden] (fp32), the input of tasft_gate_bwd.
 * flags: TASFT_GATE_CAUSAL (zero the upper block triangle, reference is_causal) |
 * TASFT_GATE_FORCE_DIAGONAL (set the diagonal blocks in hard_mask regardless of tau).
 * head_dim a multiple of 8, at most 256; any block_size >= 1.
 * Block size 64 with head_dim 64 or 128 and hidden a multiple of 32 up to 128 runs as one
 * kernel (after a one-workgroup reset of its counters in the workspace): workgroups that
 * pool the query blocks wait, bounded by 1 ms of wall clock, for the workgroups that pool
 * the key blocks. Should that wait ever give up, bit 63 of active_count is set and the
 * affected rows hold NaN scores and no mask bit; callers that read active_count check it.
 * One call at a time per workspace: calls that overlap on one workspace race.
 */
#define TASFT_GATE_CAUSAL 1
#define TASFT_GATE_FORCE_DIAGONAL 2
int tasft_gate_fwd(const void* q, const void* k, const float* w_in, const float* b_in,
                   const float* w_out, const float* thresholds, float* soft_scores, float* logits,
                   uint8_t* hard_mask, unsigned long long* active_count, float* q_means,
                   float* k_means, void* workspace, size_t workspace_bytes, int64_t batch,
                   int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len, int64_t head_dim,
                   int64_t block_size, int64_t hidden, const int64_t* q_strides,
                   const int64_t* k_strides, int flags, int dtype, void* stream);

/*
 * Diagnostic for tests of the error path above; no counterpart in the reference. While
 * enable is nonzero, the one-launch gate's key workgroups publish nothing and every query
 * workgroup's wait gives up after 20 us (bit 63 of active_count set, NaN scores); every
 * workgroup still exits normally. Returns 0.
 */
int tasft_gate_debug_wait_fault(int enable);

/*
 * The pairwise stage of the gate on precomputed projected units, for query-block rows that
 * need not start at block 0: a cached decode step's selection (one row) without pooling the
 * KV cache again. With the units of tasft_gate_fwd's workspace (u for the rows, v for the
 * key blocks) it gives exactly those rows of tasft_gate_fwd's output. No reference
 * counterpart: the reference gate rejects S_q != S_k (tasft/modules/attn_gate.py:216-221).
 *
 * uq [B, Hq, rows, hidden] fp32 contiguous: u = W_q qbar + b_in of query blocks row0 ..
 * row0 + rows - 1. uk: v = W_k kbar of key blocks 0 .. key_blocks - 1, block j of
 * (b, KV head g) at uk[(b * Hkv + g) * uk_head_stride + j * hidden] (uk_head_stride >=
 * key_blocks * hidden; it and hidden multiples of 4; 16-byte aligned). Outputs [B, Hq, rows,
 * key_blocks] as in tasft_gate_fwd; the causal zero and TASFT_GATE_FORCE_DIAGONAL compare key
 * block j with query block row0 + i. active_count is zeroed and counted by the call.
 */
int tasft_gate_rows_fwd(const float* uq, const float* uk, const float* w_out,
                        const float* thresholds, float* soft_scores, float* logits,
                        uint8_t* hard_mask, unsigned long long* active_count, int64_t batch,
                        int64_t num_q_heads, int64_t num_kv_heads, int64_t rows,
                        int64_t key_blocks, int64_t row0, int64_t hidden, int64_t uk_head_stride,
                        int flags, void* stream);

/*
 * One cached decode step's gate rows with the state update folded in: what
 * SparseAttentionDecoder does per token before its decode (the running block sums, the
 * projection of the current key block and of the query heads, then tasft_gate_rows_fwd's
 * row), in one launch per (b, KV head). No reference counterpart: the reference gate
 * rejects S_q != S_k (tasft/modules/attn_gate.py:216-221).
 *
 * q_new [B, Hq, D] and k_new [B, Hkv, D] 16-bit (dtype), with (b, head) strides
 * q_strides[0..1] / k_strides[0..1] and D contiguous: the new token. q_sum [B, Hq, D] and
 * k_sum [B, Hkv, D] fp32 contiguous: the sums of the current block's queries and keys before
 * this token, updated in place (reset_sums != 0 starts a new block: the sums are replaced by
 * the token). uk: the kept key units, block j of (b, KV head g) at uk[(b * Hkv + g) *
 * uk_head_stride + j * hidden] (16-byte aligned; uk_head_stride a multiple of 4 holding at
 * least row + 1 blocks); block `row` (the token's block) is rewritten with
 * k_sum x wk_t. wq_t and wk_t [D, hidden] fp32: W_in[:, :D] and W_in[:, D:] transposed and
 * divided by the block size (a zero-padded block mean is then sum x W); b_in, w_out
 * [hidden]; thresholds [Hq]. Outputs [B, Hq, 1, row + 1] contiguous: soft_scores (sigmoid
 * of w_out . relu(q_sum x wq_t + b_in + v_j)), hard_mask (soft >= tau, and the diagonal
 * j = row with TASFT_GATE_FORCE_DIAGONAL). active_count is zeroed and counted by the call;
 * it may be NULL, and then no count is kept (one launch fewer).
 * Limits: Hq / Hkv <= 8, head_dim <= 256, hidden <= 256 and a multiple of 4.
 */
int tasft_gate_decode_rows_fwd(const void* q_new, const void* k_new, const int64_t* q_strides,
                               const int64_t* k_strides, float* q_sum, float* k_sum, float* uk,
                               int64_t uk_head_stride, const float* wq_t, const float* wk_t,
                               const float* b_in, const float* w_out, const float* thresholds,
                               float* soft_scores, uint8_t* hard_mask,
                               unsigned long long* active_count, int64_t batch,
                               int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                               int64_t hidden, int64_t row, int reset_sums, int flags, int dtype,
                               void* stream);

/*
 * Backward of the gate's pairwise MLP, for gate training: the gradient the reference gets
 * from autograd through AttnGate.forward (tasft/modules/attn_gate.py:248-273), without the
 * [B, H, NB, NB, hidden] activations.
 *
 * soft_scores and grad_soft [B, Hq, NB, NB] fp32 contiguous (the forward's soft scores and
 * dL/dsoft); fwd_workspace: the workspace of the tasft_gate_fwd call that produced them.
 * With g = grad_soft * soft * (1 - soft) (0 where the causal zero applied) and
 * pre[i][j][c] = u[i][c] + v[j][c], partials (>= tasft_gate_bwd_workspace_bytes, fp32)
 * receives, for T = ceil(NB / 32) tiles:
 *   du_part [T][B][Hq][NB][hidden]: sum over the keys of key tile t of g * (pre > 0),
 *   dv_part [T][B][Hq][NB][hidden]: sum over the queries of query tile t of g * (pre > 0),
 *   dw_part [B*Hq*T*T][hidden]: sum over the tile's pairs of g * relu(pre).
 * Then dL/dw_out = sum(dw_part), dL/du = w_out * sum_t du_part, dL/dv = w_out * (sum_t
 * dv_part, summed over the query heads of each KV head), and dL/dW_in, dL/db_in follow from
 * u and v's definitions (plain GEMMs with the block means). flags: TASFT_GATE_CAUSAL.
 */
size_t tasft_gate_bwd_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t seq_len,
                                      int64_t block_size, int64_t hidden);
int tasft_gate_bwd(const float* soft_scores, const float* grad_soft, const void* fwd_workspace,
                   size_t fwd_workspace_bytes, float* partials, size_t partials_bytes,
                   int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t seq_len,
                   int64_t block_size, int64_t hidden, int flags, void* stream);

/*
 * Gate target from Q and K, without the [B, H, S, S] score tensor.
 * Replaces the score producer TASFTAttention._training_forward
 * (tasft/modules/tasft_attention.py:426-458) followed by
 * TASFTObjective.compute_gate_target (tasft/training/objectives.py:128-185).
 *
 * target [B, Hq, NB, NB] fp32 contiguous receives the block maxima of
 * q.k^T*scale (+ attn_mask) (causal: -inf above the diagonal and for key > query), then,
 * when normalize is 0, a softmax over the flat NB*NB grid of each (b, h) (the reference);
 * 1, a softmax over the key blocks of each row; 2, no normalisation (raw maxima).
 * Before the softmax, finite maxima are clamped to [-clamp, clamp] when clamp > 0
 * and divided by temperature (the variant of tasft/modules/tasft_attention.py:272-290).
 * attn_mask: NULL, or the additive mask of tasft_attention.py:445-449 as fp32 with
 * element (b, h, query, key) at attn_mask[b*s0 + h*s1 + query*s2 + key] for
 * mask_strides = {s0, s1, s2} (0 broadcasts a dim: a key-padding row has s1 = s2 = 0).
 * It must be addressable for every query and key below max(NB*block_size,
 * 64*ceil(seq_len/64)) (values past seq_len are ignored), 16-byte aligned, strides
 * non-negative multiples of 4.
 * block_size 128 runs over 64-token blocks: target is first filled with -inf, then each
 * 64-block maximum is merged into its 128-block by atomic max (exact, order-free).
 * block_size 32 also runs over 64-token blocks, each 32 x 32 quarter of a 64-block
 * written as one block (so a block-32 mask is read up to a multiple of 64).
 */
int tasft_gate_target_fwd(const void* q, const void* k, const float* attn_mask, float* target,
                          int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                          int64_t seq_len, int64_t head_dim, int64_t block_size,
                          const int64_t* q_strides, const int64_t* k_strides,
                          const int64_t* mask_strides, float scale, int causal, int normalize,
                          float temperature, float clamp, int dtype, void* stream);

/*
 * KL gate loss: replaces TASFTObjective.compute_gate_loss (tasft/training/objectives.py:187-221),
 * KL(target || gate) with the gate scores normalised over each (b, h) grid and reduced
 * with "batchmean". Together with tasft_gate_target_fwd it is the per-layer gate term of
 * TASFTObjective.compute (objectives.py:316-346) without the [B, H, S, S] scores.
 *
 * gate_scores, target [B, H, NBq, NBk] fp32 contiguous. loss_partials [B*H] receives each
 * (b, h)'s KL sum (the loss is their sum divided by B); grad_scores (NULL allowed) receives
 * d(loss)/d(gate_scores).
 */
int tasft_gate_kl_fwd(const float* gate_scores, const float* target, int64_t batch,
                      int64_t num_heads, int64_t num_blocks_q, int64_t num_blocks_k,
                      float* loss_partials, float* grad_scores, void* stream);

/*
 * Block mask -> compressed rows (CSR) of its active blocks.
 * No reference counterpart: the reference hands its Triton kernel the dense mask and
 * scans every byte of a row (tasft/kernels/block_sparse_fa.py:192-203); this gives
 * callers (and index-based selection) the active blocks directly.
 *
 * Rows are (b, h, query block) in row-major order, rows = batch*num_heads*num_q_blocks.
 * row_ptr [rows + 1] int32 receives the exclusive prefix of the per-row counts;
 * col_idx receives each row's active key-block indices in ascending order, at most
 * col_capacity of them in total (row_ptr[rows] is the full count, so overflow is
 * visible). causal != 0 counts only key blocks <= the query block (the AND at
 * tasft/kernels/block_sparse_fa.py:502-508). workspace: >=
 * tasft_mask_compact_workspace_bytes(...) bytes.
 */
size_t tasft_mask_compact_workspace_bytes(int64_t batch, int64_t num_heads, int64_t num_q_blocks);
int tasft_mask_compact(const uint8_t* block_mask, int64_t batch, int64_t num_heads,
                       int64_t num_q_blocks, int64_t num_k_blocks, const int64_t* mask_strides,
                       int causal, int32_t* row_ptr, int32_t* col_idx, int64_t col_capacity,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Padded index lists -> dense block mask, the input form of tasft_bsfa_decode_fwd for
 * callers that select KV blocks by index (the decode selection of a serving engine).
 * No reference counterpart (reference decode is dense:
 * tasft/inference/vllm_patch.py:189-196).
 *
 * indices [rows, k] int32 with row stride index_row_stride (elements), -1 = empty slot;
 * block_mask [rows, num_k_blocks] bytes, contiguous, receives 1 at every listed index
 * and 0 elsewhere. *error_flag (device int) becomes non-zero if an index other than -1
 * lies outside [0, num_k_blocks); such indices are skipped.
 */
int tasft_mask_from_indices(const int32_t* indices, int64_t rows, int64_t k,
                            int64_t index_row_stride, int64_t num_k_blocks, uint8_t* block_mask,
                            int* error_flag, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TASFT_AMD_H_ */
