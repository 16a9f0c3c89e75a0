/*
 * lite_lang_amd — C ABI of the MI355X (gfx950) kernels behind the Qwen2
 * token loop of lite_lang.
 *
 * Conventions (all entry points):
 *   - plain device pointers, element strides (not bytes), int64 sizes;
 *   - `dtype` is one of LL_DTYPE_* and selects the element type of every
 *     floating-point tensor argument of the call unless stated otherwise;
 *   - index arrays that the reference builds with torch.tensor(list) (int64)
 *     are accepted as int32 or int64 via the matching `*_i64` flag;
 *   - every call is asynchronous on `stream` and returns LL_OK (0) or a
 *     negative LL_ERR_* code; ll_last_error() then holds the reason. Argument
 *     errors are raised before anything is launched.
 *   - workspaces are caller-owned device buffers of the size the matching
 *     *_workspace_size query returns; calls that share one workspace must
 *     not overlap in time. Their contents need no initialisation, except the
 *     decode attention workspace, which must be zero-filled once before its
 *     first use (every call leaves it fit for the next).
 */
#ifndef LITELANG_AMD_H
#define LITELANG_AMD_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LL_ABI_VERSION 1

#define LL_DTYPE_F32 0
#define LL_DTYPE_F16 1
#define LL_DTYPE_BF16 2

#define LL_OK 0
#define LL_ERR_ARG (-1)
#define LL_ERR_UNSUPPORTED (-2)
#define LL_ERR_HIP (-3)

/* Library identification and error text (no reference counterpart: the
 * reference raises Python exceptions from Triton). */
int ll_version(void);
const char* ll_last_error(void);

/* ---------------------------------------------------------------- attention */

/* Paged GQA decode attention, split-K (the last split of each (sequence,
 * KV head) merges the partials, in the same launch).
 * Replaces token_decode_attention_flash_decoding
 *   (litelang/kernel/develop_flash_attn/flash_decoding.py:262-312).
 * q [batch, q_heads, head_dim]; k_cache / v_cache [P, kv_heads, head_dim]
 * views of the pool (last dim contiguous); req_to_tokens [max_batch, max_len]
 * int32 slot table; out [batch, q_heads, head_dim]. max_len_in_batch bounds
 * b_seq_len (it sizes the split count and the workspace; tokens beyond it are
 * ignored, as the reference's grid ignores them). workspace: at least
 * ll_decode_attention_workspace_size bytes (0 when no split is needed),
 * zero-filled before its first use: its first 16 KiB hold split tickets and
 * the rest the split partials, whose zero words mean "not yet written"; every
 * call leaves all of it at zero again, so one buffer serves calls of any
 * shape; two calls in flight at once must not share it. */
int64_t ll_decode_attention_workspace_size(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                           int64_t head_dim, int64_t max_len_in_batch);
int ll_decode_attention(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                        const void* k_cache, int64_t k_stride_tok, int64_t k_stride_head,
                        const void* v_cache, int64_t v_stride_tok, int64_t v_stride_head,
                        const int32_t* req_to_tokens, int64_t req_to_tokens_stride,
                        const void* b_req_idx, int req_idx_i64, const void* b_seq_len,
                        int seq_len_i64, void* out, int64_t out_stride_b, int64_t out_stride_h,
                        int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                        int64_t max_len_in_batch, float sm_scale, int dtype, void* workspace,
                        int64_t workspace_bytes, hipStream_t stream);

/* ll_decode_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference.
 * The split tickets and partials live in a library-owned device array of
 * ll_decode_attention_noalloc_max_bytes() bytes (4 MiB) that each GPU the
 * library runs on holds until the process ends; a shape whose partials need
 * more is rejected with LL_ERR_ARG (use ll_decode_attention with a
 * workspace). Nothing is allocated. Every call on one GPU shares that GPU's
 * array: two calls that overlap in time on one GPU (two streams, two threads)
 * race and give wrong results. The array starts zeroed (split tickets and
 * partials) and every call leaves it at zero, so nothing is cleared. The
 * first call on a device looks the array's device address up (no work is
 * queued; this may happen under graph capture); ll_decode_attention_noalloc_init
 * does that lookup for the current device ahead of time, for set-up code.
 * Results are identical to ll_decode_attention's. */
int64_t ll_decode_attention_noalloc_max_bytes(void);
int ll_decode_attention_noalloc_init(void);
int ll_decode_attention_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                const void* k_cache, int64_t k_stride_tok,
                                int64_t k_stride_head, const void* v_cache,
                                int64_t v_stride_tok, int64_t v_stride_head,
                                const int32_t* req_to_tokens, int64_t req_to_tokens_stride,
                                const void* b_req_idx, int req_idx_i64, const void* b_seq_len,
                                int seq_len_i64, void* out, int64_t out_stride_b,
                                int64_t out_stride_h, int64_t batch, int64_t q_heads,
                                int64_t kv_heads, int64_t head_dim, int64_t max_len_in_batch,
                                float sm_scale, int dtype, hipStream_t stream);

/* Launches a probe kernel on exactly the grid, block and LDS size of
 * ll_decode_attention's split stage for this shape and writes, for every
 * workgroup i, the XCD it ran on (hardware register XCC_ID) to out[i].
 * Returns the grid size (> 0) or a negative LL_ERR_* code. The split merge in
 * the same launch assumes (out[i] - i) mod 8 is the same for every i of a
 * launch (round-robin dealing, from whichever XCD the previous launch left
 * off at), so that every split of a sequence meets in one XCD's L2. No
 * reference counterpart: it exists to check that premise on the machine. */
int ll_decode_attention_xcc_probe(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                  int64_t head_dim, int64_t max_len_in_batch, int32_t* out,
                                  int64_t out_len, hipStream_t stream);
/* enable != 0 (the default): the split stage merges its splits itself when
 * the shape allows; 0: every split call merges in a separate kernel, which
 * needs no XCD premise (the runner switches it off when the probe above
 * finds the premise broken). Process-wide; returns the previous setting. No
 * reference counterpart. */
int ll_decode_attention_set_same_launch_merge(int enable);

/* NoPad varlen causal prefill attention reading K/V through the slot table,
 * with an optional shared (prompt-cache) prefix per request.
 * b_shared_seq_len == NULL replaces context_attention_fwd_with_no_pad_and_kv_cache
 *   (litelang/kernel/develop_flash_attn/flash_attn_v2.py:513-566);
 * b_shared_seq_len != NULL replaces
 *   context_attention_fwd_with_no_pad_and_kv_cache_and_prompt_cache
 *   (flash_attn_v2.py:699-762).
 * q / o [T, q_heads, head_dim] hold, for request b, the rows
 * b_start_loc[b] .. b_start_loc[b] + (b_seq_len[b] - shared[b]) - 1; the keys
 * are the first b_seq_len[b] slots of row b_req_idx[b] of req_to_tokens.
 * The bf16/fp16, head_dim 64/128 path rejects (LL_ERR_ARG) launches of 2^31
 * or more work items (query-row blocks x requests x KV heads x head groups). */
int ll_prefill_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_h,
                         const void* k_cache, int64_t k_stride_tok, int64_t k_stride_head,
                         const void* v_cache, int64_t v_stride_tok, int64_t v_stride_head,
                         void* out, int64_t out_stride_tok, int64_t out_stride_h,
                         const int32_t* req_to_tokens, int64_t req_to_tokens_stride,
                         const void* b_req_idx, int req_idx_i64, const void* b_start_loc,
                         int start_loc_i64, const void* b_seq_len, int seq_len_i64,
                         const void* b_shared_seq_len, int shared_i64, int64_t batch,
                         int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                         int64_t max_input_len, float sm_scale, int dtype, hipStream_t stream);

/* ------------------------------------------------------------- elementwise */

/* RMSNorm over rows: out = (x / sqrt(mean(x^2) + eps)) * gamma in fp32.
 * Replaces rmsnorm (litelang/kernel/develop_rmsnorm/rms_norm.py:71-98).
 * If residual != NULL, x is first updated in place to x + residual (rounded
 * to dtype) and the updated x is normalised: this fuses the residual add_
 * of transformer_layer.py:69,76 into the following norm. */
int ll_rmsnorm(void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
               const void* gamma, void* out, int64_t out_row_stride, int64_t M, int64_t N,
               float eps, int dtype, hipStream_t stream);

/* In-place rotate-half RoPE on q [T, q_heads, D] and k [T, k_heads, D] with
 * per-token cos/sin [T, D/2] (cs_dtype may differ from dtype).
 * Replaces rotary_emb_fwd (litelang/kernel/develop_rope/rope.py:154-198). */
int ll_rotary_emb(void* q, int64_t q_tok_stride, int64_t q_head_stride, int64_t q_heads, void* k,
                  int64_t k_tok_stride, int64_t k_head_stride, int64_t k_heads, const void* cos,
                  int64_t cos_tok_stride, const void* sin, int64_t sin_tok_stride, int64_t ntok,
                  int64_t head_dim, int dtype, int cs_dtype, hipStream_t stream);

/* Fused RoPE + KV-cache scatter for one layer: rotates the q heads of the
 * projection output qkv [T, (q_heads + 2*kv_heads)*D] in place, and writes
 * rotated K and plain V to pool_layer[slots[t], 0:2*kv_heads, :].
 * Replaces the index_select + rotary_emb_fwd + gather/index_put sequence of
 *   litelang/models/qwen2/layer/transformer_layer.py:102-115,142-143. */
int ll_rope_kv_scatter(void* qkv, int64_t qkv_row_stride, int64_t ntok, int64_t q_heads,
                       int64_t kv_heads, int64_t head_dim, const void* positions,
                       int positions_i64, const void* cos_table, const void* sin_table,
                       int64_t table_row_stride, int cs_dtype, const int32_t* slots,
                       void* pool_layer, int64_t pool_slot_stride, int64_t pool_head_stride,
                       int dtype, hipStream_t stream);

/* pool[slots[t], h, :] = src[t, h, :] (plain KV write, no RoPE).
 * Replaces the index_put of transformer_layer.py:143 when K is already rotated. */
int ll_kv_store(const void* src, int64_t src_tok_stride, int64_t src_head_stride, int64_t heads,
                int64_t head_dim, const int32_t* slots, void* pool, int64_t pool_slot_stride,
                int64_t pool_head_stride, int64_t ntok, int dtype, hipStream_t stream);

/* out[m, n] = up * dtype(silu(gate)), gate = x[m, n], up = x[m, N + n];
 * out may alias x (in-place over the gate half, as the reference).
 * Replaces silu_and_mul_fwd
 *   (litelang/kernel/develop_silu_and_mul/silu_and_mul.py:54-78). */
int ll_silu_and_mul(const void* x, int64_t x_row_stride, void* out, int64_t out_row_stride,
                    int64_t M, int64_t N, int dtype, hipStream_t stream);

/* ll_embedding followed by ll_rmsnorm (no residual) in one launch, bit for
 * bit: h[t] = table[ids[t]], out[t] = rmsnorm(h[t]) * gamma. Replaces
 *   Qwen2PreLayer.Forward (pre_layer.py:15-19) + the first layer's rmsnorm
 *   (transformer_layer.py:87). Ids are clamped into [0, vocab) as in
 *   ll_embedding. */
int ll_embedding_rmsnorm(const void* table, int64_t table_row_stride, int64_t vocab,
                         const void* ids, int ids_i64, void* h, int64_t h_row_stride,
                         const void* gamma, void* out, int64_t out_row_stride, int64_t ntok,
                         int64_t hidden, float eps, int dtype, hipStream_t stream);
/* ll_embedding_rmsnorm that also adds 1 to *epoch (ntok >= 1): the decode
 * step's first launch advances the epoch that the step's
 * ll_add_rmsnorm_qkv_splitk calls read, so the step needs no launch of its
 * own for it. With a non-NULL req_to_tokens the same launch also does
 * ll_assign_slots(req_to_tokens, req_to_tokens_stride, slots, rows, cols,
 * ntok), the step's slot-table update (again no launch of its own). Same
 * reference lines as ll_embedding_rmsnorm and ll_assign_slots. */
int ll_embedding_rmsnorm_epoch(const void* table, int64_t table_row_stride, int64_t vocab,
                               const void* ids, int ids_i64, void* h, int64_t h_row_stride,
                               const void* gamma, void* out, int64_t out_row_stride,
                               int64_t ntok, int64_t hidden, float eps, int dtype,
                               uint32_t* epoch, int32_t* req_to_tokens,
                               int64_t req_to_tokens_stride, const int32_t* slots,
                               const int32_t* rows, const int32_t* cols, hipStream_t stream);
/* out[t, :] = table[ids[t], :].
 * Replaces torch.embedding in Qwen2PreLayer.Forward
 *   (litelang/models/qwen2/layer/pre_layer.py:15-19).
 * An id outside [0, vocab) is clamped into it so the read stays inside the
 * table (torch.embedding raises instead; the runner rejects such ids on the
 * host when a request is admitted). */
int ll_embedding(const void* table, int64_t table_row_stride, int64_t vocab, const void* ids,
                 int ids_i64, void* out, int64_t out_row_stride, int64_t ntok, int64_t hidden,
                 int dtype, hipStream_t stream);

/* out[m] = first index of max(x[m, :]) (int64).
 * Replaces logits.argmax(dim=-1) (litelang/models/qwen2/layer/post_layer.py:75-77). */
int64_t ll_argmax_workspace_size(int64_t M, int64_t N);
int ll_argmax(const void* x, int64_t x_row_stride, int64_t M, int64_t N, int64_t* out,
              void* workspace, int64_t workspace_bytes, int dtype, hipStream_t stream);
/* ll_argmax, except that every out[m] is -1 when *status is nonzero (status:
 * the decode step's error word, ll_decode_sync_error_offset() bytes into the
 * sync words). -1 is no token id: a runner reading the tokens raises on it,
 * so a decode step whose fused launch gave up a flag wait is never taken for
 * a valid one. Same reference line as ll_argmax. */
int ll_argmax_status(const void* x, int64_t x_row_stride, int64_t M, int64_t N, int64_t* out,
                     void* workspace, int64_t workspace_bytes, int dtype, const uint32_t* status,
                     hipStream_t stream);

/* req_to_tokens[rows[i], cols[i]] = slots[i] for i < n (int32 device arrays).
 * Replaces the slot-table writes of PageCache.alloc_token_idxs and add_refs
 *   (litelang/models/cache.py:238-248, 284-285); the host keeps the free-slot
 * stack and computes (slot, row, col) exactly as the reference does. */
int ll_assign_slots(int32_t* req_to_tokens, int64_t req_to_tokens_stride, const int32_t* slots,
                    const int32_t* rows, const int32_t* cols, int64_t n, hipStream_t stream);

/* ------------------------------------------------------------------- GEMM */

/* Prefill tile GEMMs (256 x 256 output tiles on MFMA, see gemm_tiles.hip).
 * ll_gemm_tiled: Y[M, N] = T(X[M, K] . W[N, K]^T + bias[N]) in bf16/fp16 with
 * fp32 accumulation; needs N % 4 == 0, K % 32 == 0 and 16-byte aligned rows.
 * Replaces torch.addmm / torch.mm of the reference's prefill projections
 * (transformer_layer.py:80,82,95-109,193); ll_gemm uses it for M > 64.
 * ll_gemm_tiled_supported returns 1 when ll_gemm_tiled takes the shape. */
int ll_gemm_tiled_supported(int64_t M, int64_t N, int64_t K, int dtype);
int ll_gemm_tiled(const void* X, int64_t ldx, const void* W, int64_t ldw, const void* bias,
                  void* Y, int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype,
                  hipStream_t stream);

/* Copy of a [gate; up] weight ([2I, K], I % 128 == 0, elem_bytes 2 or 1)
 * with its rows interleaved in 64-row blocks (gate c..c+63, up c..c+63,
 * ...), the layout ll_gemm_gate_up_silu_tiled and
 * ll_gemm_i8_gate_up_silu_tiled read. No reference counterpart (a layout of
 * the weights load_weights.py:110,160 concatenates). */
int ll_gemm_interleave_gate_up(const void* W, int64_t ldw, int64_t I, int64_t K,
                               int64_t elem_bytes, void* out, hipStream_t stream);

/* Y[M, I] = T(up) * T(silu(T(gate))) (the rounding of ll_silu_and_mul) of
 * gate = X . Wg^T, up = X . Wu^T from the interleaved weight, in one launch:
 * the prefill gate/up projection and silu_and_mul_fwd
 * (transformer_layer.py:80-81, silu_and_mul.py:54-78) without the [M, 2I]
 * intermediate. */
int ll_gemm_gate_up_silu_tiled(const void* X, int64_t ldx, const void* W_il, int64_t M,
                               int64_t I, int64_t K, int dtype, void* Y, int64_t ldy,
                               hipStream_t stream);

/* W8A8 prefill: Y[M, N] = out(fp32(int8(X) . int8(W)^T) * s_tok[m] *
 * fp32(s_ch[n]) (+ bias[n])), the exact int32 sums dequantised as
 * ll_dequant_splitk does; out_dtype bf16/fp16 (bias allowed, in that dtype)
 * or fp32. K % 64 == 0. No reference counterpart (the reference's
 * SmoothQuant layer, quantize/smooth_quant/layer.py:19-59, has no forward). */
int ll_gemm_i8_tiled(const int8_t* Xq, int64_t ldx, const float* s_tok, const int8_t* Wq,
                     int64_t ldw, const void* s_ch, int s_ch_dtype, const void* bias, void* Y,
                     int64_t ldy, int64_t M, int64_t N, int64_t K, int out_dtype,
                     hipStream_t stream);
/* The raw int32 sums of the same product (Y int32 [M, N]). */
int ll_gemm_i8_i32_tiled(const int8_t* Xq, int64_t ldx, const int8_t* Wq, int64_t ldw,
                         int32_t* Y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                         hipStream_t stream);
/* The same int32 sums for any shape: the tile kernel where its layout holds
 * (K % 64 == 0, N % 4 == 0, 16 B aligned rows), else a plain int8
 * dot-product kernel. The int8 x int8 -> int32 product of the W8A8 prefill
 * (no reference counterpart, as ll_gemm_i8_tiled). */
int ll_gemm_i8_i32(const int8_t* Xq, int64_t ldx, const int8_t* Wq, int64_t ldw, int32_t* Y,
                   int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t stream);
/* ll_gemm_gate_up_silu_tiled for the W8A8 runtime: both halves dequantised
 * as in ll_gemm_i8_tiled (s_ch holds the [gate; up] channel scales in the
 * original order), then SiLU_and_Mul into Y (bf16/fp16). */
int ll_gemm_i8_gate_up_silu_tiled(const int8_t* Xq, int64_t ldx, const float* s_tok,
                                  const int8_t* Wq_il, const void* s_ch, int s_ch_dtype,
                                  int64_t M, int64_t I, int64_t K, int out_dtype, void* Y,
                                  int64_t ldy, hipStream_t stream);

/* Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]) with fp32 accumulation.
 * W is the nn.Linear layout [out, in]. Replaces the torch.addmm / torch.mm /
 * matmul projections of transformer_layer.py:80,82,95-109,193 and the lm_head
 * product of post_layer.py:20-22 (the reference keeps W pre-transposed
 * [in, out]; this library keeps [out, in] so both MFMA operands stream
 * 16-byte k-contiguous rows). X rows may be strided; Y is written with
 * row stride ldy. For M <= 64 with narrow N the product is split over K and
 * needs a workspace of ll_gemm_workspace_size(M, N, K) bytes (0 otherwise). */
int64_t ll_gemm_workspace_size(int64_t M, int64_t N, int64_t K);
int ll_gemm(const void* X, int64_t ldx, const void* W, int64_t ldw, const void* bias, void* Y,
            int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype, void* workspace,
            int64_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------- decode-step split-K path
 * The M <= 64 projections of a decode step write fp32 partial sums
 * part[s][m][n] (s < ll_gemm_splitk_count(M, N, K)); the consumer kernels
 * below sum them in a fixed order, store the projection output in `dtype`
 * (bit-identical to the unfused product's rounding) and fuse the next op of
 * the layer. They replace the same reference operations as the entry points
 * they are named after: the projections of transformer_layer.py:80,82,95-109,193
 * followed by, respectively, the residual add_ + rmsnorm (:69-71,76,61),
 * silu_and_mul_fwd (:81) and rotary_emb_fwd + KV-cache write (:112-115,142-143). */
int ll_gemm_splitk_count(int64_t M, int64_t N, int64_t K);
int ll_gemm_splitk(const void* X, int64_t ldx, const void* W, int64_t ldw, int64_t M, int64_t N,
                   int64_t K, int dtype, float* part, int64_t part_bytes, hipStream_t stream);
/* h = dtype(h + dtype(sum part)); out = rmsnorm(h) * gamma (h updated in place).
 * N a multiple of 4, at most 8192; 1 <= splits < 65536 (also for the _i32
 * form below). */
int ll_add_rmsnorm_splitk(void* h, int64_t h_row_stride, const float* part, int splits,
                          const void* gamma, void* out, int64_t out_row_stride, int64_t M,
                          int64_t N, float eps, int dtype, hipStream_t stream);
/* add + RMSNorm fused with the next layer's QKV projection, one launch
 * (replaces ll_add_rmsnorm_splitk + ll_gemm_splitk_packed on the decode
 * step: litelang/models/qwen2/layer/transformer_layer.py:77 (residual + the
 * post-MLP norm's successor) and :61, :95-109 (input norm, q/k/v addmm)).
 * h and x as ll_add_rmsnorm_splitk(h, ld_h, part, splits, gamma, x, hidden,
 * ...) leaves them, bit for bit; qkv_part [qkv_splits][M][nqkv] gets the
 * fp32 split-K partials of x . W^T from the ll_gemm_pack image of the
 * [nqkv, hidden] weight, qkv_splits = ll_add_rmsnorm_qkv_splits(M, hidden,
 * nqkv) (this kernel's own k split, so they sum in another order than
 * ll_gemm_splitk_packed's). qkv_part may be part. Norm and GEMM workgroups
 * meet on flags in `sync` (ll_decode_sync_bytes() bytes, zeroed once); a
 * call's flags hold *epoch * 256 + tag + 1, which the caller keeps distinct
 * from every earlier call's on the same sync words (a new *epoch per decode
 * step, the layer index < 256 as tag). Calls on one sync buffer must not
 * overlap. Every flag wait is bounded (ll_decode_sync_set_spin_limit); a
 * QKV workgroup whose wait gives up stores nothing and sets the error word
 * (ll_decode_sync_error_offset() bytes into `sync`), which stays set until
 * ll_decode_sync_status resets it and does not affect later calls' waits. */
int ll_add_rmsnorm_qkv_splits(int64_t M, int64_t hidden, int64_t nqkv); /* 0: not covered */
int ll_add_rmsnorm_qkv_splitk(void* h, int64_t ld_h, const float* part, int splits,
                              const void* gamma, float eps, void* x, const void* wqkv_packed,
                              float* qkv_part, int64_t qkv_part_bytes, int64_t M, int64_t hidden,
                              int64_t nqkv, int dtype, void* sync, const uint32_t* epoch,
                              uint32_t tag, hipStream_t stream);
int64_t ll_decode_sync_bytes(void);
int64_t ll_decode_sync_error_offset(void);
/* Polls a flag wait makes before it gives up, process-wide (0: the default,
 * 2^18). A negative value -n is a test mode: the waits look for a flag value
 * no producer writes and give up after n polls, so every consumer gives up
 * while every kernel still exits normally. No reference counterpart. */
int ll_decode_sync_set_spin_limit(int polls);
/* 1 when a flag wait gave up since the last reset (outputs then invalid), else
 * 0; reset != 0 clears the sync words after such a failure (synchronises
 * the stream) */
int ll_decode_sync_status(void* sync, int reset, hipStream_t stream);
/* part covers [M, 2N] (gate then up); out[m, n] = up * dtype(silu(gate)) */
int ll_silu_and_mul_splitk(const float* part, int splits, void* out, int64_t out_row_stride,
                           int64_t M, int64_t N, int dtype, hipStream_t stream);
/* W8A8 forms of the two consumers above (no reference counterpart: they fold
 * ll_dequant_splitk into add+RMSNorm and SiLU_and_Mul for the int8 decode
 * layer): int32 partials [splits][M][N] ([M][2N] for SiLU) with per-row
 * activation scales s_tok [M] and per-column weight scales s_ch of
 * s_ch_dtype (4-byte aligned), dequantised as ll_dequant_splitk does. With q_out (and
 * q_scale), the RMSNorm output is also quantised per token for the next
 * projection, with ll_quant_per_token's rule, into int8 q_out [M, ldq] and
 * fp32 q_scale [M]; both null skips it. */
int ll_add_rmsnorm_splitk_i32(void* h, int64_t h_row_stride, const int32_t* part, int splits,
                              const float* s_tok, const void* s_ch, int s_ch_dtype,
                              const void* gamma, void* out, int64_t out_row_stride, int64_t M,
                              int64_t N, float eps, int dtype, int8_t* q_out, int64_t ldq,
                              float* q_scale, hipStream_t stream);
int ll_silu_and_mul_splitk_i32(const int32_t* part, int splits, const float* s_tok,
                               const void* s_ch, int s_ch_dtype, void* out,
                               int64_t out_row_stride, int64_t M, int64_t N, int dtype,
                               hipStream_t stream);
/* part covers [T, (q_heads + 2*kv_heads)*D]; adds bias, rotates q into q_out
 * [T, q_heads*D] and writes rotated K and V to pool_layer[slots[t]] */
int ll_rope_kv_scatter_splitk(const float* part, int splits, const void* bias, void* q_out,
                              int64_t q_row_stride, int64_t ntok, int64_t q_heads,
                              int64_t kv_heads, int64_t head_dim, const void* positions,
                              int positions_i64, const void* cos_table, const void* sin_table,
                              int64_t table_row_stride, int cs_dtype, const int32_t* slots,
                              void* pool_layer, int64_t pool_slot_stride,
                              int64_t pool_head_stride, int dtype, hipStream_t stream);
/* ll_rope_kv_scatter_splitk followed by ll_decode_attention in one launch
 * (plus the split merge): replaces, for one decode step,
 *   rotary_emb_fwd + the KV-cache write (transformer_layer.py:112-115,142-160)
 *   and token_decode_attention_flash_decoding (flash_decoding.py:262-312).
 * qkv_part [qkv_splits][batch][(q_heads + 2*kv_heads)*head_dim] fp32 partials
 * of the QKV projection; every workgroup rebuilds its query heads from them,
 * and the one holding a sequence's last tile writes the new token's rotated K
 * and V to k_cache/v_cache[new_slots[b]]. Results (out and the pool) are bit
 * identical to the two-call sequence. Precondition: new_slots[b] is the entry
 * req_to_tokens[b_req_idx[b], b_seq_len[b] - 1] and appears in no other
 * sequence's first b_seq_len entries (what a decode step guarantees).
 * bf16/fp16, head_dim 64 or 128, q_heads/kv_heads <= 16, fp32 cos/sin tables;
 * other shapes use the two calls. workspace: ll_decode_attention_workspace_size.
 * The same-launch split merge waits for the other splits' partials with a
 * bound (the decode step's spin setting, ll_decode_sync_set_spin_limit; its
 * test mode makes every such wait give up). A merge that gives up stores NaN
 * rows and sets *error_word to 1 (error_word may be NULL), the decode step's
 * error word (ll_decode_sync_error_offset), as the fused norm launch does. */
int ll_decode_attention_rope_splitk(
    const float* qkv_part, int qkv_splits, const void* qkv_bias, const void* positions,
    int positions_i64, const void* cos_table, const void* sin_table, int64_t table_row_stride,
    int cs_dtype, const int32_t* new_slots, void* k_cache, int64_t k_stride_tok,
    int64_t k_stride_head, void* v_cache, int64_t v_stride_tok, int64_t v_stride_head,
    const int32_t* req_to_tokens, int64_t req_to_tokens_stride, const void* b_req_idx,
    int req_idx_i64, const void* b_seq_len, int seq_len_i64, void* out, int64_t out_stride_b,
    int64_t out_stride_h, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t max_len_in_batch, float sm_scale, int dtype, void* workspace,
    int64_t workspace_bytes, uint32_t* error_word, hipStream_t stream);
/* The same with the W8A8 projection's int32 partials
 * [qkv_splits][batch][(q_heads + 2*kv_heads)*head_dim] and their scales in
 * place of fp32 partials: each column is dequantised as in ll_dequant_splitk
 * (fp32(sum) * s_tok[b] * fp32(s_ch[col]), s_ch of s_ch_dtype, 4-byte aligned) and then
 * treated exactly as the fp32 entry point treats its partial sums. With q_out
 * (and q_scale; out rows contiguous, ldq >= q_heads*head_dim) the stored
 * output rows are also quantised for the o_proj, by ll_quant_per_token's rule
 * or with the calibrated scale *q_static (as ll_quant_static), in the split
 * merge when there is one. */
int ll_decode_attention_rope_splitk_i32(
    const int32_t* qkv_part, int qkv_splits, const float* s_tok, const void* s_ch, int s_ch_dtype,
    const void* qkv_bias, const void* positions, int positions_i64, const void* cos_table,
    const void* sin_table, int64_t table_row_stride, int cs_dtype, const int32_t* new_slots,
    void* k_cache, int64_t k_stride_tok, int64_t k_stride_head, void* v_cache,
    int64_t v_stride_tok, int64_t v_stride_head, const int32_t* req_to_tokens,
    int64_t req_to_tokens_stride, const void* b_req_idx, int req_idx_i64, const void* b_seq_len,
    int seq_len_i64, void* out, int64_t out_stride_b, int64_t out_stride_h, int64_t batch,
    int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t max_len_in_batch,
    float sm_scale, int dtype, void* workspace, int64_t workspace_bytes, const float* q_static,
    int8_t* q_out, int64_t ldq, float* q_scale, uint32_t* error_word, hipStream_t stream);

/* Pre-packed weights for the decode projections (no reference counterpart:
 * a layout of the same nn.Linear weight [N, K], chosen for MI355X). The
 * packed image stores every (row tile, 128-column chunk) stage of the
 * weight-streaming kernel as one contiguous, already swizzled block of
 * tile_rows * 256 bytes, blocks ordered chunk-major, so the workgroups of a
 * launch stream neighbouring blocks instead of rows 2K bytes apart. The tile
 * height (ll_gemm_packed_tile_rows: 64, or 128 when one split covers K and
 * there are more than 256 64-row tiles) is a function of (N, K) only. K % 128
 * == 0; rows are padded to a multiple of the tile height with zeros.
 * ll_gemm_packed_bytes returns the size (0 if K % 128 != 0). The packed GEMMs
 * compute what ll_gemm_splitk / ll_gemm compute for M <= 64 from the unpacked
 * weight, with Wp in place of W: same split count and split boundaries (the
 * 128-column chunks inside a split may be summed in another order). */
int ll_gemm_packed_tile_rows(int64_t N, int64_t K);
int64_t ll_gemm_packed_bytes(int64_t N, int64_t K);
int ll_gemm_pack(const void* W, int64_t ldw, int64_t N, int64_t K, int dtype, void* Wp,
                 int64_t wp_bytes, hipStream_t stream);
int ll_gemm_splitk_packed(const void* X, int64_t ldx, const void* Wp, int64_t M, int64_t N,
                          int64_t K, int dtype, float* part, int64_t part_bytes,
                          hipStream_t stream);
int ll_gemm_packed(const void* X, int64_t ldx, const void* Wp, const void* bias, void* Y,
                   int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype, void* workspace,
                   int64_t workspace_bytes, hipStream_t stream);
/* ll_gemm_packed with fp32 output Y [M, N] (the sums, + bias, never rounded
 * to the weight dtype): the decode step's logits, argmaxed unrounded (the
 * reference argmaxes its own fp16 logits, post_layer.py:20-22,75-77; fp32
 * logits keep every one of them apart that fp16 keeps apart). */
int ll_gemm_packed_f32(const void* X, int64_t ldx, const void* Wp, const void* bias, float* Y,
                       int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype, void* workspace,
                       int64_t workspace_bytes, hipStream_t stream);
/* The lm_head and the greedy pick of the post layer in one call (replaces
 * post_layer.py:20-22 + the argmax at :77 for M <= 64): Y = ll_gemm_packed_f32's
 * fp32 logits, tokens[m] = the first index of row m's maximum, exactly as
 * ll_argmax on Y (-1 in every row while *status is nonzero, as
 * ll_argmax_status; status may be NULL). For one-split plans the first argmax
 * pass runs in the GEMM's epilogue (per-tile maxima; with 128-row tiles, no
 * bias and N, ldy multiples of 4, the GEMM is a persistent grid of at most
 * one workgroup per CU), otherwise the GEMM and ll_argmax run one after the
 * other. Workspace:
 * ll_gemm_packed_f32_argmax_workspace_size(M, N, K) bytes. */
int64_t ll_gemm_packed_f32_argmax_workspace_size(int64_t M, int64_t N, int64_t K);
int ll_gemm_packed_f32_argmax(const void* X, int64_t ldx, const void* Wp, const void* bias,
                              float* Y, int64_t ldy, int64_t M, int64_t N, int64_t K, int dtype,
                              int64_t* tokens, const uint32_t* status, void* workspace,
                              int64_t workspace_bytes, hipStream_t stream);
/* Gate/up projection fused with SiLU_and_Mul (replaces the gate_up projection
 * plus silu_and_mul_fwd of transformer_layer.py:80-81 for M <= 64). The weight
 * is [gate; up] ([2I, K], the reference's two nn.Linear weights stacked);
 * ll_gemm_pack_gate_up packs it so that every tile of R rows
 * (ll_gemm_packed_gate_up_tile_rows: 64 when I <= 8192, else 96 when
 * I <= 12288, else 128) holds R/2 gate
 * rows and the R/2 up rows of the same channels (size from
 * ll_gemm_packed_gate_up_bytes, 0 if K % 128 != 0). act[m, c] =
 * dtype(dtype(up) * dtype(silu(dtype(gate)))), the rounding sequence of
 * ll_silu_and_mul_splitk, from one split (full fp32 sums). */
int ll_gemm_packed_gate_up_tile_rows(int64_t I);
int64_t ll_gemm_packed_gate_up_bytes(int64_t I, int64_t K);
int ll_gemm_pack_gate_up(const void* W, int64_t ldw, int64_t I, int64_t K, int dtype, void* Wp,
                         int64_t wp_bytes, hipStream_t stream);
int ll_gemm_gate_up_silu_packed(const void* X, int64_t ldx, const void* Wp, int64_t M, int64_t I,
                                int64_t K, int dtype, void* act, int64_t ld_act,
                                hipStream_t stream);
/* ---------------------------------------------------------------- W8A8 */

/* Symmetric int8 quantisation (replaces quantize_weight_per_channel_absmax,
 * quantize/smooth_quant/layer.py:5-16, on its float path):
 * scale[o] = dtype(max_i |W[o, i]| / 127), Q[o, i] = clamp(round_half_even(
 * fp32(W[o, i]) / fp32(scale[o])), -128, 127); an all-zero row gives Q = 0. */
int ll_quant_weight_per_channel(const void* W, int64_t ldw, int64_t N, int64_t K, int dtype,
                                int8_t* Q, int64_t ldq, void* scale, hipStream_t stream);
/* Dynamic per-token activation quantisation (no reference counterpart: the
 * reference never quantises activations at run time): scale[t] =
 * max_k |X[t, k]| / 127 in fp32 (1 for an all-zero row), Q = clamp(
 * round_half_even(X / scale), -128, 127). */
int ll_quant_per_token(const void* X, int64_t ldx, int64_t M, int64_t K, int dtype, int8_t* Q,
                       int64_t ldq, float* scale, hipStream_t stream);
/* int8 weight streaming for M <= 64 (no reference counterpart; the runtime of
 * the reference's W8A8BFP32OFP32Linear, smooth_quant/layer.py:19-59, which has
 * no forward). Wp is the packed image of an int8 [N, K] weight
 * (ll_gemm_i8_pack; K % 256 == 0; size ll_gemm_i8_packed_bytes; stages of
 * 256 int8 columns, tile height chosen as for the 16-bit layout: 128 rows
 * when one split covers K and 64-row tiles would outnumber the CUs); part
 * receives exact int32 partial sums [s][M][N], s < ll_gemm_i8_splitk_count. */
int64_t ll_gemm_i8_packed_bytes(int64_t N, int64_t K);
int ll_gemm_i8_pack(const int8_t* Wq, int64_t ldw, int64_t N, int64_t K, void* Wp,
                    int64_t wp_bytes, hipStream_t stream);
int ll_gemm_i8_splitk_count(int64_t M, int64_t N, int64_t K);
int ll_gemm_i8_splitk_packed(const int8_t* Xq, int64_t ldx, const void* Wp, int64_t M, int64_t N,
                             int64_t K, int32_t* part, int64_t part_bytes, hipStream_t stream);
/* int8 gate/up projection fused with dequantisation and SiLU_and_Mul (the
 * int8 counterpart of ll_gemm_gate_up_silu_packed, for M <= 64): Wp is the
 * int8 [gate; up] weight [2I, K] packed by ll_gemm_i8_pack_gate_up (tiles of
 * R/2 gate and the same R/2 up rows, R as ll_gemm_packed_gate_up_tile_rows),
 * s_tok [M] the activation scales of Xq, s_ch [2I] the channel scales (gate
 * then up). act[m, c] = dtype(dtype(u) * dtype(silu(dtype(g)))) with
 * g = fp32(acc) * s_tok[m] * fp32(s_ch[c]) and u likewise with s_ch[I + c]:
 * ll_silu_and_mul_splitk_i32 on the one-split int32 product, bit for bit. */
int64_t ll_gemm_i8_packed_gate_up_bytes(int64_t I, int64_t K);
int ll_gemm_i8_pack_gate_up(const int8_t* Wq, int64_t ldw, int64_t I, int64_t K, void* Wp,
                            int64_t wp_bytes, hipStream_t stream);
int ll_gemm_i8_gate_up_silu_packed(const int8_t* Xq, int64_t ldx, const void* Wp, int64_t M,
                                   int64_t I, int64_t K, const float* s_tok, const void* s_ch,
                                   int s_ch_dtype, void* act, int64_t ld_act, int dtype,
                                   hipStream_t stream);
/* Static per-tensor activation quantisation with a calibrated input scale
 * (the quant_scale buffer of W8A8BFP32OFP32LinearWithQuantScale,
 * quantize/smooth_quant/layer.py:63-94, whose runtime the reference never
 * wrote): Q[m, k] = clamp(round_half_even(fp32(X[m, k]) / s), -128, 127) with
 * s = *scale (device fp32, > 0); s_tok[m] = s for ll_dequant_splitk. */
int ll_quant_static(const void* X, int64_t ldx, int64_t M, int64_t K, int dtype,
                    const float* scale, int8_t* Q, int64_t ldq, float* s_tok,
                    hipStream_t stream);
/* out[m][n] = fp32(sum_s part[s][m][n]) * s_tok[m] * fp32(s_ch[n]): the fp32
 * single-split partial the fused consumers above read (N % 4 == 0). */
int ll_dequant_splitk(const int32_t* part, int splits, const float* s_tok, const void* s_ch,
                      int s_ch_dtype, float* out, int64_t M, int64_t N, hipStream_t stream);

/* ---- Measurement probes (no counterpart in the reference; bench.py
 * --attention-floor times the first two against the decode attention,
 * bench.py --launch-floor the third).
 * ll_probe_stream_read: a plain streaming read of `bytes` contiguous bytes
 * (16 B aligned) by `workgroups` workgroups of 256 threads.
 * ll_probe_kv_gather: the K/V rows ll_decode_attention reads, through the
 * same slot table, request rows and lengths, on its split grid (nsplit as
 * the attention chooses it), with no arithmetic: mode 0 into registers,
 * mode 1 copied into LDS. `sink` is a device word written only in a case no
 * input produces (it keeps the loads live). */
int ll_probe_stream_read(const void* src, int64_t bytes, int64_t workgroups, uint32_t* sink,
                         hipStream_t stream);
int ll_probe_kv_gather(const void* k_cache, int64_t k_stride_tok, int64_t k_stride_head,
                       const void* v_cache, int64_t v_stride_tok, int64_t v_stride_head,
                       const int32_t* req_to_tokens, int64_t req_to_tokens_stride,
                       const void* b_req_idx, int req_idx_i64, const void* b_seq_len,
                       int seq_len_i64, int64_t batch, int64_t kv_heads, int64_t head_dim,
                       int64_t elem_bytes, int64_t max_len_in_batch, int64_t nsplit, int mode,
                       uint32_t* sink, hipStream_t stream);
/* ll_probe_launch: `workgroups` workgroups of 512 threads that write
 * write_bytes (16 B aligned; 0: an empty kernel) to dst with 16-byte stores. */
int ll_probe_launch(void* dst, int64_t write_bytes, int64_t workgroups, hipStream_t stream);
/* The split count ll_decode_attention uses for this shape (1: no split). */
int ll_decode_attention_split_count(int64_t batch, int64_t kv_heads, int64_t head_dim,
                                    int64_t max_len_in_batch);

#ifdef __cplusplus
}
#endif

#endif /* LITELANG_AMD_H */
