/*
 * qwen36_hip.h -- C-ABI of the MI355X (gfx950) attention hot-path library.
 *
 * This library replaces the pybind11 module `qwen36_fp8` of the reference
 * (src/csrc/fp8_linear.cpp:5-21, declared in src/csrc/fp8_linear.h:99-119) and
 * its loader (src/cuda_loader.py:40-54) for the attention hot path.  Every
 * entry point takes plain device pointers, sizes, element strides, dtype codes
 * and a hipStream_t; none takes or returns a torch type.  Callers allocate all
 * outputs and workspaces; the library never allocates device memory.
 *
 * Return value: 0 on success, non-zero on failure; qa_last_error() then holds
 * a message (per calling thread).  Shape/dtype errors are detected on the host
 * before any launch.
 *
 * Element strides are in elements of the tensor's own dtype.  The innermost
 * (head_dim / channel) axis is always contiguous.
 */
#ifndef QWEN36_HIP_H
#define QWEN36_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
enum {
  QA_F32 = 0,
  QA_BF16 = 1,
  QA_F16 = 2,
  QA_I32 = 3,
  QA_I64 = 4
};

/* Paged KV pool descriptor.
 *
 * Element (row b, kv head g, physical block p, slot t, dim d) lives at
 *   base_b + p*stride_block + g*stride_head + t*stride_token + d
 * where base_b = key + b*stride_batch, or row_key_ptrs[b] when the per-row
 * pointer arrays are given (the reference's list-of-pools form,
 * src/fp8_cuda.py:235-250).  The reference's per-request pool layout
 * (batch, heads, P, bs, D) (src/decode_state.py:37-44) and this library's
 * shared GQA-native pool (P, H_kv, bs, D) are both expressible.
 * With per-row pointer arrays and stride_head == 0, row b's head stride is
 * row_blocks[b]*stride_block: contiguous per-request pools
 * (1, heads, P_b, bs, D) of different P_b.
 * Physical ids outside [0, num_blocks) (or row_blocks[b]) are skipped.     */
typedef struct qa_paged_kv {
  void* key;
  void* value;
  const int64_t* row_key_ptrs;   /* device (B,) or NULL */
  const int64_t* row_value_ptrs; /* device (B,) or NULL */
  const int64_t* row_blocks;     /* device (B,) physical block counts or NULL */
  int64_t num_blocks;
  int64_t stride_batch;
  int64_t stride_block;
  int64_t stride_head;
  int64_t stride_token;
  int32_t kv_heads;
  int32_t dtype;                 /* QA_F32 or QA_BF16 */
} qa_paged_kv;

/* ---- library ---------------------------------------------------------- */
const char* qa_last_error(void);
int32_t qa_version(void);
const char* qa_arch(void);

/* Opt-in timing of each operation's main kernel with HIP events recorded on
 * the launch stream around the launch (no counterpart in the reference; used
 * by the benchmark for per-kernel roofline figures).  Enabling or disabling
 * clears the totals.  Labels: decode_partial_mfma, decode_partial_generic,
 * decode_combine, paged_prefill, chunk_gated_delta, gated_delta_step,
 * causal_conv1d, fp8_linear, fp8_linear_reduce, kv_reserve (and others).
 * qa_read_kernel_timing waits for the recorded events.                   */
void qa_set_kernel_timing(int32_t enabled);
int qa_read_kernel_timing(const char* label, double* total_ms, int64_t* launches);

/* ---- paged GQA decode ------------------------------------------------- */
/* Bytes of fp32 workspace the decode entry points need for these sizes.   */
int64_t qa_paged_attention_decode_workspace(int64_t batch, int32_t heads, int32_t head_dim,
                                            int64_t max_tokens, int32_t block_size);

/* Single-table decode.  Replaces `paged_attention_decode`
 * (src/fp8_cuda.py:217-232 -> src/csrc/fp8_linear.h:106-112,
 * src/csrc/fp8_linear_cuda.cu:1192-1266).  All `batch` rows read the same
 * block table (len table_len) and attend over `sequence_length` tokens of
 * their own pool row.  query/output: (batch, heads, head_dim) rows with
 * element strides q_stride_b / q_stride_h; output is contiguous.
 * scale <= 0 selects head_dim^-0.5 (src/csrc/fp8_linear_cuda.cu:912).     */
int qa_paged_attention_decode(const void* query, int32_t q_dtype, int64_t q_stride_b, int64_t q_stride_h,
                              int64_t batch, int32_t heads, int32_t head_dim,
                              const qa_paged_kv* kv,
                              const void* block_table, int32_t table_dtype, int64_t table_len,
                              int64_t sequence_length, int32_t block_size, float scale,
                              void* output, void* workspace, int64_t workspace_bytes,
                              hipStream_t stream);

/* Batched decode with per-row tables (B, max_blocks), -1 padded, and
 * per-row device lengths (int32 or int64).  Rows with length <= 0 produce
 * zeros.  Replaces `paged_attention_decode_batched`
 * (src/fp8_cuda.py:235-250 -> src/csrc/fp8_linear.h:113-119,
 * src/csrc/fp8_linear_cuda.cu:1269-1365).                                  */
int qa_paged_attention_decode_batched(const void* query, int32_t q_dtype, int64_t q_stride_b, int64_t q_stride_h,
                                      int64_t batch, int32_t heads, int32_t head_dim,
                                      const qa_paged_kv* kv,
                                      const void* block_tables, int32_t table_dtype, int64_t table_stride,
                                      int64_t max_blocks,
                                      const void* sequence_lengths, int32_t lengths_dtype,
                                      int32_t block_size, float scale,
                                      void* output, void* workspace, int64_t workspace_bytes,
                                      hipStream_t stream);

/* qa_paged_attention_decode_batched without a workspace argument: the split-K
 * partials live in a static device array of this library (32 MiB, one copy per
 * device, held until the process ends), so the call allocates nothing and
 * needs no caller memory beyond inputs and outputs.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Sizes whose
 * partials exceed 32 MiB are rejected (status 1, message names the bytes
 * needed); at D = 256 and 8 query heads per KV head the MFMA path fits about
 * 1,900 (row, KV head) groups.  Every call on a device shares that device's
 * array, and nothing in it needs to start at zero: calls that overlap on one
 * device (e.g. on two streams) race and must be serialised by the caller.   */
int qa_paged_attention_decode_batched_noalloc(const void* query, int32_t q_dtype, int64_t q_stride_b, int64_t q_stride_h,
                                              int64_t batch, int32_t heads, int32_t head_dim,
                                              const qa_paged_kv* kv,
                                              const void* block_tables, int32_t table_dtype, int64_t table_stride,
                                              int64_t max_blocks,
                                              const void* sequence_lengths, int32_t lengths_dtype,
                                              int32_t block_size, float scale, void* output,
                                              hipStream_t stream);

/* ---- paged KV cache --------------------------------------------------- */
/* Write `new_tokens` tokens of each row into its slots
 * (table[pos/bs], pos%bs) for pos = start_b .. start_b + count_b - 1.
 * key_new/value_new: (batch, kv_heads, new_tokens, head_dim) with element
 * strides (src_stride_b, src_stride_h, src_stride_s).  start positions are
 * per-row device values (int32/int64) or, when starts == NULL, start_scalar.
 * counts (device, may be NULL = all new_tokens) limits each row.  Same dtype
 * as the pool; a bit-exact copy.  Positions whose logical block is past
 * max_blocks or whose block id is invalid are not written.  Replaces FullAttentionCache.append_blocks
 * (src/decode_state.py:271-293).                                          */
int qa_paged_kv_append(const void* key_new, const void* value_new, int32_t dtype,
                       int64_t src_stride_b, int64_t src_stride_h, int64_t src_stride_s,
                       int64_t batch, int32_t kv_heads, int64_t new_tokens, int32_t head_dim,
                       const qa_paged_kv* kv,
                       const void* block_tables, int32_t table_dtype, int64_t table_stride,
                       int64_t max_blocks,
                       const void* starts, int32_t starts_dtype, int64_t start_scalar,
                       const void* counts, int32_t counts_dtype,
                       int32_t block_size, hipStream_t stream);

/* Dense logical-order copy of the first `valid` tokens of each row:
 * out (batch, kv_heads, valid, head_dim) contiguous.  Replaces
 * FullAttentionCache.as_tensors / _gather_blocks (src/decode_state.py:295-303,
 * 395-404).  Tokens whose block id is invalid are written as zeros.        */
int qa_paged_kv_gather(const qa_paged_kv* kv, int32_t head_dim, int64_t batch,
                       const void* block_tables, int32_t table_dtype, int64_t table_stride,
                       int64_t max_blocks, int64_t valid, int32_t block_size,
                       void* key_out, void* value_out, hipStream_t stream);

/* ---- fp8 E4M3 block-scaled linear ------------------------------------- */
/* y (rows, out_features) = x (rows, in_features) . W^T, W[n][k] =
 * E4M3(weight[n][k]) * scale[n/128][k/128]: weight (out, in) fp8 E4M3 (fn)
 * codes, row-major; scale (out/128, in/128) bf16; x float32 or bfloat16 rows
 * (x_stride elements apart, 16-byte aligned); y float32 or bfloat16.  Both
 * feature counts must be multiples of 128.  Weight values are converted
 * exactly, scales applied per 128-deep block in fp32.  fp32 x of fewer than 16
 * rows enters as a bf16 hi + lo pair (the reference's fp32 matvec regime),
 * of 16 rows or more rounded to fp16 (its fp16 GEMM regime, .cu:1411-1460); bf16
 * x as itself.  weight_packed = 1: weight is in qa_fp8_pack_weight's
 * order (same bytes, streamed contiguously).  workspace: qa_fp8_linear_workspace(rows, out, in) bytes
 * (0 when no K split is used; then it may be NULL).  Replaces
 * fp8_e4m3_bf16_linear (src/fp8_cuda.py:16-17 -> src/csrc/fp8_linear.h,
 * src/csrc/fp8_linear_cuda.cu:1368-1466) and the dequantised F.linear of
 * src/reference_ops.py:436-506.                                            */
int64_t qa_fp8_linear_workspace(int64_t rows, int64_t out_features, int64_t in_features);
/* Weight re-laid once (at load time) for streaming: 16-row x 128-column
 * tiles of 2 KB, consecutive along K, bytes in the order the products read
 * them; pass weight_packed = 1 with the result.  No counterpart in the
 * reference (its weights stay row-major).                                  */
int qa_fp8_pack_weight(const void* weight, void* packed, int64_t out_features, int64_t in_features,
                       hipStream_t stream);
int qa_fp8_linear(const void* x, int32_t x_dtype, int64_t x_stride, int64_t rows,
                  const void* weight, int32_t weight_packed, const void* scale,
                  int64_t out_features, int64_t in_features,
                  void* y, int32_t y_dtype, int64_t y_stride, void* workspace, int64_t workspace_bytes,
                  hipStream_t stream);

/* Device-side block reservation for a batched step (one kernel, no host
 * round trip, so a decode step can be captured in a HIP graph).  Row b grows
 * from lengths[b] to lengths[b] + n_b tokens (n_b = counts[b], or count_scalar
 * when counts == NULL); the logical blocks ceil(len/bs) .. ceil((len+n)/bs)-1
 * of its table get ids from the front of the free list, rows in order: the
 * lowest-free-id policy of PagedKVBlockPool.allocate (src/decode_state.py:72-78)
 * and of FullAttentionCache._grow_to's allocate calls (:365-374).  free_list
 * holds ascending ids; free_state (device int32[2]) = {head, count} marks
 * free_list[head .. head+count) as free and is advanced.  positions (may be
 * NULL) receives the old lengths (the append positions); lengths are advanced
 * in place.  All-or-nothing: status (device int32) = 0 on success, 1 not
 * enough free blocks, 2 a row would pass max_blocks, 3 corrupt free_state,
 * 4 negative or overflowing length/count -- then nothing else is written.
 * Replaces the host-side allocate + page_table_tensor rebuild of
 * src/decode_state.py:72-78,305-328 for the shared pool.                  */
int qa_paged_kv_reserve(void* block_tables, int32_t table_dtype, int64_t table_stride, int64_t max_blocks,
                        void* lengths, int32_t lengths_dtype, void* positions, int32_t positions_dtype,
                        const void* counts, int32_t counts_dtype, int64_t count_scalar, int64_t batch,
                        int32_t block_size, const int32_t* free_list, int64_t free_capacity,
                        int32_t* free_state, int32_t* status, hipStream_t stream);

/* ---- paged prefill ------------------------------------------------------ */
/* Causal attention of packed new tokens over their paged KV (prefix + the
 * new tokens, already appended): query (total_new, heads, head_dim) bf16
 * with element strides (q_stride_t, q_stride_h); cu_seqlens (batch+1) and
 * prefix_lens (batch) device index arrays (int32/int64); new token n of
 * sequence b sits at position prefix_lens[b] + n.  Optional gate
 * bf16 logits, element (n, h, d) at gate[n*gate_stride_t + h*gate_stride_h + d]
 * (gate_stride_h 0 means head_dim): out *= sigmoid(gate).  Writes
 * output (total_new, heads, head_dim) bf16 contiguous.  bf16 MFMA, head_dim
 * 128 or 256, block size 16, GQA group <= 8, one shared pool.  Replaces the
 * reference's dense multi-token fallback (src/tp_runtime.py:551-610 ->
 * :698-730; src/reference_ops.py:353-360) with a chunked paged kernel.      */
int qa_paged_attention_prefill(const void* query, int32_t q_dtype, int64_t q_stride_t, int64_t q_stride_h,
                               const void* cu_seqlens, const void* prefix_lens, int32_t idx_dtype,
                               int64_t batch, int64_t max_new, int32_t heads, int32_t head_dim,
                               const qa_paged_kv* kv, const void* block_tables, int32_t table_dtype,
                               int64_t table_stride, int64_t max_blocks, int32_t block_size, float scale,
                               const void* gate, int64_t gate_stride_t, int64_t gate_stride_h, void* output,
                               hipStream_t stream);

/* ---- full-attention prologue: q/k RMSNorm + partial RoPE + K/V append ---- */
/* For new token n of row b (n in [cu_seqlens[b], cu_seqlens[b+1]), position
 * starts[b] + n - cu_seqlens[b]): q = q_proj[n, h, 0:head_dim] (element strides
 * q_stride_t, q_stride_h; the gate half of each q_proj head is left in place for
 * qa_paged_attention_prefill), k = k_proj[n, g, :], v = v_proj[n, g, :], bf16.
 * q and k get the reference's RMSNorm with the (1 + w) weight (q_norm_weight,
 * k_norm_weight: head_dim, bf16 or fp32; eps) and the rotary embedding of their
 * first rotary_dim elements at the token's position, rounding to bf16 where the
 * reference's bf16 tensors do.  The bf16 cos/sin come from cos_sin_table
 * (table_positions, 2, rotary_dim/2) for positions it covers and are computed
 * from inv_freq (rotary_dim/2 fp32, device) otherwise.  q
 * goes to q_out (tokens, heads, head_dim) bf16 contiguous; k and v (copied
 * bit-exactly) go to slot (block_tables[b][pos/bs], pos%bs) of the shared pool
 * (table entries outside the pool are skipped).  head_dim 64, 128 or 256.
 * Replaces src/reference_ops.py:343-352 (rms_norm :166-169, rotary_embeddings
 * :203-213, apply_rotary_pos_emb :216-224), src/tp_runtime.py:511-525 and the
 * append of src/decode_state.py:271-293 for one layer's new tokens.          */
int qa_qk_norm_rope_append(const void* q_proj, int64_t q_stride_t, int64_t q_stride_h, const void* k_proj,
                           int64_t k_stride_t, int64_t k_stride_h, const void* v_proj, int64_t v_stride_t,
                           int64_t v_stride_h, int32_t act_dtype, const void* q_norm_weight, const void* k_norm_weight,
                           int32_t weight_dtype, float eps, const float* inv_freq, const void* cos_sin_table,
                           int64_t table_positions, int32_t rotary_dim,
                           const void* cu_seqlens, const void* starts, int32_t idx_dtype, int64_t batch, int64_t max_new,
                           int32_t heads, int32_t head_dim, const qa_paged_kv* kv, const void* block_tables,
                           int32_t table_dtype, int64_t table_stride, int64_t max_blocks, int32_t block_size, void* q_out,
                           hipStream_t stream);

/* ---- gated delta-rule linear attention --------------------------------- */
/* Depthwise causal conv1d over `seq` tokens (+ optional SiLU), fp32 math.
 * x: (batch, seq, channels) with element strides (x_stride_b, x_stride_t),
 * channels contiguous, float32 or bfloat16.  initial_state/final_state:
 * (state_rows, channels, kernel-1) fp32 (row = slots[b] when slots != NULL,
 * else b); a NULL initial_state means zeros.  A row whose state row lies
 * outside [0, state_rows) (e.g. a -1 pad) touches no state and outputs zeros.
 * weight: (channels, kernel) fp32.
 * out: (batch, seq, channels) float32 or bfloat16.  Replaces the conv of
 * linear_attention (src/reference_ops.py:240-258, src/tp_runtime.py:2635-2659). */
int qa_causal_conv1d_prefill(const void* x, int32_t x_dtype, int64_t x_stride_b, int64_t x_stride_t,
                             const float* initial_state, float* final_state, int64_t state_stride_b,
                             const void* slots, int32_t slots_dtype, int64_t state_rows,
                             const float* weight, int64_t batch, int64_t seq, int32_t channels, int32_t kernel,
                             void* out, int32_t out_dtype, int64_t out_stride_b, int64_t out_stride_t,
                             int32_t apply_silu, hipStream_t stream);

/* Single-token conv update with the (state_rows, channels, kernel-1) conv
 * state updated in place (the cache's conv_tail, src/reference_ops.py:253-257);
 * rows whose slot is outside [0, state_rows) output zeros.                  */
int qa_causal_conv1d_update(const void* x, int32_t x_dtype, int64_t x_stride_b,
                            float* conv_state, int64_t state_stride_b, const void* slots, int32_t slots_dtype,
                            int64_t state_rows, const float* weight, int64_t batch, int32_t channels, int32_t kernel,
                            void* out, int32_t out_dtype, int64_t out_stride_b, int32_t apply_silu,
                            hipStream_t stream);

/* Token-serial gated delta rule on prepared inputs: query/key (B, H, S, dk),
 * value (B, H, S, dv), g/beta (B, H, S), initial_state (B, H, dk, dv), all
 * contiguous fp32; output (B, H, S, dv) and final_state (B, H, dk, dv) fp32
 * (final_state may alias initial_state).  Replaces
 * `linear_attention_recurrent_core` (src/fp8_cuda.py:206-214 ->
 * src/csrc/fp8_linear.h:99-105, src/csrc/fp8_linear_cuda.cu:2491-2573).   */
int qa_linear_attention_recurrent_core(const float* query, const float* key, const float* value,
                                       const float* g, const float* beta, const float* initial_state,
                                       float* output, float* final_state,
                                       int64_t batch, int32_t heads, int64_t seq_len,
                                       int32_t key_dim, int32_t value_dim, hipStream_t stream);

/* Fused single-token decode step of a linear-attention layer after its conv:
 * qkv (B, 2*Hqk*dk + Hv*dv) fp32 = SiLU(conv) output; a, b (B, Hv) raw
 * projection outputs; a_log, dt_bias (Hv) fp32.  Computes
 * beta = sigmoid(b), g = -exp(a_log) softplus(a + dt_bias), L2-normalised
 * q*dk^-0.5 and k (value head j reads key head j / (Hv/Hqk)), one recurrence
 * step on state[slot(b)] (state_rows, Hv, dk, dv) fp32 in place, and writes
 * out (B, Hv, dv).  A row whose slot lies outside [0, state_rows) (a -1 pad, a
 * stale id) reads and writes no state and gets zero outputs.
 * dk = dv = 128.  Replaces the per-request state stacking
 * and recurrence of src/tp_runtime.py:2613-2717 with a slot-indexed pool
 * (src/reference_ops.py:271-283, :291-322).                               */
int qa_gated_delta_step(const float* qkv, int64_t qkv_stride_b,
                        const void* a, const void* b, int32_t ab_dtype, int64_t ab_stride_b,
                        const float* a_log, const float* dt_bias,
                        float* state, int64_t state_stride_slot, const void* slots, int32_t slots_dtype,
                        int64_t state_rows, void* out, int32_t out_dtype, int64_t out_stride_b,
                        int64_t batch, int32_t key_heads, int32_t value_heads,
                        int32_t key_dim, int32_t value_dim, hipStream_t stream);

/* qa_gated_delta_step followed, in the same kernel, by the layer's output
 * stage: out[b, h, :] = (w * o / sqrt(mean(o^2) + eps)) * silu(z[b, h, :])
 * on the step's fp32 output o of value head h, with z (B, Hv*dv) rows of
 * z_stride_b elements (the in_proj_z output) and norm_weight (dv), both
 * float32 or bfloat16.  The head's 128 outputs never leave the workgroup.
 * Replaces gated_rms_norm (src/reference_ops.py:172-178) applied to the
 * decode token's core (src/reference_ops.py:284-287, src/tp_runtime.py:
 * 853-857), where the core is fp32 and its cast of the normalised value is
 * the identity.                                                           */
int qa_gated_delta_step_norm(const float* qkv, int64_t qkv_stride_b,
                             const void* a, const void* b, int32_t ab_dtype, int64_t ab_stride_b,
                             const float* a_log, const float* dt_bias,
                             float* state, int64_t state_stride_slot, const void* slots, int32_t slots_dtype,
                             int64_t state_rows, const void* z, int32_t z_dtype, int64_t z_stride_b,
                             const void* norm_weight, int32_t norm_dtype, float eps,
                             void* out, int32_t out_dtype, int64_t out_stride_b,
                             int64_t batch, int32_t key_heads, int32_t value_heads,
                             int32_t key_dim, int32_t value_dim, hipStream_t stream);

/* qa_causal_conv1d_update and qa_gated_delta_step(_norm) in one kernel:
 * x (B, 2*Hqk*dk + Hv*dv) is the token's raw in_proj_qkv row (float32 or
 * bfloat16, rows of x_stride_b elements); conv_state (state_rows, C, K-1)
 * fp32 (rows of conv_state_stride_b elements) and state are both updated in
 * place at slot(b); conv_weight (C, K) fp32, 2 <= K <= 8.  z == NULL runs
 * no output stage (then norm_weight is ignored).  A workgroup per (row, key
 * head) owns the key head's q/k channels and its value heads' v channels,
 * so every conv state entry has one writer; Hv / Hqk must be 1, 2 or 4.
 * The activations are those of qa_causal_conv1d_update, so the outputs and
 * states equal the two calls'.  Replaces, per decode token, the conv1d with
 * cache of src/reference_ops.py:252-258 followed by the steps of
 * :271-322 (src/tp_runtime.py:2613-2717), in one launch.                  */
int qa_gated_delta_step_conv(const void* x, int32_t x_dtype, int64_t x_stride_b,
                             float* conv_state, int64_t conv_state_stride_b,
                             const float* conv_weight, int32_t conv_kernel,
                             const void* a, const void* b, int32_t ab_dtype, int64_t ab_stride_b,
                             const float* a_log, const float* dt_bias,
                             float* state, int64_t state_stride_slot, const void* slots, int32_t slots_dtype,
                             int64_t state_rows, const void* z, int32_t z_dtype, int64_t z_stride_b,
                             const void* norm_weight, int32_t norm_dtype, float eps,
                             void* out, int32_t out_dtype, int64_t out_stride_b,
                             int64_t batch, int32_t key_heads, int32_t value_heads,
                             int32_t key_dim, int32_t value_dim, hipStream_t stream);

/* Chunked gated delta-rule prefill of one linear-attention layer, from the
 * raw in_proj outputs.  mixed_qkv (B, T, 2*Hqk*dk + Hv*dv) bfloat16,
 * a, b (B, T, Hv), a_log/dt_bias (Hv) fp32, conv_weight (C, 4) fp32,
 * conv_state_in/out (B, C, 3) fp32 (NULL in = zeros, NULL out = not kept),
 * initial_state/final_state (B, Hv, dk, dv) fp32 (NULL in = zeros).  Writes
 * out (B, T, Hv, dv) float32/bfloat16.  Computes the conv1d + SiLU, L2 norm,
 * q scale and gating of src/reference_ops.py:240-283 and the recurrence of
 * :291-322 in 64-token chunks (WY/UT form) on fp16 MFMA with fp32
 * accumulation and an fp32 state.  dk = dv = 128, conv kernel 4.  The
 * workspace (256-byte aligned, qa_chunk_gated_delta_workspace bytes) holds the
 * normalised fp16 q/k and the gates between the launches (the v channels are
 * convolved inside the second launch).  The reference
 * has no chunked kernel: its prefill runs the token-serial recurrence
 * (src/tp_runtime.py:2744-2787).                                          */
int qa_chunk_gated_delta_rule(const void* mixed_qkv, int32_t x_dtype, int64_t x_stride_b, int64_t x_stride_t,
                              const void* a, const void* b, int32_t ab_dtype, int64_t ab_stride_b, int64_t ab_stride_t,
                              const float* a_log, const float* dt_bias, const float* conv_weight,
                              const float* conv_state_in, float* conv_state_out,
                              const float* initial_state, float* final_state,
                              void* out, int32_t out_dtype, int64_t out_stride_b, int64_t out_stride_t,
                              int64_t batch, int64_t seq, int32_t key_heads, int32_t value_heads,
                              int32_t key_dim, int32_t value_dim, int32_t conv_kernel,
                              void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* Workspace bytes qa_chunk_gated_delta_rule needs for these sizes (dk = dv = 128);
 * no counterpart in the reference, whose prefill keeps no intermediate buffers. */
int64_t qa_chunk_gated_delta_workspace(int64_t batch, int64_t seq, int32_t key_heads, int32_t value_heads);

/* LDS bytes one chunked-prefill workgroup reserves (for capacity planning). */
int64_t qa_chunk_gated_delta_lds_bytes(void);

/* ---- linear-attention output stage: gated RMSNorm + SiLU(z) ---------------- */
/* For token t and value head h, over the head's head_dim elements
 * x = x[t*x_stride_t + h*x_stride_h + d] and z = gate[t*gate_stride_t +
 * h*gate_stride_h + d]:  n = (x / sqrt(mean(x^2) + eps)) cast to x's dtype,
 * out[t*out_stride_t + h*out_stride_h + d] = (weight[d] * n) * silu(z) in fp32,
 * stored as out_dtype.  x, gate, weight, out: float32 or bfloat16 (weight
 * head_dim elements); head_dim 64, 128 or 256; rows start on 16-byte
 * boundaries.  Replaces gated_rms_norm (src/reference_ops.py:172-178) as the
 * linear-attention layers apply it to the recurrence output
 * (src/reference_ops.py:284-287, src/tp_runtime.py:853-857), where the core
 * arrives in fp32 and the result stays fp32 until the output projection.    */
int qa_gated_rms_norm(const void* x, int32_t x_dtype, int64_t x_stride_t, int64_t x_stride_h,
                      const void* gate, int32_t gate_dtype, int64_t gate_stride_t, int64_t gate_stride_h,
                      const void* weight, int32_t weight_dtype, float eps,
                      int64_t tokens, int32_t heads, int32_t head_dim,
                      void* out, int32_t out_dtype, int64_t out_stride_t, int64_t out_stride_h,
                      hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN36_HIP_H */
