/*
 * cie_attn.h - C ABI of the MI355X (gfx950) attention library `libcie_attn.so`.
 *
 * Two entry points carry the attention hot path of the engine:
 *
 *   cie_flash_fwd   dense (prefill) attention. Replaces the Triton launch behind
 *                   engine/attention.py:6-32 -> kernels/flash_attention.py:136-209
 *                   (kernel kernels/flash_attention.py:21-120).
 *   cie_paged_fwd   decode / speculative-verify attention that reads K and V
 *                   straight out of the paged pool through the block table.
 *                   Replaces the gather-then-dense sequence of
 *                   engine/model/block.py:56-71 (cache.gather at
 *                   engine/cache/kv_cache.py:141-165 followed by flash_attention).
 *
 * Around them: cie_kv_append (the pool write of new tokens), cie_rope_apply
 * (rotary embedding), the _rope variants that fuse the rotation into the
 * append and the query loads, and cie_int8_matmul (the INT8-weight
 * projections around attention).
 *
 * Conventions shared by every entry point:
 *   - Every pointer is a device pointer (e.g. torch.Tensor.data_ptr()).
 *   - Strides are in elements, four per tensor, outermost first. The innermost
 *     (head_dim) stride must be 1; every other stride is free, so transposed
 *     views such as the (1, Hk, N, D) view of a gathered (N, Hk, D) history
 *     need no copy.
 *   - `stream` is a hipStream_t (0 = null stream). Work is enqueued
 *     asynchronously; nothing synchronises, allocates or frees.
 *   - Return value 0 means success; a negative CIE_E* code means nothing was
 *     enqueued and cie_last_error() holds a message (thread-local).
 *   - dtype: CIE_DTYPE_F16 or CIE_DTYPE_BF16 for q, k, v and the output alike.
 *   - Semantics follow kernels/ref/flash_attention_ref.py:8-56: query head h
 *     reads kv head h / (Hq / Hk); with causal != 0 query row i sees key j iff
 *     j <= Lk - Lq + i (bottom-right aligned); scores and the softmax run in
 *     fp32, the probabilities are rounded to the input dtype before P.V, and
 *     the result is written in the input dtype. A row with keys but none
 *     visible is NaN; Lk == 0 gives zeros.
 */
#ifndef CIE_ATTN_H
#define CIE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CIE_ABI_VERSION 3

enum cie_dtype { CIE_DTYPE_F16 = 0, CIE_DTYPE_BF16 = 1 };

/* Element type of the rotary cos / sin tables. */
enum cie_table_dtype { CIE_TABLE_F16 = 0, CIE_TABLE_BF16 = 1, CIE_TABLE_F32 = 2 };

enum cie_status {
  CIE_OK = 0,
  CIE_EINVAL = -1,       /* bad pointer, negative size, bad stride, H % Hk != 0 */
  CIE_EHEADDIM = -2,     /* head_dim not a power of two in [16, 256]            */
  CIE_EDTYPE = -3,       /* dtype other than f16 / bf16                         */
  CIE_EWORKSPACE = -4,   /* paged workspace missing or too small                */
  CIE_ELAUNCH = -5       /* the HIP runtime refused the launch                  */
};

/* ABI version compiled into the library (CIE_ABI_VERSION). */
int cie_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* cie_last_error(void);

/*
 * Compute units of the current device, as the library sizes its launches
 * for it (queried once per device; 256, an unpartitioned MI355X, when no
 * device can be queried). No reference counterpart.
 */
int cie_device_cus(void);

/* Prefill kernels cie_flash_fwd chooses between (cie_prefill_kernel). */
enum cie_prefill_kernel_kind {
  CIE_PREFILL_32ROW = 0,       /* 32 query rows per wave, any head_dim but 128       */
  CIE_PREFILL_HEAD_PAIRS = 1,  /* head_dim 64: the same 32 rows of two query heads   */
  CIE_PREFILL_64ROW = 2,       /* head_dim 64: 64 rows of one query head per wave    */
  CIE_PREFILL_INTERLEAVED = 3  /* head_dim 128: MFMA and softmax issued interleaved  */
};

/*
 * The prefill kernel cie_flash_fwd runs for this launch shape (a
 * CIE_PREFILL_* value), or a negative CIE_E* code for arguments
 * cie_flash_fwd would reject. cu_count: compute units to size for, or <= 0
 * for the current device's (cie_device_cus). No reference counterpart: a
 * query for tests and profiles that must name the kernel they exercise.
 */
int cie_prefill_kernel(int B, int Hq, int Hk, int Lq, int Lk, int D, int causal, int dtype, int cu_count);

/*
 * Dense attention: o = softmax(q k^T * scale [+ causal mask]) v.
 *   q: (B, Hq, Lq, D)   k, v: (B, Hk, Lk, D)   o: (B, Hq, Lq, D)
 * Reference: engine/attention.py:6-32 (argument checks :17-25, call :27-32)
 * and kernels/flash_attention.py:136-209 (GQA mapping :150-155, default scale
 * :157-158 -- the caller passes the resolved scale here).
 */
int cie_flash_fwd(const void* q, const void* k, const void* v, void* o,
                  const int64_t* q_stride, const int64_t* k_stride,
                  const int64_t* v_stride, const int64_t* o_stride,
                  int B, int Hq, int Hk, int Lq, int Lk, int D,
                  float scale, int causal, int dtype, void* stream);

/*
 * Bytes of device workspace cie_paged_fwd needs for this shape on the
 * current device (0 for an unsupported shape): per-sequence piece
 * descriptors and the partial states of sequences split across workgroups
 * (the split follows the device's compute units). Any contents; calls that
 * run concurrently must not share a workspace.
 * max_context bounds every context_lens[b]; pass <= 0 to use the table bound
 * max_blocks_per_seq * block_size (the value cie_paged_fwd uses the same way).
 * No reference counterpart: the reference never splits a context.
 */
size_t cie_paged_workspace_bytes(int B, int Hq, int Hk, int Lq, int D,
                                 int max_context, int block_size,
                                 int max_blocks_per_seq);

/*
 * Paged attention over the engine's KV pool.
 *   q: (B, Hq, Lq, D) -- the Lq newest tokens of each sequence
 *   k_cache, v_cache: (num_blocks, block_size, Hk, D), the per-layer pool
 *        layout of engine/cache/kv_cache.py:55-63
 *   block_tables: int32 [B, max_blocks_per_seq], row b = BlockTable.blocks of
 *        sequence b (engine/cache/block_table.py:16-18); token t of sequence b
 *        lives at pool[block_tables[b][t / block_size], t % block_size]
 *        (engine/cache/block_table.py:23-26)
 *   context_lens: int32 [B], tokens already in the pool for each sequence,
 *        the Lq new ones included (the reference appends before it attends,
 *        engine/model/block.py:57-65)
 *   o: (B, Hq, Lq, D)
 * Equals flash_attention_ref(q[b], gather(b), causal, scale) per sequence.
 * A block id outside [0, num_blocks) or a context length outside
 * [0, min(max_context, max_blocks_per_seq * block_size)] is never
 * dereferenced: the affected sequence's output is written as NaN instead.
 * (Hq / Hk) * Lq must be at most 256 (128 at D = 256). workspace: at least
 * cie_paged_workspace_bytes bytes, 16-byte aligned. Two kernels are launched
 * on the stream: the main pass and the merge of split sequences.
 */
int cie_paged_fwd(const void* q, const void* k_cache, const void* v_cache,
                  const int32_t* block_tables, const int32_t* context_lens,
                  void* o, void* workspace, size_t workspace_bytes,
                  const int64_t* q_stride, const int64_t* kc_stride,
                  const int64_t* vc_stride, const int64_t* o_stride,
                  int B, int Hq, int Hk, int Lq, int D,
                  int num_blocks, int block_size, int max_blocks_per_seq,
                  int max_context, float scale, int causal, int dtype,
                  void* stream);

/*
 * Host-built work plan for paged attention (no reference counterpart: the
 * reference never splits a context). Built once per engine step on the host
 * from the host copies of the context lengths and block tables the step
 * uploads anyway (BlockTable.blocks / .length, engine/cache/block_table.py:
 * 16-18), copied to the device by the caller, and shared by every layer's
 * launch of that step: the launch then reads each workgroup's share of the
 * work directly instead of deriving it on the device from the lengths (three
 * dependent memory round trips before the first KV tile).
 *
 * cie_paged_plan_bytes: host (and device) bytes of the plan for this launch
 * shape, 0 for an unsupported shape. Arguments as cie_paged_workspace_bytes.
 *
 * cie_paged_plan: fills `plan` (host memory, at least cie_paged_plan_bytes)
 * from host arrays context_lens [B] and block_tables [B rows of
 * block_table_row_stride ints]. for_append: 1 when the plan is for a launch
 * with k_new / v_new (cie_paged_fwd_ex), whose contexts must count their Lq
 * new tokens. Returns the number of sequences split across workgroups
 * (>= 0; pass it to cie_paged_fwd_ex as plan_split: with 0 the merge pass
 * is not launched and no workspace is needed), or a negative CIE_E* code.
 * Context lengths and block ids are validated here as cie_paged_fwd
 * validates them (NaN output, never an out-of-range read).
 */
size_t cie_paged_plan_bytes(int B, int Hq, int Hk, int Lq, int D, int max_context, int block_size,
                            int max_blocks_per_seq);
int cie_paged_plan(void* plan, size_t plan_bytes, const int32_t* context_lens, const int32_t* block_tables,
                   int64_t block_table_row_stride, int B, int Hq, int Hk, int Lq, int D, int num_blocks,
                   int block_size, int max_blocks_per_seq, int max_context, int for_append);

/*
 * One entry for every paged attention variant: cie_paged_fwd with, each
 * optional, the fused append (k_new, v_new non-NULL: cie_paged_fwd_append),
 * RoPE (rope_cos, rope_sin non-NULL: the _rope entries) and a device copy of
 * a plan from cie_paged_plan (plan non-NULL; plan_bytes = the size of that
 * device buffer; plan_split = cie_paged_plan's return value; block_tables
 * and context_lens are then not read and may be NULL: the plan holds the
 * lengths and validated block ids it was built from, and a plan built from
 * older lengths or tables attends over those). The results equal the
 * corresponding entry's bit for bit. The workspace must hold
 * cie_paged_workspace_bytes bytes; with a plan whose plan_split is 0 it may
 * be NULL. A plan_bytes below cie_paged_plan_bytes for this call's
 * arguments is rejected with CIE_EINVAL (the launch reads each workgroup's
 * share of the plan in the same round trip as the plan's header, so every
 * offset it computes must lie inside the buffer). The plan's header records
 * B, Hq, Lq, head_dim, the head grouping, num_blocks, block_size,
 * max_blocks_per_seq, the context bound, the fused append flag, the
 * device's workgroup count and its split count; a plan whose header differs
 * from this call's arguments (or from plan_split) is used no further and
 * every output row is NaN.
 */
int cie_paged_fwd_ex(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                     const int32_t* block_tables, const int32_t* context_lens, const void* plan,
                     size_t plan_bytes, int plan_split,
                     void* o, void* workspace, size_t workspace_bytes,
                     const int64_t* q_stride, const int64_t* kn_stride, const int64_t* vn_stride,
                     const int64_t* kc_stride, const int64_t* vc_stride, const int64_t* o_stride,
                     int B, int Hq, int Hk, int Lq, int D,
                     int num_blocks, int block_size, int max_blocks_per_seq,
                     int max_context, float scale, int causal, int dtype,
                     const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                     void* stream);

/*
 * cie_paged_fwd without a caller workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture that must not call the
 * allocator, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. Same arguments, semantics and results as
 * cie_paged_fwd, bit for bit; the workspace is a static 16 MiB device array
 * of the library (one per GPU, held until the process ends), so this entry
 * allocates and frees nothing. A shape whose cie_paged_workspace_bytes
 * exceeds 16 MiB is rejected with CIE_EWORKSPACE before any HIP call.
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (concurrent streams, threads) race and must be serialised by the caller.
 */
int cie_paged_fwd_noalloc(const void* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_tables, const int32_t* context_lens, void* o,
                          const int64_t* q_stride, const int64_t* kc_stride,
                          const int64_t* vc_stride, const int64_t* o_stride,
                          int B, int Hq, int Hk, int Lq, int D,
                          int num_blocks, int block_size, int max_blocks_per_seq,
                          int max_context, float scale, int causal, int dtype,
                          void* stream);

/*
 * Paged KV append: writes the new tokens of B sequences into the pool.
 *   k_new, v_new: (T, Hk, D) rows; the rows of sequence b are
 *        cu_new[b] .. cu_new[b+1]-1 (int32 [B+1], cu_new[0] = 0, cu_new[B] = T)
 *   new_stride / v_new_stride: element strides of (T, Hk, D) (last must be 1)
 *   k_cache, v_cache: (num_blocks, block_size, Hk, D) pools as in cie_paged_fwd
 *   block_tables: int32 [B, max_blocks_per_seq] (already holding the blocks the
 *        new tokens need); start: int32 [B], position of each sequence's first
 *        new token; token i of sequence b goes to position start[b] + i
 *   max_new: an upper bound of cu_new[b+1] - cu_new[b] (sizes the launch)
 *   status: optional uint32 on the device; 1 is ORed into it when a position
 *        falls outside the table or a block id outside [0, num_blocks) (such
 *        tokens are not written); may be NULL
 * Reference: the per-block slice loop of PagedKVCache.append,
 * engine/cache/kv_cache.py:128-136 (block allocation, :122-125, stays on the
 * host), with the block ids read on the device instead of copied per call
 * (kv_cache.py:154).
 */
int cie_kv_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                  const int64_t* new_stride, const int64_t* v_new_stride,
                  const int64_t* kc_stride, const int64_t* vc_stride,
                  const int32_t* block_tables, const int32_t* cu_new, const int32_t* start,
                  uint32_t* status, int B, int T, int max_new, int Hk, int D,
                  int num_blocks, int block_size, int max_blocks_per_seq, int dtype, void* stream);

/*
 * Rotary position embedding (RoPE).
 *
 * rope_cos, rope_sin: device tables of shape (rope_rows, D/2), row-major and
 * 16-byte aligned, of element type rope_dtype (CIE_TABLE_*):
 * RotaryEmbedding's cos / sin buffers (engine/model/rope.py:12-16, built in
 * fp32 by kernels/ref/rope_apply_ref.py:6-19; the reference engine casts
 * them to the activation dtype, engine/runtime.py:22-37).
 * Every entry point below rotates exactly as apply_rotary_ref
 * (kernels/ref/rope_apply_ref.py:46-53): x1 = x[:D/2], x2 = x[D/2:],
 * rot1 = x1*c - x2*s, rot2 = x1*s + x2*c, with torch's arithmetic for the
 * two operand types: tables of the element type -> each product, difference
 * and sum rounded to the element type; fp32 tables (or 16-bit tables of the
 * other 16-bit type) -> each rounded to fp32 and the result rounded to the
 * element type. No fused multiply-add, so the output is bit-identical to the
 * reference's.
 */

/*
 * out = RoPE(x): x, out (B, H, L, D) (out may be x). positions: int32 on the
 * device, position of row l of batch b = positions[b * pos_batch_stride + l]
 * (pos_batch_stride 0: one (L,) vector for every batch, as
 * apply_rotary_ref's 1-d positions; L: a (B, L) matrix), or NULL for 0..L-1
 * (the reference's default). A position outside [0, rope_rows) makes its row
 * NaN and ORs 2 into *status (optional device uint32), where the
 * reference's table indexing raises.
 * Reference: RotaryEmbedding.apply (engine/model/rope.py:18-19) ->
 * apply_rotary_ref (kernels/ref/rope_apply_ref.py:22-53).
 */
int cie_rope_apply(const void* x, void* out, const int64_t* x_stride, const int64_t* out_stride,
                   const int32_t* positions, int64_t pos_batch_stride,
                   const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                   uint32_t* status, int B, int H, int L, int D, int dtype, void* stream);

/*
 * cie_flash_fwd with RoPE fused into the query load: q holds the projected,
 * un-rotated queries; row i of batch b is rotated at position q_pos0[b] + i
 * (q_pos0: int32 [B] on the device, or NULL for position i) before the
 * scores are formed. k must already be rotated (cie_kv_append_rope writes a
 * dense rotated copy for this). The result is bit-identical to
 * cie_rope_apply on q followed by cie_flash_fwd. A row whose position is
 * outside [0, rope_rows) is NaN.
 * Reference: engine/model/block.py:53-54 (q = rope.apply(q, positions))
 * followed by the attention call of block.py:69-71.
 */
int cie_flash_fwd_rope(const void* q, const void* k, const void* v, void* o,
                       const int64_t* q_stride, const int64_t* k_stride,
                       const int64_t* v_stride, const int64_t* o_stride,
                       int B, int Hq, int Hk, int Lq, int Lk, int D,
                       float scale, int causal, int dtype,
                       const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                       const int32_t* q_pos0, void* stream);

/*
 * cie_paged_fwd with RoPE fused into the query load: query row i of sequence
 * b is rotated at position context_lens[b] - Lq + i, the position of that
 * token in the sequence (the same alignment the causal mask uses; the
 * engine's positions, arange(start, start + Lq) with start + Lq the context
 * length, engine/model/transformer.py:35-37). Bit-identical to cie_rope_apply
 * on q followed by cie_paged_fwd. A row whose position is outside
 * [0, rope_rows) is NaN.
 * Reference: engine/model/block.py:53 followed by block.py:65-71.
 */
int cie_paged_fwd_rope(const void* q, const void* k_cache, const void* v_cache,
                       const int32_t* block_tables, const int32_t* context_lens,
                       void* o, void* workspace, size_t workspace_bytes,
                       const int64_t* q_stride, const int64_t* kc_stride,
                       const int64_t* vc_stride, const int64_t* o_stride,
                       int B, int Hq, int Hk, int Lq, int D,
                       int num_blocks, int block_size, int max_blocks_per_seq,
                       int max_context, float scale, int causal, int dtype,
                       const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                       void* stream);

/*
 * cie_kv_append followed by cie_paged_fwd in one launch pair, for new tokens
 * that are the Lq newest positions of every context (context_lens[b]
 * already counts them, as after the reference's append). k_new, v_new:
 * (B * Lq, Hk, D), row b * Lq + i = new token i of sequence b, strides
 * {token, head} in elements (multiples of 8), unit head_dim stride,
 * 16-byte aligned. Attention reads those rows straight from k_new / v_new;
 * each is also written into the pool at position context_lens[b] - Lq + i
 * through the block table, so the pool afterwards equals what cie_kv_append
 * leaves, and o equals cie_kv_append then cie_paged_fwd bit for bit.
 * A context shorter than Lq is invalid here (NaN output, nothing written);
 * a token whose block id is out of range is not written (its sequence's
 * output is NaN, as in cie_paged_fwd). K must already be rotated (no RoPE
 * is applied to it; cie_paged_fwd_append_rope rotates it). Same workspace as
 * cie_paged_fwd.
 * Reference: engine/model/block.py:57-71 (append, then gather + attend).
 */
int cie_paged_fwd_append(const void* q, const void* k_new, const void* v_new,
                         void* k_cache, void* v_cache,
                         const int32_t* block_tables, const int32_t* context_lens,
                         void* o, void* workspace, size_t workspace_bytes,
                         const int64_t* q_stride, const int64_t* kn_stride, const int64_t* vn_stride,
                         const int64_t* kc_stride, const int64_t* vc_stride, const int64_t* o_stride,
                         int B, int Hq, int Hk, int Lq, int D,
                         int num_blocks, int block_size, int max_blocks_per_seq,
                         int max_context, float scale, int causal, int dtype,
                         void* stream);

/*
 * cie_paged_fwd_append with RoPE: k_new and q are un-rotated; new token i of
 * sequence b is rotated at position context_lens[b] - Lq + i, K as it is
 * used and as it is written into the pool, q as it is loaded. Pool and
 * output are bit-identical to cie_kv_append_rope (start = context_lens[b] -
 * Lq) followed by cie_paged_fwd_rope. A position outside [0, rope_rows)
 * gives NaN output rows, and neither K nor V of that token is written (as
 * cie_kv_append_rope leaves the pool; there is no status word here).
 * Reference: engine/model/block.py:53-54 (RoPE) and :57-71.
 */
int cie_paged_fwd_append_rope(const void* q, const void* k_new, const void* v_new,
                              void* k_cache, void* v_cache,
                              const int32_t* block_tables, const int32_t* context_lens,
                              void* o, void* workspace, size_t workspace_bytes,
                              const int64_t* q_stride, const int64_t* kn_stride, const int64_t* vn_stride,
                              const int64_t* kc_stride, const int64_t* vc_stride, const int64_t* o_stride,
                              int B, int Hq, int Hk, int Lq, int D,
                              int num_blocks, int block_size, int max_blocks_per_seq,
                              int max_context, float scale, int causal, int dtype,
                              const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                              void* stream);

/*
 * cie_kv_append with RoPE fused into the write of K: k_new holds the
 * projected, un-rotated keys; token i of sequence b is rotated at position
 * start[b] + i, then written (V is copied as is). k_out (optional, may be
 * NULL; k_out_stride: strides of its (T, Hk, D) layout) receives the rotated
 * K rows as well, for attention over the new tokens themselves (prefill).
 * A position outside [0, rope_rows) writes neither K nor V of that token and
 * ORs 2 into *status; positions outside the block table OR in 1 as in
 * cie_kv_append.
 * Reference: engine/model/block.py:54 (k = rope.apply(k, positions))
 * followed by the append of block.py:57-64 -> kv_cache.py:128-136.
 */
int cie_kv_append_rope(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                       const int64_t* new_stride, const int64_t* v_new_stride,
                       const int64_t* kc_stride, const int64_t* vc_stride,
                       const int32_t* block_tables, const int32_t* cu_new, const int32_t* start,
                       uint32_t* status, int B, int T, int max_new, int Hk, int D,
                       int num_blocks, int block_size, int max_blocks_per_seq, int dtype,
                       const void* rope_cos, const void* rope_sin, int rope_rows, int rope_dtype,
                       void* k_out, const int64_t* k_out_stride, void* stream);

/*
 * INT8-weight linear layer: y = (x . w_int8^T) * scales[n] (+ bias[n]).
 *   x: (M, K) fp16 / bf16 (dtype), row stride x_row_stride elements
 *        (a multiple of 8: rows start 16-byte aligned)
 *   w_int8: (N, K) int8, row stride w_row_stride bytes (multiple of 16)
 *   scales: (N,) per output channel, fp16 / bf16 / fp32 (scale_dtype 0 / 1 / 2)
 *   bias: (N,) in x's dtype, or NULL
 *   y: (M, N) in x's dtype, row stride y_row_stride elements (8-byte aligned)
 * Any K >= 1: each kernel's vector loop covers the largest prefix of K its
 * step divides and the remaining k (fewer than 64) of every output are added
 * in the epilogue, as the reference masks the K tail of its last tile
 * (kernels/int8_matmul.py:43-50); nothing past column K of a row is read.
 * The products x * w are exact and summed in
 * fp32; the sum is multiplied by the scale once and rounded to x's dtype,
 * then the bias is added in x's dtype (rounded again), as the reference does.
 * workspace: cie_int8_matmul_workspace_bytes(M, N, K) bytes, 16-byte
 * aligned (0 bytes -- NULL allowed -- when the launch does not split K,
 * which is always the case for M <= 64);
 * any contents, not shared by concurrent calls. One kernel is launched on
 * the stream, or two when K is split (the second sums the split partials).
 * Reference: kernels/int8_matmul.py:65-110 (wrapper; bias :107-109) and
 * :16-62 (kernel), called by Int8Linear.forward
 * (engine/quant/int8_linear.py:37-41).
 */
size_t cie_int8_matmul_workspace_bytes(int M, int N, int K);
int cie_int8_matmul(const void* x, const int8_t* w_int8, const void* scales, const void* bias, void* y,
                    int64_t x_row_stride, int64_t w_row_stride, int64_t y_row_stride,
                    int M, int N, int K, int dtype, int scale_dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CIE_ATTN_H */
