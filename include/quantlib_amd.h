/*
 * quantlib_amd.h -- C ABI of the MI355X (gfx950) fused per-layer kernels.
 *
 * Every entry point:
 *   - takes plain device pointers, sizes and a hipStream_t (NULL = default stream);
 *   - validates its arguments on the host and returns hipErrorInvalidValue before
 *     touching the GPU when they are unusable;
 *   - returns hipSuccess without launching anything when the problem is empty
 *     (rows == 0, n == 0, n_tokens == 0);
 *   - otherwise enqueues its kernel(s) on `stream` and returns the launch status.
 *     The kernel entry points never synchronise, allocate or free.  Exceptions,
 *     each stated at its declaration: ql_gemm_f16 creates its per-device
 *     library context on first use and allocates a 64 MB workspace the first
 *     time it runs on a given stream (kept until the process ends); the
 *     setup-time calls (ql_gemm_tune_f16, ql_engine_tune, ql_engine_create*,
 *     ql_batcher_create, ql_graph_*) allocate, and the tuners synchronise.
 *
 * fp16 tensors are passed as `uint16_t*` holding IEEE-754 binary16 bit patterns
 * (the storage of `__half`).  Buffers must not alias unless an entry point says
 * it works in place.  Fast paths use 16-byte vector accesses when every pointer
 * (and row stride) is 16-byte aligned; other layouts take a scalar path that
 * computes the same arithmetic.
 *
 * The reference names each function replaces are given as file:line of
 * samfrazerdutton/Quant-lib.  The reference launchers use C++ linkage and
 * return void; the drop-in shims with those exact names live in
 * quantlib_compat.h and forward here.
 */
#ifndef QUANTLIB_AMD_H
#define QUANTLIB_AMD_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* RoPE pairing of the head vector x[0..d).
 * QL_ROPE_INTERLEAVED: pairs (2i, 2i+1) -- the reference's behaviour
 *   (kernels/rope.cu:27-29,40-41; kernels/fp16_ops.cu:54,59-62).
 * QL_ROPE_HALF: pairs (i, i + d/2) ("rotate-half", Llama/HF layout).
 * Both use inv_freq_i = 1 / theta^(2i/d) for pair i. */
#define QL_ROPE_INTERLEAVED 0
#define QL_ROPE_HALF        1

/* Tokens per paged-KV block (include/paged_kvcache.h:7, include/fp16_types.h:60). */
#define QL_PAGE_SIZE 16

/* Library version as 10000*major + 100*minor + patch. */
int ql_version(void);

/* ---- RMSNorm --------------------------------------------------------------
 * out[r,i] = (x[r,i] * inv_rms_r) * w[i],  inv_rms_r = 1/sqrt(sum_i x[r,i]^2 / dim + eps)
 * fp32 math; fp16 variant reads/writes binary16 and rounds the output RNE.
 * Replaces launch_rmsnorm (kernels/rmsnorm.cu:51-57) and
 * launch_fp16_rmsnorm (kernels/fp16_ops.cu:113-118). */
hipError_t ql_rmsnorm_f32(const float* x, const float* w, float* out,
                          int rows, int dim, float eps, hipStream_t stream);
hipError_t ql_rmsnorm_f16(const uint16_t* x, const uint16_t* w, uint16_t* out,
                          int rows, int dim, float eps, hipStream_t stream);

/* ---- fused residual add + RMSNorm -----------------------------------------
 * x[r,i] <- x[r,i] + d[r,i]   (in place; fp16: rounded RNE to binary16 first)
 * out    <- rmsnorm(x_updated)  (normalises the rounded sum, so the result is
 *                                identical to the unfused add then rmsnorm)
 * Replaces the add_residual + launch_rmsnorm pair of src/forward.cu:228-232
 * and the launch_fp16_add + launch_fp16_rmsnorm pair of
 * src/fp16_forward.cu:213-216 with one pass. */
hipError_t ql_add_rmsnorm_f32(float* x, const float* d, const float* w, float* out,
                              int rows, int dim, float eps, hipStream_t stream);
hipError_t ql_add_rmsnorm_f16(uint16_t* x, const uint16_t* d, const uint16_t* w,
                              uint16_t* out, int rows, int dim, float eps,
                              hipStream_t stream);

/* ---- residual add (in place) ----------------------------------------------
 * fp32: x += d  (add_residual_kernel, src/forward.cu:128-135)
 * fp16: x = h(f(x) + f(d)) (fp16_add_kernel / launch_fp16_add, kernels/fp16_ops.cu:92-100,144-147) */
hipError_t ql_add_f32(float* x, const float* d, int64_t n, hipStream_t stream);
hipError_t ql_add_f16(uint16_t* x, const uint16_t* d, int64_t n, hipStream_t stream);

/* ---- rotary position embedding (in place, Q and K in one launch) ----------
 * q: [n_tokens rows of q_row_stride elements], head h of token t at q + t*q_row_stride + h*head_dim
 * k: likewise with n_kv_heads heads and k_row_stride (GQA: n_kv_heads <= n_heads)
 * Either q or k may be NULL (its head count is then ignored).
 * position of token t = positions ? positions[t] : pos_offset + t
 * pair i of a head:  inv_freq = 1/theta^((2i)/d) (fp32 exponent, as kernels/rope.cu:35)
 *                    a = (float)pos * inv_freq,  c = cos(a), s = sin(a) (accurate)
 *                    y0 = fma(x0, c, -(x1*s)),  y1 = fma(x0, s, x1*c)
 * head_dim must be even and <= 2048.
 * Replaces launch_rope (kernels/rope.cu:44-50) and launch_fp16_rope
 * (kernels/fp16_ops.cu:120-127), which take one tensor per call and use
 * position = row index. */
hipError_t ql_rope_f32(float* q, float* k, int n_tokens, int n_heads, int n_kv_heads,
                       int head_dim, int64_t q_row_stride, int64_t k_row_stride,
                       const int32_t* positions, int pos_offset, float theta,
                       int pairing, hipStream_t stream);
hipError_t ql_rope_f16(uint16_t* q, uint16_t* k, int n_tokens, int n_heads,
                       int n_kv_heads, int head_dim, int64_t q_row_stride,
                       int64_t k_row_stride, const int32_t* positions, int pos_offset,
                       float theta, int pairing, hipStream_t stream);

/* ---- fused RoPE + KV-cache append ------------------------------------------
 * One launch that does what ql_rope_f16/f32(q, k, ...) followed by the cache
 * append of the rotated K rows and of the V rows does, with identical results:
 * Q and K are rotated in place, and token t's rotated K row and V row
 * (v + t*v_row_stride, n_kv_heads*head_dim elements) are written to the cache.
 * It saves the second launch and the re-read of K.  This is the "fused KV-cache
 * append" of the reference's layer order: launch_fp16_rope on q and k, then
 * fp16_kvcache_append (src/fp16_forward.cu:190-199).
 * Paged: cache arguments as ql_paged_kv_append_f16 (slot < 0 or a block
 * >= n_blocks skips that token's cache write; Q/K are still rotated).
 * Contiguous: cache [n_layers, max_seq, n_kv_heads, head_dim], token t at
 * position pos + t (pos + n_tokens <= max_seq). */
hipError_t ql_rope_paged_kv_append_f16(uint16_t* q, uint16_t* k, const uint16_t* v, int n_tokens,
                                       int n_heads, int n_kv_heads, int head_dim,
                                       int64_t q_row_stride, int64_t k_row_stride,
                                       int64_t v_row_stride, const int32_t* positions,
                                       int pos_offset, float theta, int pairing,
                                       uint16_t* const* k_blocks, uint16_t* const* v_blocks,
                                       int n_blocks, const int32_t* slot_mapping, int layer,
                                       int n_layers, hipStream_t stream);
/* As ql_rope_paged_kv_append_f16, except that k is only read: the rotated K rows
 * go to the paged cache and nowhere else, and the caller's k rows are left as
 * they were.  For callers that read K only from the cache afterwards, which is
 * the reference layer's case: attention takes K_full from the cache
 * (src/fp16_forward.cu:194-209), so its in-place rotated K is never read.  This
 * saves one write of the K rows. */
hipError_t ql_rope_q_paged_kv_append_f16(uint16_t* q, const uint16_t* k, const uint16_t* v,
                                         int n_tokens, int n_heads, int n_kv_heads, int head_dim,
                                         int64_t q_row_stride, int64_t k_row_stride,
                                         int64_t v_row_stride, const int32_t* positions,
                                         int pos_offset, float theta, int pairing,
                                         uint16_t* const* k_blocks, uint16_t* const* v_blocks,
                                         int n_blocks, const int32_t* slot_mapping, int layer,
                                         int n_layers, hipStream_t stream);
hipError_t ql_rope_kv_append_f16(uint16_t* q, uint16_t* k, const uint16_t* v, int n_tokens,
                                 int n_heads, int n_kv_heads, int head_dim, int64_t q_row_stride,
                                 int64_t k_row_stride, int64_t v_row_stride,
                                 const int32_t* positions, int pos_offset, float theta,
                                 int pairing, uint16_t* k_cache, uint16_t* v_cache, int layer,
                                 int pos, int max_seq, int n_layers, hipStream_t stream);
hipError_t ql_rope_kv_append_f32(float* q, float* k, const float* v, int n_tokens, int n_heads,
                                 int n_kv_heads, int head_dim, int64_t q_row_stride,
                                 int64_t k_row_stride, int64_t v_row_stride,
                                 const int32_t* positions, int pos_offset, float theta,
                                 int pairing, float* k_cache, float* v_cache, int layer, int pos,
                                 int max_seq, int n_layers, hipStream_t stream);

/* ---- SwiGLU -----------------------------------------------------------------
 * out = (g / (1 + exp(-g))) * u, elementwise over rows*ffn_dim elements.
 * Replaces launch_swiglu (kernels/feedforward.cu:27-35) and
 * launch_fp16_swiglu (kernels/fp16_ops.cu:129-135). */
hipError_t ql_swiglu_f32(const float* gate, const float* up, float* out,
                         int rows, int ffn_dim, hipStream_t stream);
hipError_t ql_swiglu_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out,
                         int rows, int ffn_dim, hipStream_t stream);

/* ---- row softmax ------------------------------------------------------------
 * m = max(-FLT_MAX, max_c x[r,c]);  e = exp(x - m);  out = e * (1 / sum_c e)
 * Reads each row once and writes it once.  -inf entries give exactly 0.
 * Replaces launch_softmax (kernels/softmax.cu:88-94).  The fp16 variant has no
 * reference kernel: it is the fp32 arithmetic with binary16 I/O (RNE output). */
hipError_t ql_softmax_f32(const float* in, float* out, int rows, int cols,
                          hipStream_t stream);
hipError_t ql_softmax_f16(const uint16_t* in, uint16_t* out, int rows, int cols,
                          hipStream_t stream);

/* ---- token-embedding gather (batched) ----------------------------------------
 * out[t, :] = table[ids[t], :] for t < n_tokens; bit-exact copy.
 * ids outside [0, vocab) produce a zero row (the reference does no check).
 * table and out must be aligned to their element size (hipErrorInvalidValue
 * otherwise); any other offset and any dim are accepted.
 * Replaces embed_kernel (src/forward.cu:137-141, launched :256-257) and
 * launch_fp16_embed (kernels/fp16_ops.cu:81-89,137-142), which gather one token. */
hipError_t ql_embed_f32(const float* table, const int32_t* ids, int n_tokens,
                        int vocab, int dim, float* out, hipStream_t stream);
hipError_t ql_embed_f16(const uint16_t* table, const int32_t* ids, int n_tokens,
                        int vocab, int dim, uint16_t* out, hipStream_t stream);

/* One token whose id is passed by value, as embed_kernel (src/forward.cu:137-141)
 * and launch_fp16_embed (kernels/fp16_ops.cu:137-142) take it; no vocab bound is
 * known, so only a negative id gives the zero row. */
hipError_t ql_embed_token_f32(const float* table, int token_id, int dim, float* out,
                              hipStream_t stream);
hipError_t ql_embed_token_f16(const uint16_t* table, int token_id, int dim, uint16_t* out,
                              hipStream_t stream);

/* ---- contiguous KV-cache append ---------------------------------------------
 * cache layout [n_layers, max_seq, n_kv_heads, head_dim]; writes n_tokens
 * consecutive positions pos .. pos+n_tokens-1 of `layer` from
 * k_new/v_new [n_tokens, n_kv_heads, head_dim].  Bit-exact copy.
 * Replaces kvcache_append (src/kv_cache.cu:44-58, two cudaMemcpyAsync) and
 * fp16_kvcache_append (src/fp16_forward.cu:148-164, one token). */
hipError_t ql_kv_append_f32(float* k_cache, float* v_cache, const float* k_new,
                            const float* v_new, int layer, int pos, int n_tokens,
                            int n_kv_heads, int head_dim, int max_seq, int n_layers,
                            hipStream_t stream);
hipError_t ql_kv_append_f16(uint16_t* k_cache, uint16_t* v_cache, const uint16_t* k_new,
                            const uint16_t* v_new, int layer, int pos, int n_tokens,
                            int n_kv_heads, int head_dim, int max_seq, int n_layers,
                            hipStream_t stream);

/* ---- paged KV-cache append ----------------------------------------------------
 * k_blocks/v_blocks: DEVICE arrays of n_blocks device pointers, one per block;
 * each block is [n_layers, QL_PAGE_SIZE, n_kv_heads, head_dim] binary16
 * (the pool of src/paged_kvcache.cu:26-46).
 * slot_mapping[t] = physical_block * QL_PAGE_SIZE + offset_in_block for token t;
 * a negative slot (padding) or a block >= n_blocks skips the token.
 * Element (t, h, j) goes to k_blocks[b][((layer*16 + o)*n_kv_heads + h)*head_dim + j].
 * The reference ships the pool and block tables but no append kernel. */
hipError_t ql_paged_kv_append_f16(uint16_t* const* k_blocks, uint16_t* const* v_blocks,
                                  int n_blocks, const int32_t* slot_mapping,
                                  const uint16_t* k_new, const uint16_t* v_new,
                                  int n_tokens, int layer, int n_layers, int n_kv_heads,
                                  int head_dim, hipStream_t stream);

/* Host helper: slot_mapping[i] = block_table[(start_pos+i)/16]*16 + (start_pos+i)%16
 * for i < n_tokens (the per-sequence logical->physical block map of
 * include/scheduler.h:17-19).  Host memory only.  Returns hipErrorInvalidValue if a
 * needed block_table entry is negative or beyond n_table. */
hipError_t ql_paged_slot_mapping(const int32_t* block_table, int n_table, int start_pos,
                                 int n_tokens, int32_t* slot_mapping);

/* ---- fp16 -> fp32 widening (launch_fp16_to_fp32, kernels/fp16_ops.cu:103-110,149-153) */
hipError_t ql_f16_to_f32(const uint16_t* src, float* dst, int64_t n, hipStream_t stream);

/* ---- fp32 -> fp16 narrowing, round to nearest even (__float2half): the
 * fp32_to_fp16_kernel of src/quant_forward.cu:18-21, launched by the fp32 engine's
 * quantized GEMM bridge (sgemm, src/forward.cu:52-70: narrow A, quantlib FP8 GEMM,
 * widen C).  Overflow gives +-inf, NaN stays NaN. */
hipError_t ql_f32_to_f16(const float* src, uint16_t* dst, int64_t n, hipStream_t stream);

/* ---- attention (fp16 I/O, fp32 softmax state, gfx950 matrix cores) ----------------
 * out[i, h, :] = sum_j softmax_j((q[i,h,:] . k[j,g,:]) * scale) v[j,g,:] with
 * g = h * n_kv_heads / n_heads (grouped-query heads, kernels/flash_attention.cu:45),
 * scale = 1/sqrtf(head_dim) (:173), normalised as O / (l + 1e-8) (:161).  Causal:
 * key j is visible to query i when j <= its position.  head_dim 64 and 128 run on
 * the matrix cores and need rows 16-byte aligned (strides multiples of 8 elements);
 * every other head_dim from 1 to 64 (the reference kernel's range) runs a vector-ALU
 * kernel at any row alignment, with fp32 probabilities, in one pass (the workspace
 * sizes below are 0 for it).  Other head_dims are rejected. */

/* Replaces launch_flash_attention (kernels/flash_attention.cu:169-182): Q, out
 * [seq_len, n_heads, head_dim]; K, V [seq_len, n_kv_heads, head_dim], query i at
 * position i.  (The reference's tiles hold head_dim <= 64 only; 128 is an extension.) */
hipError_t ql_flash_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                  uint16_t* out, int seq_len, int n_heads, int n_kv_heads,
                                  int head_dim, int causal, hipStream_t stream);

/* General contiguous form: the q_len queries are the LAST q_len positions of the
 * kv_len keys (query i sits at kv_len - q_len + i).  Decode against the contiguous
 * cache of src/fp16_forward.cu:202-209 is q_len = 1, kv_len = pos + 1,
 * k = k_cache + layer*max_seq*n_kv_heads*head_dim, kv_row_stride = n_kv_heads*head_dim
 * (the reference passes its one-token Q with seq_len = ctx_len and so reads past it).
 * q_len == 1 runs the decode kernel (the query heads of a KV head share one pass). */
hipError_t ql_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            uint16_t* out, int q_len, int kv_len, int n_heads, int n_kv_heads,
                            int head_dim, int64_t q_row_stride, int64_t kv_row_stride,
                            int64_t out_row_stride, int causal, hipStream_t stream);

/* Decode against the contiguous cache with the keys split over workgroups: the one
 * query row q / out ([n_heads, head_dim]) of the token at position kv_len - 1
 * against K/V rows 0 .. kv_len-1 (row stride kv_row_stride elements) -- the
 * decode call of src/fp16_forward.cu:202-209 (launch_flash_attention over the
 * layer's K_full/V_full with ctx_len keys) with its query count stated.  Same
 * kernel as ql_attention_f16 with q_len = 1; with the
 * ql_decode_attention_workspace_size() bytes the keys are split over more
 * workgroups (fp32 partials in the workspace, then a combine kernel), a smaller
 * or NULL workspace uses fewer splits (down to ql_attention_f16's single pass).
 * Results for a given workspace size are deterministic; calls that share a
 * workspace must be ordered on one stream. */
hipError_t ql_decode_attention_workspace_size(int n_heads, int n_kv_heads, int head_dim,
                                              int kv_len, size_t* bytes);
hipError_t ql_decode_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                   uint16_t* out, int kv_len, int n_heads, int n_kv_heads,
                                   int head_dim, int64_t kv_row_stride, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);

/* Attention over the paged KV cache (pool layout of src/paged_kvcache.cu:26-46, the
 * layout ql_paged_kv_append_f16 writes), for n_seqs sequences at once.  Device
 * arrays: cu_q_lens[n_seqs+1] (sequence s owns query rows cu_q_lens[s] ..
 * cu_q_lens[s+1]-1 of q/out, all < n_q_rows), ctx_lens[n_seqs] (its keys,
 * including the new ones), block_tables[n_seqs * max_blocks_per_seq] (logical ->
 * physical block, include/scheduler.h:17-19).  max_q_len bounds every sequence's
 * query count (host value: it sizes the grid).  A sequence whose rows fall outside
 * [0, n_q_rows) is skipped; a table entry outside [0, n_blocks) reads as zero
 * keys.  max_q_len == 1 (every sequence decodes one token) runs the decode kernel
 * (see ql_paged_decode_attention_f16) in one pass. */
hipError_t ql_paged_attention_f16(const uint16_t* q, uint16_t* out, int64_t q_row_stride,
                                  int64_t out_row_stride, int n_q_rows, int n_seqs,
                                  const int32_t* cu_q_lens, const int32_t* ctx_lens,
                                  int max_q_len, const int32_t* block_tables,
                                  int max_blocks_per_seq, const uint16_t* const* k_blocks,
                                  const uint16_t* const* v_blocks, int n_blocks, int layer,
                                  int n_layers, int n_heads, int n_kv_heads, int head_dim,
                                  int causal, hipStream_t stream);

/* Decode over the paged KV cache: sequence s (< n_seqs) has ONE query, row s of q,
 * at position ctx_lens[s] - 1, and its output goes to row s of out (the attention
 * step of the per-token decode in src/fp16_forward.cu:202-209 and
 * src/continuous_batch.cu:104-127, batched over sequences).  The query heads
 * that share a KV head read its K/V rows once.  With a workspace of
 * ql_paged_decode_workspace_size() bytes the keys of each sequence are split over
 * more workgroups (partials in the workspace, then a combine kernel); a smaller or
 * NULL workspace uses fewer splits (down to one pass, no workspace).  max_ctx_len
 * is a host-side bound of ctx_lens used to size the split.  Results for a given
 * workspace size are deterministic.  Calls that share a workspace must be ordered
 * on one stream. */
hipError_t ql_paged_decode_workspace_size(int n_seqs, int n_heads, int n_kv_heads, int head_dim,
                                          int max_ctx_len, size_t* bytes);
hipError_t ql_paged_decode_attention_f16(const uint16_t* q, uint16_t* out, int64_t q_row_stride,
                                         int64_t out_row_stride, int n_seqs,
                                         const int32_t* ctx_lens, int max_ctx_len,
                                         const int32_t* block_tables, int max_blocks_per_seq,
                                         const uint16_t* const* k_blocks,
                                         const uint16_t* const* v_blocks, int n_blocks,
                                         int layer, int n_layers, int n_heads, int n_kv_heads,
                                         int head_dim, void* workspace, size_t workspace_bytes,
                                         hipStream_t stream);

/* ql_paged_decode_attention_f16 for callers that cannot allocate (code under HIP
 * graph capture, serving loops that forbid hipMalloc): no workspace argument and no
 * allocation.  It runs the key split that ql_paged_decode_workspace_size sizes --
 * the same kernels and results as ql_paged_decode_attention_f16 given that many
 * workspace bytes -- with the partials in a library-owned device array of
 * QL_DECODE_SCRATCH_BYTES per GPU, held until the process ends.  A problem whose
 * split would need more (possible only with more than 8 query heads per KV head at
 * head_dim 128 and several hundred sequences) returns hipErrorInvalidValue before
 * touching the GPU.  Nothing in the array needs clearing: every split writes its
 * partials before the combine reads them.  Every call on one GPU shares that
 * GPU's array, so calls that overlap on one GPU (two streams, two host threads)
 * race; order them on one stream.  The first call on each device looks up the
 * array's device address (hipGetSymbolAddress); make it outside graph capture.
 * No counterpart in the reference. */
#define QL_DECODE_SCRATCH_BYTES (8u << 20)
hipError_t ql_paged_decode_attention_f16_noalloc(const uint16_t* q, uint16_t* out,
                                                 int64_t q_row_stride, int64_t out_row_stride,
                                                 int n_seqs, const int32_t* ctx_lens,
                                                 int max_ctx_len, const int32_t* block_tables,
                                                 int max_blocks_per_seq,
                                                 const uint16_t* const* k_blocks,
                                                 const uint16_t* const* v_blocks, int n_blocks,
                                                 int layer, int n_layers, int n_heads,
                                                 int n_kv_heads, int head_dim, hipStream_t stream);

/* ---- continuous batching over the paged pool (host only, no GPU calls) -------------
 * The bookkeeping of the reference scheduler (scheduler_create / scheduler_add_request
 * / scheduler_step, src/continuous_batch.cu:48-174, include/scheduler.h:6-54) over the
 * LIFO block allocator of src/paged_kvcache.cu:49-53,89-98, with the model step left
 * to the caller and every active sequence served by ONE batched step:
 *   ql_batcher_plan   admits pending requests (FIFO; the head waits until
 *                     ceil(prompt_len/16) blocks are free and fewer than max_active
 *                     run -- head-of-line blocking), gives a decoding sequence a new
 *                     block when its next position starts one (evicting it, finished
 *                     early, when none is free), and lists the step's work: per
 *                     sequence in active order its query rows (whole prompt for a
 *                     prefill, the newest token for a decode) with token ids,
 *                     positions and KV slots, plus cu_q_lens / ctx_lens /
 *                     block_tables for ql_paged_attention_f16 and slot_mapping for
 *                     ql_rope_paged_kv_append_f16 / ql_paged_kv_append_f16;
 *   ql_batcher_commit takes the sampled token of each planned sequence (the logits
 *                     of row sample_rows[i]), finishes sequences at prompt_len + max_gen
 *                     tokens or at eos_token, and returns their blocks (table order,
 *                     swap-with-last removal from the active list, as the reference).
 * Plans and commits alternate.  Plan arrays are host memory owned by the batcher,
 * valid until the next ql_batcher_plan.  Difference from the reference: the token
 * sampled after the prefill is kept as the first generated token (the reference's
 * stub forward discards it), so a request finishes one step earlier; growth and
 * eviction happen at the same positions. */
#define QL_FINISH_LENGTH  0   /* reached prompt_len + max_gen tokens */
#define QL_FINISH_EOS     1   /* sampled eos_token */
#define QL_FINISH_EVICTED 2   /* no free block for its next position */

typedef struct ql_batcher ql_batcher;

typedef struct {
    int n_seqs;                   /* sequences that run this step */
    int n_rows;                   /* query rows (tokens) in this step */
    int max_q_len;                /* largest rows of one sequence */
    int max_ctx_len;              /* largest ctx_lens[i] */
    int max_blocks;               /* row length of block_tables */
    const int32_t* req_ids;       /* [n_seqs] */
    const int32_t* is_prefill;    /* [n_seqs] 1 = prompt rows, 0 = one decode row */
    const int32_t* cu_q_lens;     /* [n_seqs + 1] rows of sequence i: cu[i] .. cu[i+1]-1 */
    const int32_t* ctx_lens;      /* [n_seqs] keys after this step's rows are appended */
    const int32_t* block_tables;  /* [n_seqs * max_blocks] physical blocks, -1 padded */
    const int32_t* token_ids;     /* [n_rows] token of each row (embedding input) */
    const int32_t* positions;     /* [n_rows] its position (RoPE) */
    const int32_t* slot_mapping;  /* [n_rows] its KV slot = block*16 + position%16 */
    const int32_t* sample_rows;   /* [n_seqs] row whose logits give the next token */
} ql_step_plan;

typedef struct {
    int n_active, n_pending, free_blocks, n_finished;
} ql_batcher_counts;

typedef struct {
    int req_id, reason, prompt_len, n_tokens;   /* n_tokens = prompt + generated */
} ql_finished;

/* A batcher owning an allocator of n_blocks (fresh-pool LIFO order 0, 1, 2, ...). */
hipError_t ql_batcher_create(int n_blocks, int max_active, int eos_token, ql_batcher** out);
/* A batcher using an existing LIFO stack of free block indices (e.g. PagedKVCache's
 * free_blocks / free_count): blocks are popped and pushed exactly as
 * paged_kv_allocate_block / paged_kv_free_block do. */
hipError_t ql_batcher_create_on_stack(int* free_blocks, int* free_count, int n_blocks,
                                      int max_active, int eos_token, ql_batcher** out);
hipError_t ql_batcher_destroy(ql_batcher* b);
/* prompt_len > 0, max_gen > 0; the prompt is copied. */
hipError_t ql_batcher_add_request(ql_batcher* b, int req_id, const int32_t* prompt,
                                  int prompt_len, int max_gen);
hipError_t ql_batcher_plan(ql_batcher* b, ql_step_plan* plan);
hipError_t ql_batcher_commit(ql_batcher* b, const int32_t* sampled, int n_seqs);
hipError_t ql_batcher_stats(const ql_batcher* b, ql_batcher_counts* counts);
/* Oldest finished request: *got = 1 and up to cap of its tokens copied, or *got = 0. */
hipError_t ql_batcher_pop_finished(ql_batcher* b, ql_finished* ev, int32_t* tokens, int cap,
                                   int* got);

/* ---- greedy sampling ----------------------------------------------------------------
 * out[r] = the first index of the maximum of row r (logits + r*ld, cols values): the
 * strict-">" scan of argmax_kernel (src/continuous_batch.cu:12-25), batched over
 * rows, starting from its -1e20f: NaN and values at or below -1e20 never win, and a
 * row with no value above -1e20 gives 0.  (src/fp16_forward.cu:259-283 starts from
 * -FLT_MAX; the two agree on every row holding a value above -1e20, which includes
 * every binary16 row with a finite value.) */
hipError_t ql_argmax_f32(const float* logits, int rows, int cols, int64_t ld, int32_t* out,
                         hipStream_t stream);
hipError_t ql_argmax_f16(const uint16_t* logits, int rows, int cols, int64_t ld, int32_t* out,
                         hipStream_t stream);

/* ---- fp16 library GEMM ------------------------------------------------------------------
 * y[M, N] = x[M, K] W[N, K]^T (row-major, weights [out_features, in_features]), fp16
 * in/out, fp32 accumulation, on hipBLASLt -- the hgemm/cuBLAS projections of
 * src/fp16_forward.cu:184-186,204,211,219-221.  A per-device library context
 * (handle, per-(M,N,K) plans, a 64 MB workspace per stream) is created on first use
 * and kept until the process ends. */
hipError_t ql_gemm_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, int M, int N, int K,
                       hipStream_t stream);
/* Replaces the cached plan's algorithm for (M, N, K) by the fastest of the library
 * heuristic's first 32 candidates, timed on scratch operands by the host's clock
 * from launch to completion, launch costs included (the weights rotate
 * over copies of >= 512 MB in total, so they stream from HBM as in a multi-layer
 * step).  The fastest four are re-timed with the heuristic's first choice in three
 * alternating rounds, and the first choice is kept unless one of them is more than
 * 3% faster over those rounds.  Setup only: allocates and frees scratch, synchronizes `stream`, and must
 * not run under graph capture.  Later ql_gemm_f16 calls of that shape use the
 * chosen algorithm; results stay within the GEMM's fp32-accumulation tolerance
 * but may differ in the last bits from the untuned plan.  No counterpart in the
 * reference (its cuBLAS calls take the library default). */
hipError_t ql_gemm_tune_f16(int M, int N, int K, hipStream_t stream);

/* ---- FP8 weight codec and FP8-weight GEMM (quantlib) ------------------------------------
 * quantlib_fp16_to_fp8_e4m3/e5m2, quantlib_fp8_to_fp16, quantlib_fp8_gemm
 * (quantlib_src/include/quantlib.h:10-28, kernels/fp8_convert.cu:15-173,
 * kernels/fp8_gemm.cu:34-139).  Scales per group of the row-major [rows, cols] matrix
 * (per-tensor: all of it; per-channel: one row; per-group: runs of group_size
 * elements): scale = fmax / max|x| (max < 1e-8 -> 1), fmax 448 (E4M3) / 57344 (E5M2);
 * q = encode(x * scale); dequant = binary16(decode(q) / scale).
 * QL_FP8_MODE_REFERENCE: the reference's algorithm in IEEE arithmetic -- its max
 *   reduction sees only the elements at offsets < 32 mod 128 of each group, and its
 *   encoder truncates the mantissa, flushes subnormals to zero and clamps.
 * QL_FP8_MODE_OCP: the whole group's max and the OCP E4M3FN / E5M2 encodings (round
 *   to nearest even, subnormals, saturation to +-fmax), on gfx950's FP8 conversions. */
#define QL_FP8_E4M3 0
#define QL_FP8_E5M2 1
#define QL_FP8_MODE_REFERENCE 0
#define QL_FP8_MODE_OCP 1
/* Decoding only (ql_fp8_dequantize, ql_fp8_gemm_f16, the FP8 engine layers):
 * reference-mode codes that ql_fp8_count_ref_special found free of the codes whose
 * reference decode differs from the OCP decode (the reference encoder writes them
 * only for NaN inputs).  Such codes decode to the same values either way (0x80:
 * -0 against the reference's +0, which no product or sum sees), so the GEMM skips
 * the per-code check of QL_FP8_MODE_REFERENCE and gives its results;
 * ql_fp8_dequantize runs the reference decoder as for QL_FP8_MODE_REFERENCE.  No
 * counterpart in the reference: for callers that hold static weights. */
#define QL_FP8_MODE_REFERENCE_CLEAN 2
#define QL_QUANT_PER_TENSOR 0    /* QuantGranularity values of quant_types.h:17-21 */
#define QL_QUANT_PER_CHANNEL 1
#define QL_QUANT_PER_GROUP 2

/* number of scales for a [rows, cols] matrix (host) */
hipError_t ql_fp8_num_scales(int rows, int cols, int granularity, int group_size, int* n_scales);
hipError_t ql_fp8_scales(const uint16_t* src, int rows, int cols, int format, int granularity,
                         int group_size, int mode, float* scales, hipStream_t stream);
/* scales (device, n_scales floats) are computed and written too */
hipError_t ql_fp8_quantize(const uint16_t* src, int rows, int cols, int format, int granularity,
                           int group_size, int mode, uint8_t* dst, float* scales,
                           hipStream_t stream);
hipError_t ql_fp8_dequantize(const uint8_t* src, const float* scales, int rows, int cols,
                             int format, int granularity, int group_size, int mode,
                             uint16_t* dst, hipStream_t stream);
/* *count (device) = the number of the n codes (16-byte aligned) whose reference decode
 * differs from the OCP decode: E4M3 exponent 0 with a mantissa and |code| 0x7F, E5M2
 * exponent 0 with a mantissa and exponent 31.  Zero: the codes may be decoded with
 * QL_FP8_MODE_REFERENCE_CLEAN.  No counterpart in the reference. */
hipError_t ql_fp8_count_ref_special(const uint8_t* codes, size_t n, int format,
                                    unsigned long long* count, hipStream_t stream);
/* C[M, N] = A[M, K] (dequant W[N, K])^T, fp32 accumulation, fp16 out
 * (quantlib_src/kernels/fp8_gemm.cu:34-139, quantlib_fp8_gemm).  M <= 2 with
 * K % 16 == 0, M * ceil(K / 1024) <= 32, scales per tensor, per row or in groups of
 * a multiple of 16 dividing K, and 16-byte aligned A and W streams W as contiguous
 * runs of rows (no matrix cores, no workspace used).  Otherwise M <= 64 with
 * N % 16 == 0, K % 64 == 0, 16 | group length and 16-byte aligned A and W streams W
 * once and dequantizes in registers (multiplying by 1/scale); there the workspace
 * is optional and, when it holds ql_fp8_gemm_workspace_size bytes (16-byte aligned,
 * C 8-byte aligned), splits K over more workgroups with fp32 partials summed in a
 * fixed order.  Otherwise W is dequantized into workspace (N*K*2 bytes, 16-byte
 * aligned) and ql_gemm_f16 runs. */
hipError_t ql_fp8_gemm_workspace_size(int M, int N, int K, int granularity, int group_size,
                                      size_t* bytes);
hipError_t ql_fp8_gemm_f16(const uint16_t* A, const uint8_t* W, const float* scales, int M, int N,
                           int K, int format, int granularity, int group_size, int mode,
                           uint16_t* C, void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

/* ---- decoder-layer engine (fp16; hipBLASLt GEMMs + the kernels above) -----------------
 * One fp16 decoder layer for every row of a batched step, in the order of
 * fp16_layer_forward (src/fp16_forward.cu:167-223):
 *   x += delta_in; y = rmsnorm(x)*attn_norm; qkv = y Wqkv^T; RoPE + paged KV append;
 *   a = attention over the paged pool; x += a Wo^T; y = rmsnorm(x)*ffn_norm;
 *   delta_out = (silu(y Wg^T) * (y Wu^T)) Wd^T
 * delta_in = NULL for the first layer; delta_out is added by the next layer (or by
 * ql_engine_logits_f16).  Weights are row-major [out_features, in_features] fp16;
 * wqkv stacks the Q rows (n_heads*head_dim), then K, then V (n_kv_heads*head_dim
 * each).  The step arrays are a ql_step_plan's, on the device.  A step whose rows
 * are all single-token decodes (max_q_len == 1, n_rows == n_seqs) uses the split
 * decode with the engine's workspace.  The engine owns its activation buffers and
 * workspaces (allocated once by ql_engine_create, sized for max_rows rows,
 * max_seqs sequences and max_ctx_len keys); the per-step calls allocate nothing.
 * GEMM plans are cached per (rows, out, in) shape; use an engine from one host
 * thread at a time. */
typedef struct {
    int hidden, n_heads, n_kv_heads, head_dim, ffn;
    float rope_theta, rms_eps;
    int rope_pairing;
} ql_layer_dims;

typedef struct {
    const uint16_t* attn_norm;   /* [hidden] */
    const uint16_t* wqkv;        /* [(n_heads + 2*n_kv_heads)*head_dim, hidden] */
    const uint16_t* wo;          /* [hidden, n_heads*head_dim] */
    const uint16_t* ffn_norm;    /* [hidden] */
    const uint16_t* w_gate;      /* [ffn, hidden] */
    const uint16_t* w_up;        /* [ffn, hidden] */
    const uint16_t* w_down;      /* [hidden, ffn] */
} ql_layer_weights;

typedef struct {
    int n_rows, n_seqs, max_q_len, max_ctx_len, max_blocks;
    const int32_t* positions;     /* device [n_rows] */
    const int32_t* slot_mapping;  /* device [n_rows] */
    const int32_t* cu_q_lens;     /* device [n_seqs + 1] */
    const int32_t* ctx_lens;      /* device [n_seqs] */
    const int32_t* block_tables;  /* device [n_seqs * max_blocks] */
    uint16_t* const* k_blocks;    /* device block-pointer tables of the pool */
    uint16_t* const* v_blocks;
    int n_blocks, n_layers;
} ql_step_device;

typedef struct ql_engine ql_engine;

hipError_t ql_engine_create(const ql_layer_dims* dims, int max_rows, int max_seqs, int max_ctx_len,
                            ql_engine** out);
hipError_t ql_engine_destroy(ql_engine* e);
hipError_t ql_engine_layer_f16(ql_engine* e, const ql_layer_weights* w, int layer, uint16_t* x,
                               const uint16_t* delta_in, uint16_t* delta_out,
                               const ql_step_device* step, hipStream_t stream);
/* ql_gemm_tune_f16 for the four fp16 layer GEMM shapes of a step of `rows` rows
 * (1 <= rows <= max_rows): QKV, O, gate/up, down.  Setup only (see
 * ql_gemm_tune_f16).  No counterpart in the reference. */
hipError_t ql_engine_tune(ql_engine* e, int rows, hipStream_t stream);
/* ---- the same layer on FP8 weights (W8A16) --------------------------------------------
 * The quantized forward of the reference: quantize_model
 * (src/quant_forward.cu:57-101) stores every weight matrix as FP8 codes + scales
 * and the layer GEMMs run through quantlib_fp8_gemm (src/forward.cu:52-70,
 * 185-238).  Here each layer GEMM is ql_fp8_gemm_f16 (the register path for steps
 * of <= 64 rows); the norms stay fp16.  The five matrices share one format,
 * granularity, group size and mode; wqkv is the row-wise stack of the Q, K and V
 * matrices, whose per-channel or per-group (group_size dividing hidden) codes and
 * scales are those of the three matrices quantized separately.
 * ql_engine_create_fp8 is ql_engine_create plus the FP8 GEMM workspace for that
 * granularity and group size; such an engine runs both layer kinds. */
typedef struct {
    const uint8_t* codes;   /* [out_features, in_features] FP8 codes */
    const float* scales;    /* ql_fp8_num_scales(out_features, in_features, ...) floats */
} ql_fp8_weight;

typedef struct {
    const uint16_t* attn_norm;
    ql_fp8_weight wqkv, wo;
    const uint16_t* ffn_norm;
    ql_fp8_weight w_gate, w_up, w_down;
    int format, granularity, group_size, mode;   /* QL_FP8_*, QL_QUANT_*, QL_FP8_MODE_* */
} ql_layer_weights_fp8;

hipError_t ql_engine_create_fp8(const ql_layer_dims* dims, int max_rows, int max_seqs,
                                int max_ctx_len, int granularity, int group_size, ql_engine** out);
hipError_t ql_engine_layer_fp8(ql_engine* e, const ql_layer_weights_fp8* w, int layer, uint16_t* x,
                               const uint16_t* delta_in, uint16_t* delta_out,
                               const ql_step_device* step, hipStream_t stream);

/* ---- HIP graphs of library calls ----------------------------------------------------------
 * No counterpart in the reference (it launches every op of every token from the host).
 * ql_graph_begin starts capturing `stream` (not the null stream; thread-local mode, so
 * an allocation or synchronisation on this thread during capture fails); the library
 * calls that follow are recorded, not run; ql_graph_end instantiates them.
 * ql_graph_launch replays them on any stream.  Capturable: every entry point above
 * once each GEMM shape has run eagerly (plan and workspace created).  Values read
 * from device memory (positions, slots, ctx_lens, block tables, inputs) may change
 * between replays; host arguments and pointers are those of the capture. */
typedef struct ql_graph ql_graph;
hipError_t ql_graph_begin(hipStream_t stream);
hipError_t ql_graph_end(hipStream_t stream, ql_graph** out);
hipError_t ql_graph_launch(ql_graph* g, hipStream_t stream);
hipError_t ql_graph_destroy(ql_graph* g);

/* x += delta_in over all n_rows rows, final RMSNorm, gather the n_sample rows
 * sample_rows[] (device), logits = rows lm_head^T ([n_sample, vocab] fp16) and, if
 * tokens is not NULL, tokens[i] = argmax of logits row i (device). */
hipError_t ql_engine_logits_f16(ql_engine* e, uint16_t* x, const uint16_t* delta_in,
                                const uint16_t* final_norm, const uint16_t* lm_head, int vocab,
                                const int32_t* sample_rows, int n_sample, int n_rows,
                                uint16_t* logits, int32_t* tokens, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QUANTLIB_AMD_H */
