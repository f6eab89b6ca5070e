/*
 * quantlib_compat.h -- drop-in replacements for the reference's launchers and
 * KV-cache types, with the reference's names, argument order and meaning
 * (cudaStream_t becomes hipStream_t).  A caller of samfrazerdutton/Quant-lib's
 * kernels links libquantlib_amd.so instead of the .cu objects and keeps its
 * call sites.
 *
 * Like the reference, the launchers return void: a launch error stays pending
 * for the caller's next hipGetLastError()/hipStreamSynchronize() check.  An
 * argument the reference would pass to a malformed launch (negative sizes,
 * odd head_dim) is rejected without launching; hipGetLastError() does not
 * report it, ql_* entry points do (quantlib_amd.h).
 *
 * Behaviour kept from the reference on purpose:
 *   - launch_rope / launch_fp16_rope rotate interleaved pairs (2i, 2i+1) and
 *     use the row index as the position (kernels/rope.cu:20,36).
 *   - kvcache_append writes at cache->current_len; the caller advances it
 *     (src/forward.cu:264).
 *   - paged_kv_create hands out blocks from a LIFO free list, so a fresh pool
 *     gives blocks 0,1,2,... (src/paged_kvcache.cu:49-53,89-93).
 */
#ifndef QUANTLIB_COMPAT_H
#define QUANTLIB_COMPAT_H

#include <hip/hip_runtime_api.h>
#include <hip/hip_fp16.h>
#include <stddef.h>

/* ---- kernels/ launchers (C++ linkage, as in the reference) ------------ */
/* kernels/rmsnorm.cu:51 */
void launch_rmsnorm(const float* x, const float* weight, float* out, int rows, int dim,
                    float eps, hipStream_t stream);
/* kernels/rope.cu:44 */
void launch_rope(float* x, int seq_len, int n_heads, int head_dim, float theta,
                 hipStream_t stream);
/* kernels/feedforward.cu:27 */
void launch_swiglu(const float* gate, const float* up, float* out, int rows, int ffn_dim,
                   hipStream_t stream);
/* kernels/softmax.cu:88 */
void launch_softmax(const float* input, float* output, int rows, int cols,
                    hipStream_t stream);
/* kernels/fp16_ops.cu:113 */
void launch_fp16_rmsnorm(const __half* x, const __half* w, __half* out, int rows, int dim,
                         float eps, hipStream_t stream);
/* kernels/fp16_ops.cu:120 */
void launch_fp16_rope(__half* x, int seq_len, int n_heads, int head_dim, float theta,
                      hipStream_t stream);
/* kernels/fp16_ops.cu:129 */
void launch_fp16_swiglu(const __half* gate, const __half* up, __half* out, int rows,
                        int ffn_dim, hipStream_t stream);
/* kernels/fp16_ops.cu:137 */
void launch_fp16_embed(const __half* table, __half* out, int token_id, int hidden_dim,
                       hipStream_t stream);
/* kernels/fp16_ops.cu:144 */
void launch_fp16_add(__half* x, const __half* y, int n, hipStream_t stream);
/* kernels/fp16_ops.cu:149 */
void launch_fp16_to_fp32(const __half* src, float* dst, int n, hipStream_t stream);
/* kernels/flash_attention.cu:169-182 (head_dim 1..64, the reference's range, or 128;
 * see ql_flash_attention_f16) */
void launch_flash_attention(const __half* Q, const __half* K, const __half* V, __half* Out,
                            int seq_len, int n_heads, int n_kv_heads, int head_dim, int causal,
                            hipStream_t stream);
/* src/fp16_forward.cu:285-297: the index of the largest of logits[0 .. vocab_size)
 * (the first such index), copied to the host; the call synchronises the stream and,
 * like the reference, allocates and frees a 4-byte device buffer.  Where the
 * reference would exit (a failed HIP call) it returns -1; vocab_size <= 0 gives 0,
 * as the reference's empty scan does. */
int fp16_greedy_sample(const float* logits, int vocab_size, hipStream_t stream);

/* ---- inline kernels of src/forward.cu / src/fp16_forward.cu given launchers ---- */
/* src/forward.cu:128-135 (add_residual_kernel + its static launcher) */
void add_residual(float* x, const float* d, int n, hipStream_t stream);
/* src/forward.cu:137-141 (embed_kernel, launched at :256-257) */
void launch_embed(float* out, const float* tbl, int tok, int hd, hipStream_t stream);
/* src/fp16_forward.cu:148-154 (fp16_kvcache_append, launched at :194-199) */
void launch_fp16_kvcache_append(__half* k_cache, __half* v_cache, const __half* k_new,
                                const __half* v_new, int layer, int pos, int n_kv_heads,
                                int head_dim, int max_seq, int n_layers,
                                hipStream_t stream);

/* src/quant_forward.cu:18-21 (fp32_to_fp16_kernel, launched by sgemm at
 * src/forward.cu:62-64): dst[i] = __float2half(src[i]).  Its partner
 * fp16_to_fp32_kernel (src/quant_forward.cu:23-26, src/forward.cu:66-67) is
 * launch_fp16_to_fp32 above. */
void launch_fp32_to_fp16(const float* src, __half* dst, int n, hipStream_t stream);

/* ---- fp32 contiguous KV cache (include/kv_cache.h:12-36) ------------------- */
typedef struct {
    float* k_cache; /* [n_layers * max_seq_len * n_heads * head_dim] */
    float* v_cache;
    int n_layers;
    int max_seq_len;
    int n_heads;
    int head_dim;
    int current_len;
} KVCache;

KVCache* kvcache_create(int n_layers, int max_seq_len, int n_heads, int head_dim);
void kvcache_free(KVCache* cache);
void kvcache_append(KVCache* cache, int layer, const float* new_k, const float* new_v,
                    hipStream_t stream);
float* kvcache_get_k(KVCache* cache, int layer);
float* kvcache_get_v(KVCache* cache, int layer);

/* ---- fp16 contiguous KV cache (src/fp16_forward.cu:115-145) ---------------- */
typedef struct {
    __half* k_cache; /* [n_layers, max_seq, n_kv_heads, head_dim] */
    __half* v_cache;
    int n_layers, max_seq, n_kv_heads, head_dim;
    int current_len;
} FP16KVCache;

FP16KVCache* fp16_kvcache_create(int n_layers, int max_seq, int n_kv_heads, int head_dim);
void fp16_kvcache_free(FP16KVCache* c);

/* ---- paged KV cache (include/paged_kvcache.h:9-34) ------------------------- */
#ifndef PAGE_SIZE
#define PAGE_SIZE 16
#endif

typedef struct {
    __half** k_blocks; /* [n_blocks] device array of device pointers to K blocks */
    __half** v_blocks;
    int n_blocks;
    int n_layers;
    int n_kv_heads;
    int head_dim;
    int* free_blocks; /* host LIFO stack of free block indices */
    int free_count;
    int** block_tables; /* host: seq -> block indices (-1 = unused) */
    int max_seqs;
    int max_blocks_per_seq;
} PagedKVCache;

extern "C" {
PagedKVCache* paged_kv_create(int n_blocks, int n_layers, int n_kv_heads, int head_dim,
                              int max_seqs, int max_blocks_per_seq);
void paged_kv_free(PagedKVCache* cache);
int paged_kv_allocate_block(PagedKVCache* cache);
void paged_kv_free_block(PagedKVCache* cache, int block_idx);
}

/* ---- quantlib FP8 (quantlib_src/include/quant_types.h:15-45, quantlib.h:10-43) -----
 * Same types and names; the conversions run the reference's algorithm
 * (QL_FP8_MODE_REFERENCE of quantlib_amd.h) and, like the reference, allocate the
 * QuantMatrix's device buffers (freed by quantlib_free).  quantlib_fp8_gemm keeps
 * its workspace (split-K partials, or the dequantized weights when M > 64) in a
 * device buffer per (device, stream) that grows on demand: the first call with
 * a larger need on a stream allocates (after waiting for that stream), so calls
 * on different streams never share a buffer. */
typedef uint8_t fp8_e4m3_t;
typedef uint8_t fp8_e5m2_t;

typedef enum {
    QUANT_PER_TENSOR = 0,
    QUANT_PER_CHANNEL = 1,
    QUANT_PER_GROUP = 2
} QuantGranularity;

typedef struct {
    float* scales;
    float* zeros;
    int group_size;
    QuantGranularity granularity;
    int n_scales;
} QuantParams;

typedef struct {
    void* data;
    QuantParams params;
    int rows;
    int cols;
    int bits;
    char format[16];
} QuantMatrix;

extern "C" {
QuantMatrix quantlib_fp16_to_fp8_e4m3(const __half* src, int rows, int cols, QuantGranularity gran,
                                      int group_size, hipStream_t stream);
QuantMatrix quantlib_fp16_to_fp8_e5m2(const __half* src, int rows, int cols, QuantGranularity gran,
                                      int group_size, hipStream_t stream);
void quantlib_fp8_to_fp16(const QuantMatrix* qm, __half* dst, hipStream_t stream);
void quantlib_fp8_gemm(const __half* A, const QuantMatrix* W, __half* C, int M, int N, int K,
                       hipStream_t stream);
void quantlib_free(QuantMatrix* qm);
float quantlib_quant_error(const __half* original, const __half* dequantized, int n_elements);
void quantlib_print_stats(const QuantMatrix* qm);
}

#endif /* QUANTLIB_COMPAT_H */
