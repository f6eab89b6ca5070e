/*
 * oracle.h -- CPU restatement of samfrazerdutton/Quant-lib's fused per-layer
 * kernels, used ONLY as the parity checker (tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg).  It is never linked into, loaded by or
 * called from the product library.
 *
 * Plain scalar C, one element at a time, in the order the reference kernels
 * state the arithmetic.  Where the reference relies on CUDA fast-math
 * intrinsics (__expf, powf/sinf/cosf under --use_fast_math, rsqrtf) the
 * oracle uses the accurate libm function instead: the CUDA bits are not
 * reproducible here and are not the specification; the BASELINE tolerances
 * are.  Reductions accumulate in double, so the oracle is at least as accurate
 * as any fp32 reduction order.
 *
 * binary16 values are uint16_t bit patterns; or_f32_to_f16 rounds to nearest
 * even (IEEE 754 default, as __float2half).
 *
 * Which checks pin each function is listed in each function's comment in
 * oracle.c and exercised by tests/test_oracle.py.
 */
#ifndef QL_ORACLE_H
#define QL_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);
void or_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n);
void or_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n);

void or_rmsnorm_f32(const float* x, const float* w, float* out, int rows, int dim, float eps);
void or_rmsnorm_f16(const uint16_t* x, const uint16_t* w, uint16_t* out, int rows, int dim,
                    float eps);
void or_add_rmsnorm_f32(float* x, const float* d, const float* w, float* out, int rows, int dim,
                        float eps);
void or_add_rmsnorm_f16(uint16_t* x, const uint16_t* d, const uint16_t* w, uint16_t* out,
                        int rows, int dim, float eps);
void or_add_f32(float* x, const float* d, int64_t n);
void or_add_f16(uint16_t* x, const uint16_t* d, int64_t n);

float or_rope_inv_freq(int pair, int head_dim, float theta);
void or_rope_cos_sin(int pos, int pair, int head_dim, float theta, float* c, float* s);
void or_rope_f32(float* x, int n_tokens, int n_heads, int head_dim, int64_t row_stride,
                 const int32_t* positions, int pos_offset, float theta, int pairing);
void or_rope_f16(uint16_t* x, int n_tokens, int n_heads, int head_dim, int64_t row_stride,
                 const int32_t* positions, int pos_offset, float theta, int pairing);

void or_swiglu_f32(const float* g, const float* u, float* out, int64_t n);
void or_swiglu_f16(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n);

void or_softmax_f32(const float* in, float* out, int rows, int cols);
void or_softmax_f16(const uint16_t* in, uint16_t* out, int rows, int cols);

/* The reference test's own CPU loop (tests/test_softmax.cu:19-30): fp32
 * sequential sum, per-element division.  Used to rerun that test's check. */
void or_softmax_reftest_cpu(const float* in, float* out, int rows, int cols);
/* Inputs of tests/test_softmax.cu:45-47: srand(seed); x = rand()/RAND_MAX*4-2. */
void or_reftest_softmax_inputs(float* out, int64_t n, unsigned seed);

void or_embed_f32(const float* table, const int32_t* ids, int n_tokens, int vocab, int dim,
                  float* out);
void or_embed_f16(const uint16_t* table, const int32_t* ids, int n_tokens, int vocab, int dim,
                  uint16_t* out);

void or_kv_append_f32(float* k_cache, float* v_cache, const float* k_new, const float* v_new,
                      int layer, int pos, int n_tokens, int n_kv_heads, int head_dim,
                      int max_seq, int n_layers);
void or_kv_append_f16(uint16_t* k_cache, uint16_t* v_cache, const uint16_t* k_new,
                      const uint16_t* v_new, int layer, int pos, int n_tokens, int n_kv_heads,
                      int head_dim, int max_seq, int n_layers);

/* Paged append into a host pool: block b of K starts at k_pool + block_offset[b]
 * elements (so any block->address map can be checked), block layout
 * [n_layers, 16, n_kv_heads, head_dim]. */
void or_paged_kv_append_f16(uint16_t* k_pool, uint16_t* v_pool, const int64_t* block_offset,
                            int n_blocks, const int32_t* slots, const uint16_t* k_new,
                            const uint16_t* v_new, int n_tokens, int layer, int n_layers,
                            int n_kv_heads, int head_dim);

/* Attention (fp32 / fp16 I/O, double inside): queries are the last q_len
 * positions of a kv_len-long context; kv head of head h = h*n_kv_heads/n_heads. */
void or_attention_f32(const float* q, const float* k, const float* v, float* out, int q_len,
                      int kv_len, int n_heads, int n_kv_heads, int head_dim, int64_t q_stride,
                      int64_t kv_stride, int64_t o_stride, int causal);
void or_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                      int q_len, int kv_len, int n_heads, int n_kv_heads, int head_dim,
                      int64_t q_stride, int64_t kv_stride, int64_t o_stride, int causal);
/* The reference test's fp32 CPU loop and inputs (tests/test_attention.cu:22-56, 77-82). */
void or_attention_reftest_cpu(const float* Q, const float* K, const float* V, float* out,
                              int seq_len, int n_heads, int head_dim);
void or_reftest_attention_inputs(float* q, float* k, float* v, int64_t n, unsigned seed);

/* y = x W^T (weights [out, in]), double accumulation, binary16 result. */
void or_matmul_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, int M, int N, int K);
/* First index of the row maximum (strict >, NaN ignored, 0 if none above -inf). */
void or_argmax_f32(const float* x, int rows, int cols, int32_t* out);

/* FP8 codec: fmt 0 = E4M3, 1 = E5M2; mode 0 = the reference's (warp-0 scale,
 * truncating), 1 = OCP (full-group scale, RNE, saturating); gran 0/1/2 =
 * per-tensor / per-channel / per-group. */
uint8_t or_fp8_encode_ref(float v, int fmt);
float or_fp8_decode_ref(uint8_t q, int fmt);
uint8_t or_fp8_encode_ocp(float v, int fmt);
float or_fp8_decode_ocp(uint8_t q, int fmt);
int or_fp8_num_scales(int rows, int cols, int gran, int group_size);
void or_fp8_scales(const uint16_t* src, int rows, int cols, int fmt, int gran, int group_size,
                   int mode, float* scales);
void or_fp8_quantize(const uint16_t* src, int rows, int cols, int fmt, int gran, int group_size,
                     int mode, uint8_t* dst, float* scales);
void or_fp8_dequantize(const uint8_t* src, const float* scales, int rows, int cols, int fmt,
                       int gran, int group_size, int mode, uint16_t* dst);

/* Inputs of quantlib_src/tests/test_fp8.cu:27-29. */
void or_reftest_fp8_inputs(float* out, int64_t n, unsigned seed);
void or_reftest_gemm_inputs(float* a, int64_t na, float* w, int64_t nw, unsigned seed);
void or_gemm_reftest_cpu(const uint16_t* a, const uint16_t* w, float* c, int M, int N, int K);
long long or_check_recip_division(void);

#ifdef __cplusplus
}
#endif

#endif
