/*
 * oracle.c -- CPU restatement of the reference's hot-path arithmetic.
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the parity checker, never the
 * thing measured or shipped.  Built with -O2 -ffp-contract=off, no fast-math,
 * so every rounding step below happens exactly as written.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- binary16 codec --------------------------------------------------------
 * IEEE 754 binary16 <-> binary32, round to nearest even.  The arithmetic of
 * __float2half/__half2float used throughout kernels/fp16_ops.cu.
 * Pinned by: exhaustive comparison with numpy float16 over all 65536 halves,
 * every half-way point between consecutive halves, overflow and subnormal
 * boundaries (tests/test_oracle.py::test_f16_*). */
uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan (quiet, top payload bits kept) */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
    if (ax >= 0x477ff000u) /* >= 65520: rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) { /* below 2^-14: binary16 subnormal or zero */
        if (ax <= 0x33000000u) return (uint16_t)sign; /* <= 2^-25 rounds to 0 */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e; /* value / 2^-24 = m >> shift */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    const uint32_t r = ax - 0x38000000u; /* rebias 127 -> 15 */
    uint32_t h = r >> 13;
    const uint32_t rem = r & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: m * 2^-24, normalise */
            e = 113;
            while (!(m & 0x400u)) {
                m <<= 1;
                e--;
            }
            bits = sign | (e << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void or_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = or_f32_to_f16(src[i]);
}

void or_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = or_f16_to_f32(src[i]);
}

/* ---- RMSNorm -----------------------------------------------------------------
 * kernels/rmsnorm.cu:27-48 (fp32) and kernels/fp16_ops.cu:18-41 (fp16):
 *   ss = sum x^2;  r = 1/sqrt(ss/dim + eps)  (rsqrtf in the reference);
 *   out = (x*r)*w.
 * ss is accumulated in double and rounded once to fp32.
 * Pinned by: constant-row and one-hot closed forms, scale invariance
 * (eps = 0), the eps term (all-zero row gives 0, tiny rows feel eps), weight
 * indexing with a non-uniform w (tests/test_oracle.py::test_rmsnorm_*). */
static float rms_inv(double ss, int dim, float eps) {
    const float ms = (float)ss / (float)dim;
    return 1.0f / sqrtf(ms + eps);
}

void or_rmsnorm_f32(const float* x, const float* w, float* out, int rows, int dim, float eps) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * dim;
        double ss = 0.0;
        for (int i = 0; i < dim; ++i) ss += (double)xr[i] * (double)xr[i];
        const float inv = rms_inv(ss, dim, eps);
        for (int i = 0; i < dim; ++i) out[(size_t)r * dim + i] = (xr[i] * inv) * w[i];
    }
}

void or_rmsnorm_f16(const uint16_t* x, const uint16_t* w, uint16_t* out, int rows, int dim,
                    float eps) {
    for (int r = 0; r < rows; ++r) {
        const uint16_t* xr = x + (size_t)r * dim;
        double ss = 0.0;
        for (int i = 0; i < dim; ++i) {
            const double v = or_f16_to_f32(xr[i]);
            ss += v * v;
        }
        const float inv = rms_inv(ss, dim, eps);
        for (int i = 0; i < dim; ++i)
            out[(size_t)r * dim + i] =
                or_f32_to_f16((or_f16_to_f32(xr[i]) * inv) * or_f16_to_f32(w[i]));
    }
}

/* Residual add then RMSNorm of the updated (rounded) row: the unfused chain
 * add_residual + launch_rmsnorm (src/forward.cu:228-232) and
 * launch_fp16_add + launch_fp16_rmsnorm (src/fp16_forward.cu:213-216).
 * Pinned by: equality with or_add_* followed by or_rmsnorm_* (the unfused
 * chain) and the rmsnorm pins above. */
void or_add_rmsnorm_f32(float* x, const float* d, const float* w, float* out, int rows, int dim,
                        float eps) {
    or_add_f32(x, d, (int64_t)rows * dim);
    or_rmsnorm_f32(x, w, out, rows, dim, eps);
}

void or_add_rmsnorm_f16(uint16_t* x, const uint16_t* d, const uint16_t* w, uint16_t* out,
                        int rows, int dim, float eps) {
    or_add_f16(x, d, (int64_t)rows * dim);
    or_rmsnorm_f16(x, w, out, rows, dim, eps);
}

/* src/forward.cu:128-130: x += d.  kernels/fp16_ops.cu:92-100: x = h(f(x)+f(d)).
 * Pinned by: numpy float32 / float16 addition (same rounding), exhaustive on
 * a grid of binary16 pairs. */
void or_add_f32(float* x, const float* d, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] + d[i];
}

void or_add_f16(uint16_t* x, const uint16_t* d, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        x[i] = or_f32_to_f16(or_f16_to_f32(x[i]) + or_f16_to_f32(d[i]));
}

/* ---- RoPE ---------------------------------------------------------------------
 * kernels/rope.cu:20-41 and kernels/fp16_ops.cu:49-62, pair i of each head:
 *   inv_freq = 1 / theta^((2i)/d)   exponent as an fp32 division (rope.cu:35),
 *                                   the power in double rounded to fp32
 *   angle    = (float)pos * inv_freq                       (rope.cu:36)
 *   c, s     = cos/sin(angle) in double rounded to fp32    (rope.cu:37-38)
 *   y0 = fma(x0, c, -(x1*s)),  y1 = fma(x0, s, x1*c)       (rope.cu:40-41)
 * pairing 0 = interleaved (2i, 2i+1) as the reference; 1 = rotate-half (i, i+d/2).
 * position = positions ? positions[t] : pos_offset + t (reference: row index).
 * Pinned by: pos = 0 identity; pair 0 has inv_freq = 1 so its angle is pos;
 * inv_freq closed form at d = 4 (theta^-1/2); per-pair norm preservation (the
 * reference's own test, tests/test_attention.cu:110-121); agreement with a
 * complex-exponential formulation (x0 + i x1) e^{i angle} in float64; the
 * interleaved/rotate-half permutation identity (tests/test_oracle.py::test_rope_*). */
float or_rope_inv_freq(int pair, int head_dim, float theta) {
    const float e = (2.0f * (float)pair) / (float)head_dim;
    const float p = (float)pow((double)theta, (double)e);
    return 1.0f / p;
}

void or_rope_cos_sin(int pos, int pair, int head_dim, float theta, float* c, float* s) {
    const float a = (float)pos * or_rope_inv_freq(pair, head_dim, theta);
    *c = (float)cos((double)a);
    *s = (float)sin((double)a);
}

static void rope_pair(float x0, float x1, float c, float s, float* y0, float* y1) {
    *y0 = fmaf(x0, c, -(x1 * s));
    *y1 = fmaf(x0, s, x1 * c);
}

void or_rope_f32(float* x, int n_tokens, int n_heads, int head_dim, int64_t row_stride,
                 const int32_t* positions, int pos_offset, float theta, int pairing) {
    const int np = head_dim / 2;
    for (int t = 0; t < n_tokens; ++t) {
        const int pos = positions ? positions[t] : pos_offset + t;
        for (int p = 0; p < np; ++p) {
            float c, s;
            or_rope_cos_sin(pos, p, head_dim, theta, &c, &s);
            const int i0 = pairing == 0 ? 2 * p : p;
            const int i1 = pairing == 0 ? 2 * p + 1 : p + np;
            for (int h = 0; h < n_heads; ++h) {
                float* v = x + (size_t)t * row_stride + (size_t)h * head_dim;
                float y0, y1;
                rope_pair(v[i0], v[i1], c, s, &y0, &y1);
                v[i0] = y0;
                v[i1] = y1;
            }
        }
    }
}

void or_rope_f16(uint16_t* x, int n_tokens, int n_heads, int head_dim, int64_t row_stride,
                 const int32_t* positions, int pos_offset, float theta, int pairing) {
    const int np = head_dim / 2;
    for (int t = 0; t < n_tokens; ++t) {
        const int pos = positions ? positions[t] : pos_offset + t;
        for (int p = 0; p < np; ++p) {
            float c, s;
            or_rope_cos_sin(pos, p, head_dim, theta, &c, &s);
            const int i0 = pairing == 0 ? 2 * p : p;
            const int i1 = pairing == 0 ? 2 * p + 1 : p + np;
            for (int h = 0; h < n_heads; ++h) {
                uint16_t* v = x + (size_t)t * row_stride + (size_t)h * head_dim;
                float y0, y1;
                rope_pair(or_f16_to_f32(v[i0]), or_f16_to_f32(v[i1]), c, s, &y0, &y1);
                v[i0] = or_f32_to_f16(y0);
                v[i1] = or_f32_to_f16(y1);
            }
        }
    }
}

/* ---- SwiGLU ---------------------------------------------------------------------
 * kernels/feedforward.cu:4-6,24 and kernels/fp16_ops.cu:74-77:
 *   out = (g / (1 + exp(-g))) * u   (fp32; fp16 variant rounds the result).
 * Pinned by: silu(0) = 0; u = 0 gives 0; silu(g) - silu(-g) = g; large |g|
 * limits; scipy.special.expit(g) * g * u in float64 (tests/test_oracle.py::test_swiglu_*). */
static float silu_mul(float g, float u) {
    const float e = expf(-g);
    return (g / (1.0f + e)) * u;
}

void or_swiglu_f32(const float* g, const float* u, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = silu_mul(g[i], u[i]);
}

void or_swiglu_f16(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        out[i] = or_f32_to_f16(silu_mul(or_f16_to_f32(g[i]), or_f16_to_f32(u[i])));
}

/* ---- softmax --------------------------------------------------------------------
 * kernels/softmax.cu:44-85:
 *   m = max(-FLT_MAX, x...);  e = exp(x - m);  out = e * (1/sum e)
 * The sum is accumulated in double and rounded to fp32 before the reciprocal.
 * The fp16 variant (no reference kernel) is the same arithmetic on widened
 * inputs with an RNE binary16 result.
 * Pinned by: the reference test's own check (tests/test_softmax.cu:88-106:
 * max abs error < 1e-5 against its cpu_softmax on srand(7) inputs, row sums
 * within 1e-5); scipy.special.softmax; shift invariance; causal row 0 = e_0;
 * uniform row = 1/n; -inf gives exactly 0 (tests/test_oracle.py::test_softmax_*). */
static void softmax_row(const float* x, float* e, int cols, float* out_scale) {
    float m = -FLT_MAX;
    for (int c = 0; c < cols; ++c) m = fmaxf(m, x[c]);
    double s = 0.0;
    for (int c = 0; c < cols; ++c) {
        e[c] = expf(x[c] - m);
        s += e[c];
    }
    *out_scale = 1.0f / (float)s;
}

void or_softmax_f32(const float* in, float* out, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        float* o = out + (size_t)r * cols;
        float inv;
        softmax_row(in + (size_t)r * cols, o, cols, &inv);
        for (int c = 0; c < cols; ++c) o[c] = o[c] * inv;
    }
}

void or_softmax_f16(const uint16_t* in, uint16_t* out, int rows, int cols) {
    float* x = (float*)malloc(sizeof(float) * (size_t)cols);
    float* e = (float*)malloc(sizeof(float) * (size_t)cols);
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < cols; ++c) x[c] = or_f16_to_f32(in[(size_t)r * cols + c]);
        float inv;
        softmax_row(x, e, cols, &inv);
        for (int c = 0; c < cols; ++c) out[(size_t)r * cols + c] = or_f32_to_f16(e[c] * inv);
    }
    free(x);
    free(e);
}

void or_softmax_reftest_cpu(const float* in, float* out, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        const float* x = in + (size_t)r * cols;
        float* o = out + (size_t)r * cols;
        float mx = -FLT_MAX;
        for (int c = 0; c < cols; ++c) mx = fmaxf(mx, x[c]);
        float s = 0.0f;
        for (int c = 0; c < cols; ++c) {
            o[c] = expf(x[c] - mx);
            s += o[c];
        }
        for (int c = 0; c < cols; ++c) o[c] /= s;
    }
}

void or_reftest_softmax_inputs(float* out, int64_t n, unsigned seed) {
    srand(seed);
    for (int64_t i = 0; i < n; ++i) out[i] = (float)rand() / RAND_MAX * 4.0f - 2.0f;
}

/* ---- embedding gather -------------------------------------------------------------
 * src/forward.cu:137-141, kernels/fp16_ops.cu:81-89: out[t,:] = table[id,:];
 * ids outside [0, vocab) give a zero row (the build's documented choice).
 * Pinned by: numpy fancy indexing table[ids] (tests/test_oracle.py::test_embed_*). */
void or_embed_f32(const float* table, const int32_t* ids, int n_tokens, int vocab, int dim,
                  float* out) {
    for (int t = 0; t < n_tokens; ++t) {
        const int32_t id = ids[t];
        for (int i = 0; i < dim; ++i)
            out[(size_t)t * dim + i] =
                (id >= 0 && id < vocab) ? table[(size_t)id * dim + i] : 0.0f;
    }
}

void or_embed_f16(const uint16_t* table, const int32_t* ids, int n_tokens, int vocab, int dim,
                  uint16_t* out) {
    for (int t = 0; t < n_tokens; ++t) {
        const int32_t id = ids[t];
        for (int i = 0; i < dim; ++i)
            out[(size_t)t * dim + i] =
                (id >= 0 && id < vocab) ? table[(size_t)id * dim + i] : (uint16_t)0;
    }
}

/* ---- contiguous KV append ----------------------------------------------------------
 * src/kv_cache.cu:44-58 and src/fp16_forward.cu:148-164, for n_tokens
 * consecutive positions: cache[layer][pos + t][h][j] = new[t][h][j] with
 * offset layer*max_seq*kv + (pos+t)*kv + h*d + j.
 * Pinned by: the reference's readback known answer (tests/test_kvcache.cu:47-70:
 * after 16 tokens x 32 layers, layer 0 token 7 reads k[0] = 7.0) and numpy
 * reshape-view assignment cache.reshape(L, S, H, d)[layer, pos:pos+T] = new
 * (tests/test_oracle.py::test_kv_*). */
#define KV_APPEND_BODY                                                                    \
    const size_t kv = (size_t)n_kv_heads * head_dim;                                      \
    (void)n_layers;                                                                       \
    for (int t = 0; t < n_tokens; ++t)                                                    \
        for (size_t i = 0; i < kv; ++i) {                                                 \
            const size_t o = ((size_t)layer * max_seq + (size_t)(pos + t)) * kv + i;     \
            k_cache[o] = k_new[(size_t)t * kv + i];                                       \
            v_cache[o] = v_new[(size_t)t * kv + i];                                       \
        }

void or_kv_append_f32(float* k_cache, float* v_cache, const float* k_new, const float* v_new,
                      int layer, int pos, int n_tokens, int n_kv_heads, int head_dim,
                      int max_seq, int n_layers) {
    KV_APPEND_BODY
}

void or_kv_append_f16(uint16_t* k_cache, uint16_t* v_cache, const uint16_t* k_new,
                      const uint16_t* v_new, int layer, int pos, int n_tokens, int n_kv_heads,
                      int head_dim, int max_seq, int n_layers) {
    KV_APPEND_BODY
}

/* ---- paged KV append -----------------------------------------------------------------
 * Pool layout of src/paged_kvcache.cu:26-46 (block = [n_layers, 16, H_kv, d],
 * include/fp16_types.h:63): element (layer, token t, head h, j) of slot s goes
 * to block s/16, row (layer*16 + s%16).  Negative slots and blocks >= n_blocks
 * are skipped.
 * Pinned by: numpy view assignment pool.reshape(B, L, 16, H, d)[b, layer, o] = new
 * for the fresh-pool LIFO block order 0,1,2,... and a permuted block map
 * (tests/test_oracle.py::test_paged_*). */
void or_paged_kv_append_f16(uint16_t* k_pool, uint16_t* v_pool, const int64_t* block_offset,
                            int n_blocks, const int32_t* slots, const uint16_t* k_new,
                            const uint16_t* v_new, int n_tokens, int layer, int n_layers,
                            int n_kv_heads, int head_dim) {
    const size_t kv = (size_t)n_kv_heads * head_dim;
    (void)n_layers;
    for (int t = 0; t < n_tokens; ++t) {
        const int32_t s = slots[t];
        if (s < 0) continue;
        const int b = s / 16, o = s % 16;
        if (b >= n_blocks) continue;
        const size_t base = (size_t)block_offset[b] + ((size_t)layer * 16 + (size_t)o) * kv;
        for (size_t i = 0; i < kv; ++i) {
            k_pool[base + i] = k_new[(size_t)t * kv + i];
            v_pool[base + i] = v_new[(size_t)t * kv + i];
        }
    }
}

/* ---- attention -----------------------------------------------------------------------
 * kernels/flash_attention.cu:29-182 (fp16 flash attention) and
 * kernels/attention.cu:14-97 / tests/test_attention.cu:22-56 (fp32 SDPA):
 *   s_j  = (q . k_j) * scale, scale = 1/sqrtf(head_dim) (flash_attention.cu:173)
 *   kv head of query head h = h * n_kv_heads / n_heads        (flash_attention.cu:45)
 *   causal: key j is masked when j > the query's position     (flash_attention.cu:106)
 *   out  = sum_j e^(s_j - max) v_j / (sum_j e^(s_j - max) + 1e-8)   (:161)
 * Generalised as the kernels are: the q_len queries are the last q_len
 * positions of a kv_len-long context (query i sits at kv_len - q_len + i), rows
 * are strided.  Dot products, exponentials and sums in double; a query with no
 * visible key gives 0 (0 / 1e-8), as in the reference.
 * Pinned by: closed forms (identical keys -> mean of the visible V rows; causal
 * query 0 -> V[0]; two keys with a known score gap -> the logistic weight;
 * one dominant key -> its V row; the GQA head map via head-distinct V) and the
 * reference's own test (tests/test_attention.cu:77-141: srand(99) U(-0.5,0.5)
 * [128, 32, 128], max abs error < 1e-3 against its fp32 CPU loop, restated as
 * or_attention_reftest_cpu) (tests/test_oracle.py::test_attention_*). */
void or_attention_f32(const float* q, const float* k, const float* v, float* out, int q_len,
                      int kv_len, int n_heads, int n_kv_heads, int head_dim, int64_t q_stride,
                      int64_t kv_stride, int64_t o_stride, int causal) {
    const double scale = (double)(1.0f / sqrtf((float)head_dim));
    double* e = (double*)malloc(sizeof(double) * (size_t)(kv_len > 0 ? kv_len : 1));
    double* acc = (double*)malloc(sizeof(double) * (size_t)head_dim);
    for (int i = 0; i < q_len; ++i) {
        const long pos = (long)kv_len - q_len + i;
        long nk = kv_len;
        if (causal) nk = pos + 1 < kv_len ? pos + 1 : kv_len;
        if (nk < 0) nk = 0;
        for (int h = 0; h < n_heads; ++h) {
            const int kvh = (int)(((long long)h * n_kv_heads) / n_heads);
            const float* qr = q + (size_t)i * q_stride + (size_t)h * head_dim;
            double mx = -DBL_MAX;
            for (long j = 0; j < nk; ++j) {
                const float* kr = k + (size_t)j * kv_stride + (size_t)kvh * head_dim;
                double dot = 0.0;
                for (int d = 0; d < head_dim; ++d) dot += (double)qr[d] * (double)kr[d];
                e[j] = dot * scale;
                if (e[j] > mx) mx = e[j];
            }
            double l = 0.0;
            for (long j = 0; j < nk; ++j) {
                e[j] = exp(e[j] - mx);
                l += e[j];
            }
            for (int d = 0; d < head_dim; ++d) acc[d] = 0.0;
            for (long j = 0; j < nk; ++j) {
                const float* vr = v + (size_t)j * kv_stride + (size_t)kvh * head_dim;
                for (int d = 0; d < head_dim; ++d) acc[d] += e[j] * (double)vr[d];
            }
            float* orow = out + (size_t)i * o_stride + (size_t)h * head_dim;
            for (int d = 0; d < head_dim; ++d) orow[d] = (float)(acc[d] / (l + 1e-8));
        }
    }
    free(e);
    free(acc);
}

static float* widen_rows(const uint16_t* src, int rows, int64_t stride, int width) {
    float* f = (float*)malloc(sizeof(float) * ((size_t)(rows > 0 ? rows : 1) * (size_t)stride));
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < width; ++c)
            f[(size_t)r * stride + c] = or_f16_to_f32(src[(size_t)r * stride + c]);
    return f;
}

/* fp16 inputs widened exactly, the same double computation, then the fp32
 * result rounded to binary16 (RNE). */
void or_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                      int q_len, int kv_len, int n_heads, int n_kv_heads, int head_dim,
                      int64_t q_stride, int64_t kv_stride, int64_t o_stride, int causal) {
    float* qf = widen_rows(q, q_len, q_stride, n_heads * head_dim);
    float* kf = widen_rows(k, kv_len, kv_stride, n_kv_heads * head_dim);
    float* vf = widen_rows(v, kv_len, kv_stride, n_kv_heads * head_dim);
    float* of = (float*)malloc(sizeof(float) * ((size_t)(q_len > 0 ? q_len : 1) * (size_t)o_stride));
    or_attention_f32(qf, kf, vf, of, q_len, kv_len, n_heads, n_kv_heads, head_dim, q_stride,
                     kv_stride, o_stride, causal);
    for (int r = 0; r < q_len; ++r)
        for (int c = 0; c < n_heads * head_dim; ++c)
            out[(size_t)r * o_stride + c] = or_f32_to_f16(of[(size_t)r * o_stride + c]);
    free(qf);
    free(kf);
    free(vf);
    free(of);
}

/* The reference test's own CPU loop (tests/test_attention.cu:22-56): fp32
 * sequential dot products and sums, no causal mask, n_heads K/V heads. */
void or_attention_reftest_cpu(const float* Q, const float* K, const float* V, float* out,
                              int seq_len, int n_heads, int head_dim) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    float* sc = (float*)malloc(sizeof(float) * (size_t)seq_len);
    const size_t rs = (size_t)n_heads * head_dim;
    for (int i = 0; i < seq_len; ++i)
        for (int h = 0; h < n_heads; ++h) {
            float mx = -FLT_MAX;
            for (int j = 0; j < seq_len; ++j) {
                float dot = 0.0f;
                for (int d = 0; d < head_dim; ++d)
                    dot += Q[i * rs + (size_t)h * head_dim + d] * K[j * rs + (size_t)h * head_dim + d];
                sc[j] = dot * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            float s = 0.0f;
            for (int j = 0; j < seq_len; ++j) {
                sc[j] = expf(sc[j] - mx);
                s += sc[j];
            }
            for (int j = 0; j < seq_len; ++j) sc[j] /= s;
            for (int d = 0; d < head_dim; ++d) {
                float a = 0.0f;
                for (int j = 0; j < seq_len; ++j) a += sc[j] * V[j * rs + (size_t)h * head_dim + d];
                out[i * rs + (size_t)h * head_dim + d] = a;
            }
        }
    free(sc);
}

/* Inputs of tests/test_attention.cu:77-82: srand(seed); per element i, in this
 * order, Q[i], K[i], V[i] = rand()/RAND_MAX - 0.5. */
void or_reftest_attention_inputs(float* q, float* k, float* v, int64_t n, unsigned seed) {
    srand(seed);
    for (int64_t i = 0; i < n; ++i) {
        q[i] = (float)rand() / RAND_MAX - 0.5f;
        k[i] = (float)rand() / RAND_MAX - 0.5f;
        v[i] = (float)rand() / RAND_MAX - 0.5f;
    }
}

/* ---- linear layer and greedy sampling ---------------------------------------------------
 * y[m, n] = sum_k x[m, k] w[n, k] (weights [out, in], y = x W^T), the projections of
 * src/fp16_forward.cu:184-186,204,211,219-221 (hgemm with fp32 accumulation);
 * products and sum in double, result rounded to binary16.
 * Pinned by: numpy float64 matmul of the widened values; identity and permutation
 * weights reproduce / permute x exactly (tests/test_oracle.py::test_matmul_*). */
void or_matmul_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, int M, int N, int K) {
    float* wf = (float*)malloc(sizeof(float) * (size_t)N * (size_t)K);
    for (size_t i = 0; i < (size_t)N * (size_t)K; ++i) wf[i] = or_f16_to_f32(w[i]);
    double* xr = (double*)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
    for (int m = 0; m < M; ++m) {
        for (int k = 0; k < K; ++k) xr[k] = or_f16_to_f32(x[(size_t)m * K + k]);
        for (int n = 0; n < N; ++n) {
            const float* wr = wf + (size_t)n * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += xr[k] * (double)wr[k];
            y[(size_t)m * N + n] = or_f32_to_f16((float)acc);
        }
    }
    free(wf);
    free(xr);
}

/* argmax_kernel (src/continuous_batch.cu:12-25): the first index whose value is
 * strictly greater than all earlier ones and than the start value -1e20f (:15);
 * NaN never is; a row without a value above -1e20f gives 0.
 * Pinned by: numpy argmax (first occurrence) on NaN-free rows; ties, all -inf,
 * NaN rows and rows at or below -1e20 by closed forms
 * (tests/test_oracle.py::test_argmax_*). */
void or_argmax_f32(const float* x, int rows, int cols, int32_t* out) {
    for (int r = 0; r < rows; ++r) {
        float best = -1e20f;
        int32_t idx = 0;
        for (int c = 0; c < cols; ++c) {
            const float v = x[(size_t)r * cols + c];
            if (v > best) {
                best = v;
                idx = c;
            }
        }
        out[r] = idx;
    }
}

/* ---- FP8 weight codec (quantlib) ----------------------------------------------------
 * Two modes.
 * REFERENCE (quantlib_src/include/quant_types.h:47-84, kernels/fp8_convert.cu:15-89):
 *   scale  = fmax / m, m = max |x| over the elements the reference's reduction sees
 *            (128 threads stride the group, only warp 0's lanes are reduced: the
 *            elements whose offset within the group is < 32 mod 128); m < 1e-8 -> 1;
 *   encode = clamp to +-fmax, rebias the exponent, TRUNCATE the mantissa, exponent
 *            <= 0 -> signed zero, above the top -> top code;
 *   decode = (1 + m/2^M) * 2^(e - bias), code with e = m = 0 -> +0;
 *   dequant = decode(q) / scale, rounded to binary16.
 * OCP (E4M3FN / E5M2 of the OCP 8-bit floating point spec): scale from the max over
 *   the whole group; encode = round to nearest even with subnormals, saturating to
 *   +-fmax (NaN stays NaN); decode per the spec.
 * fmax = 448 (E4M3) or 57344 (E5M2).  Groups are runs of group_size elements of
 * the row-major matrix (per-tensor: rows*cols, per-channel: cols).
 * Pinned by: exhaustive code tables against the formats' closed forms, round trips
 * of every code, brute-force nearest-value search for the OCP encoder, the
 * reference's own truncation examples, and the reference test's max abs error
 * bar (tests/test_oracle.py::test_fp8_*). */
static float fp8_fmax(int fmt) { return fmt == 0 ? 448.0f : 57344.0f; }

uint8_t or_fp8_encode_ref(float v, int fmt) {
    const float fm = fp8_fmax(fmt);
    v = v > fm ? fm : (v < -fm ? -fm : v);
    uint32_t bits;
    memcpy(&bits, &v, 4);
    const uint8_t sign = (uint8_t)((bits >> 31) & 1);
    const int mbits = fmt == 0 ? 3 : 2, bias = fmt == 0 ? 7 : 15, emax = fmt == 0 ? 15 : 31;
    int e = (int)((bits >> 23) & 0xFF) - 127 + bias;
    uint8_t m = (uint8_t)((bits >> (23 - mbits)) & ((1u << mbits) - 1));
    if (e <= 0) return (uint8_t)(sign << 7);
    if (e > emax) {
        e = emax;
        m = (uint8_t)((1u << mbits) - 1);
    }
    return (uint8_t)((sign << 7) | (e << mbits) | m);
}

float or_fp8_decode_ref(uint8_t q, int fmt) {
    const int mbits = fmt == 0 ? 3 : 2, bias = fmt == 0 ? 7 : 15;
    const int e = (q >> mbits) & (fmt == 0 ? 0xF : 0x1F);
    const int m = q & ((1 << mbits) - 1);
    if (e == 0 && m == 0) return 0.0f;
    const float r = ldexpf(1.0f + (float)m / (float)(1 << mbits), e - bias);
    return (q >> 7) ? -r : r;
}

float or_fp8_decode_ocp(uint8_t q, int fmt) {
    const int mbits = fmt == 0 ? 3 : 2, bias = fmt == 0 ? 7 : 15;
    const int emask = fmt == 0 ? 0xF : 0x1F;
    const int e = (q >> mbits) & emask, m = q & ((1 << mbits) - 1);
    const int s = q >> 7;
    float r;
    if (fmt == 0 && e == 0xF && m == 7) return NAN;                 /* E4M3FN: only NaN */
    if (fmt == 1 && e == 0x1F) r = m ? NAN : INFINITY;               /* E5M2: IEEE-like */
    else if (e == 0) r = ldexpf((float)m / (float)(1 << mbits), 1 - bias);
    else r = ldexpf(1.0f + (float)m / (float)(1 << mbits), e - bias);
    return s ? -r : r;
}

/* Round to nearest even onto the format grid, saturating at +-fmax. */
uint8_t or_fp8_encode_ocp(float v, int fmt) {
    const int mbits = fmt == 0 ? 3 : 2, bias = fmt == 0 ? 7 : 15;
    if (isnan(v)) return fmt == 0 ? 0x7F : 0x7E;
    const uint8_t sign = signbit(v) ? 0x80 : 0;
    double a = fabs((double)v);
    const double fm = fp8_fmax(fmt);
    if (a >= fm) return (uint8_t)(sign | (fmt == 0 ? 0x7E : 0x7B));
    /* quantum at a's binade (subnormal quantum below the first normal binade) */
    int ex;
    frexp(a, &ex);                     /* a = f * 2^ex, f in [0.5, 1) */
    int e_unb = ex - 1;                /* a in [2^e_unb, 2^(e_unb+1)) */
    if (e_unb < 1 - bias) e_unb = 1 - bias;
    const double quantum = ldexp(1.0, e_unb - mbits);
    double n = a / quantum;            /* exact: power-of-two quantum */
    double fl = floor(n);
    double r = n - fl;
    if (r > 0.5 || (r == 0.5 && fmod(fl, 2.0) != 0.0)) fl += 1.0;
    const double val = fl * quantum;
    if (val >= fm) return (uint8_t)(sign | (fmt == 0 ? 0x7E : 0x7B));
    if (val == 0.0) return sign;
    /* encode val */
    int ev;
    frexp(val, &ev);
    int e = ev - 1 + bias;
    int m;
    if (e <= 0) {
        e = 0;
        m = (int)(val / ldexp(1.0, 1 - bias - mbits));
    } else {
        m = (int)((val / ldexp(1.0, ev - 1) - 1.0) * (1 << mbits));
    }
    return (uint8_t)(sign | (e << mbits) | m);
}

int or_fp8_num_scales(int rows, int cols, int gran, int group_size) {
    const long long n = (long long)rows * cols;
    if (gran == 0) return 1;
    if (gran == 1) return rows;
    return (int)((n + group_size - 1) / group_size);
}

static long long fp8_group(int rows, int cols, int gran, int group_size) {
    return gran == 0 ? (long long)rows * cols : (gran == 1 ? cols : group_size);
}

void or_fp8_scales(const uint16_t* src, int rows, int cols, int fmt, int gran, int group_size,
                   int mode, float* scales) {
    const long long n = (long long)rows * cols, gs = fp8_group(rows, cols, gran, group_size);
    const int ns = or_fp8_num_scales(rows, cols, gran, group_size);
    for (int g = 0; g < ns; ++g) {
        float mx = 0.0f;
        for (long long i = 0; i < gs && g * gs + i < n; ++i) {
            if (mode == 0 && (i % 128) >= 32) continue;   /* lanes the reference reduces */
            const float a = fabsf(or_f16_to_f32(src[g * gs + i]));
            mx = fmaxf(mx, a);
        }
        scales[g] = mx < 1e-8f ? 1.0f : fp8_fmax(fmt) / mx;
    }
}

void or_fp8_quantize(const uint16_t* src, int rows, int cols, int fmt, int gran, int group_size,
                     int mode, uint8_t* dst, float* scales) {
    or_fp8_scales(src, rows, cols, fmt, gran, group_size, mode, scales);
    const long long n = (long long)rows * cols, gs = fp8_group(rows, cols, gran, group_size);
    for (long long i = 0; i < n; ++i) {
        const float v = or_f16_to_f32(src[i]) * scales[i / gs];
        dst[i] = mode == 0 ? or_fp8_encode_ref(v, fmt) : or_fp8_encode_ocp(v, fmt);
    }
}

void or_fp8_dequantize(const uint8_t* src, const float* scales, int rows, int cols, int fmt,
                       int gran, int group_size, int mode, uint16_t* dst) {
    const long long n = (long long)rows * cols, gs = fp8_group(rows, cols, gran, group_size);
    for (long long i = 0; i < n; ++i) {
        const float d = mode == 0 ? or_fp8_decode_ref(src[i], fmt) : or_fp8_decode_ocp(src[i], fmt);
        dst[i] = or_f32_to_f16(d / scales[i / gs]);
    }
}

/* Inputs of quantlib_src/tests/test_fp8.cu:27-29 (glibc rand, default seed 1):
 * x = ((float)rand() / RAND_MAX) * 2 - 1. */
void or_reftest_fp8_inputs(float* out, int64_t n, unsigned seed) {
    srand(seed);
    for (int64_t i = 0; i < n; ++i) out[i] = ((float)rand() / RAND_MAX) * 2.0f - 1.0f;
}

/* Inputs of quantlib_src/tests/test_gemm.cu:38-52 (srand(seed), then A [M x K] and
 * W [N x K] in that order): v = ((float)rand() / RAND_MAX) * 0.2f - 0.1f, in fp32
 * (the caller rounds them to binary16, as __float2half does).
 * Pinned by: glibc rand() called through ctypes (tests/test_oracle.py). */
void or_reftest_gemm_inputs(float* a, int64_t na, float* w, int64_t nw, unsigned seed) {
    srand(seed);
    for (int64_t i = 0; i < na; ++i) a[i] = ((float)rand() / RAND_MAX) * 0.2f - 0.1f;
    for (int64_t i = 0; i < nw; ++i) w[i] = ((float)rand() / RAND_MAX) * 0.2f - 0.1f;
}

/* The CPU check of quantlib_src/tests/test_gemm.cu:17-27: C[m, n] = sum over k in
 * order of f(A[m, k]) * f(W[n, k]), fp32 products and sums (f = binary16 -> fp32).
 * Pinned by: numpy float64 matmul within the fp32 sum's rounding bound, and exact
 * small-integer cases (tests/test_oracle.py). */
void or_gemm_reftest_cpu(const uint16_t* a, const uint16_t* w, float* c, int M, int N, int K) {
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float s = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float p = or_f16_to_f32(a[(size_t)m * K + k]) * or_f16_to_f32(w[(size_t)n * K + k]);
                s = s + p;
            }
            c[(size_t)m * N + n] = s;
        }
}

/* Not a restatement of the reference: an exhaustive check of the division the
 * GPU dequantizer uses in place of fp32 division (decoded FP8 value d over the
 * group's scale s): r = RN(1/s) once per group, then per element q0 = RN(d*r),
 * e = RN(d - s*q0) (one fma, exact), q = RN(q0 + e*r) (one fma).  Returns how many
 * (s, d) pairs give q != RN(d/s) over every fp32 s in [1, 2) and every d = +-(1 +
 * m/16), m = 0..15 (every FP8 mantissa).  In the normal range every step scales
 * exactly with s and d by powers of two, so this binade covers all normal cases. */
long long or_check_recip_division(void) {
    long long bad = 0;
    for (uint32_t bits = 0x3f800000u; bits < 0x40000000u; ++bits) {
        float s;
        memcpy(&s, &bits, 4);
        const float r = 1.0f / s;
        for (int m = 0; m < 16; ++m)
            for (int sg = -1; sg <= 1; sg += 2) {
                const float d = (float)sg * (1.0f + (float)m / 16.0f);
                const float q0 = d * r;
                const float e = fmaf(-q0, s, d);
                const float q = fmaf(e, r, q0);
                if (q != d / s) ++bad;
            }
    }
    return bad;
}
