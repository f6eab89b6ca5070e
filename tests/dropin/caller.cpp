// A caller written the way the reference's host code calls its kernels
// (src/forward.cu, src/fp16_forward.cu, src/kv_cache.cu, src/paged_kvcache.cu,
// quantlib_src/include/quantlib.h): it includes quantlib_compat.h instead of the
// reference's prototypes and headers, links libquantlib_amd.so, and checks each
// call against a closed-form result at toy sizes.  Exit status 0 = every check
// passed.  Built by tests/dropin/Makefile; run by tests/test_gpu_compat.py.
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <vector>

#include "quantlib_compat.h"

static int g_fail = 0;

#define HIP_OK(x)                                                                    \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            return 2;                                                                \
        }                                                                            \
    } while (0)

static void expect(bool ok, const char* what) {
    if (!ok) {
        fprintf(stderr, "FAILED: %s\n", what);
        ++g_fail;
    }
}

template <typename T>
static T* upload(const std::vector<T>& h) {
    T* d = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&d), h.size() * sizeof(T)) != hipSuccess) return nullptr;
    if (hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
    return d;
}

template <typename T>
static std::vector<T> download(const T* d, size_t n) {
    std::vector<T> h(n);
    if (hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess) h.clear();
    return h;
}

int main() {
    hipStream_t stream;
    HIP_OK(hipStreamCreate(&stream));
    const int hd = 64, vocab = 4;

    // src/forward.cu:256-257 (embed) -> 133 (add_residual) -> rmsnorm
    std::vector<float> tbl(vocab * hd);
    for (int r = 0; r < vocab; ++r)
        for (int i = 0; i < hd; ++i) tbl[r * hd + i] = (float)r + 0.5f;
    float* d_tbl = upload(tbl);
    float* d_x = upload(std::vector<float>(hd, 0.0f));
    float* d_d = upload(std::vector<float>(hd, 0.5f));
    float* d_w = upload(std::vector<float>(hd, 1.0f));
    float* d_y = upload(std::vector<float>(hd, 0.0f));
    launch_embed(d_x, d_tbl, 2, hd, stream);            // x = 2.5
    add_residual(d_x, d_d, hd, stream);                 // x = 3.0
    launch_rmsnorm(d_x, d_w, d_y, 1, hd, 1e-5f, stream);
    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipGetLastError());
    {
        const auto x = download(d_x, hd), y = download(d_y, hd);
        expect(x[0] == 3.0f && x[hd - 1] == 3.0f, "launch_embed + add_residual");
        const float want = 3.0f / sqrtf(9.0f + 1e-5f);
        expect(fabsf(y[7] - want) <= 1e-6f, "launch_rmsnorm");
    }

    // kernels/rope.cu:44: row 0 (position 0) unchanged, every pair's norm kept
    {
        const int seq = 2, heads = 2, d = 64;
        std::vector<float> q(seq * heads * d);
        for (size_t i = 0; i < q.size(); ++i) q[i] = (float)((i * 37) % 11) - 5.0f;
        float* d_q = upload(q);
        launch_rope(d_q, seq, heads, d, 10000.0f, stream);
        HIP_OK(hipStreamSynchronize(stream));
        const auto r = download(d_q, q.size());
        bool ok = memcmp(r.data(), q.data(), heads * d * sizeof(float)) == 0;
        for (int i = heads * d; i < seq * heads * d; i += 2) {
            const float n0 = q[i] * q[i] + q[i + 1] * q[i + 1], n1 = r[i] * r[i] + r[i + 1] * r[i + 1];
            ok = ok && fabsf(n0 - n1) <= 1e-4f * (1.0f + n0);
        }
        expect(ok, "launch_rope");
        (void)hipFree(d_q);
    }

    // kernels/feedforward.cu:27: silu(1) * 2, silu(0) * 5 = 0
    {
        float* d_g = upload(std::vector<float>{1.0f, 0.0f});
        float* d_u = upload(std::vector<float>{2.0f, 5.0f});
        float* d_o = upload(std::vector<float>{-1.0f, -1.0f});
        launch_swiglu(d_g, d_u, d_o, 1, 2, stream);
        HIP_OK(hipStreamSynchronize(stream));
        const auto o = download(d_o, 2);
        const float want = 2.0f / (1.0f + expf(-1.0f));
        expect(fabsf(o[0] - want) <= 1e-5f * want && o[1] == 0.0f, "launch_swiglu");
        (void)hipFree(d_g);
        (void)hipFree(d_u);
        (void)hipFree(d_o);
    }

    // kernels/softmax.cu:88: equal logits give 1/cols
    {
        float* d_in = upload(std::vector<float>(8, 3.0f));
        float* d_out = upload(std::vector<float>(8, 0.0f));
        launch_softmax(d_in, d_out, 2, 4, stream);
        HIP_OK(hipStreamSynchronize(stream));
        const auto o = download(d_out, 8);
        bool ok = true;
        for (float v : o) ok = ok && fabsf(v - 0.25f) <= 1e-7f;
        expect(ok, "launch_softmax");
        (void)hipFree(d_in);
        (void)hipFree(d_out);
    }

    // src/forward.cu:262-264: kvcache_append at current_len, the caller advances it
    {
        const int L = 2, S = 8, H = 2, d = 4;
        KVCache* c = kvcache_create(L, S, H, d);
        expect(c && c->current_len == 0 && c->max_seq_len == S, "kvcache_create");
        if (c) {
            for (int t = 0; t < 3; ++t) {
                float* k = upload(std::vector<float>(H * d, (float)t + 1.0f));
                float* v = upload(std::vector<float>(H * d, -(float)t - 1.0f));
                kvcache_append(c, 1, k, v, stream);
                HIP_OK(hipStreamSynchronize(stream));
                c->current_len += 1;
                (void)hipFree(k);
                (void)hipFree(v);
            }
            const auto k1 = download(kvcache_get_k(c, 1), S * H * d);
            const auto v1 = download(kvcache_get_v(c, 1), S * H * d);
            const auto k0 = download(kvcache_get_k(c, 0), S * H * d);
            expect(k1[2 * H * d] == 3.0f && v1[H * d] == -2.0f && k1[3 * H * d] == 0.0f && k0[0] == 0.0f,
                   "kvcache_append / kvcache_get_k / kvcache_get_v");
            kvcache_free(c);
        }
    }

    // fp16 layer pieces (src/fp16_forward.cu): conversions, cache append at pos
    {
        float* d_f = upload(std::vector<float>{1.5f, -2.25f, 65504.0f, 1e-8f});
        __half* d_h = nullptr;
        float* d_back = upload(std::vector<float>(4, 0.0f));
        HIP_OK(hipMalloc(reinterpret_cast<void**>(&d_h), 4 * sizeof(__half)));
        launch_fp32_to_fp16(d_f, d_h, 4, stream);
        launch_fp16_to_fp32(d_h, d_back, 4, stream);
        HIP_OK(hipStreamSynchronize(stream));
        const auto b = download(d_back, 4);
        expect(b[0] == 1.5f && b[1] == -2.25f && b[2] == 65504.0f && b[3] == 0.0f,
               "launch_fp32_to_fp16 / launch_fp16_to_fp32");
        FP16KVCache* c = fp16_kvcache_create(2, 8, 2, 64);
        expect(c != nullptr, "fp16_kvcache_create");
        if (c) {
            __half* kn = nullptr;
            HIP_OK(hipMalloc(reinterpret_cast<void**>(&kn), 128 * sizeof(__half)));
            launch_fp32_to_fp16(upload(std::vector<float>(128, 0.75f)), kn, 128, stream);
            launch_fp16_kvcache_append(c->k_cache, c->v_cache, kn, kn, 1, 5, 2, 64, 8, 2, stream);
            float* d_row = upload(std::vector<float>(128, 0.0f));
            launch_fp16_to_fp32(c->k_cache + (size_t)(1 * 8 + 5) * 128, d_row, 128, stream);
            HIP_OK(hipStreamSynchronize(stream));
            const auto row = download(d_row, 128);
            expect(row[0] == 0.75f && row[127] == 0.75f, "launch_fp16_kvcache_append");
            fp16_kvcache_free(c);
        }
    }

    // src/paged_kvcache.cu:49-53,89-93: a fresh pool hands out 0, 1, 2, ...; LIFO reuse
    {
        PagedKVCache* p = paged_kv_create(4, 2, 2, 64, 2, 4);
        expect(p != nullptr, "paged_kv_create");
        if (p) {
            const int b0 = paged_kv_allocate_block(p), b1 = paged_kv_allocate_block(p);
            paged_kv_free_block(p, b0);
            const int b2 = paged_kv_allocate_block(p);
            expect(b0 == 0 && b1 == 1 && b2 == 0, "paged_kv_allocate_block / paged_kv_free_block");
            paged_kv_free(p);
        }
    }

    // kernels/flash_attention.cu:169: causal, query 0 sees only key 0, so O[0] = V[0]
    // (head_dim 64, the reference's tile width, and 32, which its tiles also take)
    for (const int d : {64, 32}) {
        const int seq = 2;
        std::vector<float> qf(seq * d), kf(seq * d), vf(seq * d);
        for (int i = 0; i < seq * d; ++i) {
            qf[i] = 0.01f * (float)(i % 7);
            kf[i] = 0.02f * (float)(i % 5);
            vf[i] = 0.125f * (float)(i % 9);
        }
        __half *q, *k, *v, *o;
        HIP_OK(hipMalloc(reinterpret_cast<void**>(&q), seq * d * sizeof(__half)));
        HIP_OK(hipMalloc(reinterpret_cast<void**>(&k), seq * d * sizeof(__half)));
        HIP_OK(hipMalloc(reinterpret_cast<void**>(&v), seq * d * sizeof(__half)));
        HIP_OK(hipMalloc(reinterpret_cast<void**>(&o), seq * d * sizeof(__half)));
        launch_fp32_to_fp16(upload(qf), q, seq * d, stream);
        launch_fp32_to_fp16(upload(kf), k, seq * d, stream);
        launch_fp32_to_fp16(upload(vf), v, seq * d, stream);
        launch_flash_attention(q, k, v, o, seq, 1, 1, d, 1, stream);
        float* d_o = upload(std::vector<float>(seq * d, 0.0f));
        launch_fp16_to_fp32(o, d_o, seq * d, stream);
        HIP_OK(hipStreamSynchronize(stream));
        HIP_OK(hipGetLastError());
        const auto of = download(d_o, seq * d);
        bool ok = true;
        for (int i = 0; i < d; ++i) ok = ok && of[i] == vf[i];
        expect(ok, "launch_flash_attention");
    }

    // src/fp16_forward.cu:285-297: greedy sample of fp32 logits peaking at index 777
    {
        const int vocab = 32000;
        std::vector<float> lg(vocab);
        for (int i = 0; i < vocab; ++i) lg[i] = -0.001f * (float)((i - 777) * (i - 777));
        const int tok = fp16_greedy_sample(upload(lg), vocab, stream);
        expect(tok == 777, "fp16_greedy_sample");
    }

    // quantlib_src/include/quantlib.h:10-21: E4M3 per-channel round trip of exact values
    {
        const int rows = 2, cols = 64;
        std::vector<float> w(rows * cols);
        for (int i = 0; i < rows * cols; ++i) w[i] = (i % 2 ? -1.0f : 1.0f) * (float)(1 + i % 4);
        __half* dw = nullptr;
        __half* back = nullptr;
        HIP_OK(hipMalloc(reinterpret_cast<void**>(&dw), rows * cols * sizeof(__half)));
        HIP_OK(hipMalloc(reinterpret_cast<void**>(&back), rows * cols * sizeof(__half)));
        launch_fp32_to_fp16(upload(w), dw, rows * cols, stream);
        QuantMatrix qm = quantlib_fp16_to_fp8_e4m3(dw, rows, cols, QUANT_PER_CHANNEL, 0, stream);
        quantlib_fp8_to_fp16(&qm, back, stream);
        float* d_b = upload(std::vector<float>(rows * cols, 0.0f));
        launch_fp16_to_fp32(back, d_b, rows * cols, stream);
        HIP_OK(hipStreamSynchronize(stream));
        const auto b = download(d_b, rows * cols);
        bool ok = qm.rows == rows && qm.cols == cols && strcmp(qm.format, "E4M3") == 0;
        // the reference encoder truncates: at most one code step (1/8 relative) lost
        for (int i = 0; i < rows * cols; ++i) ok = ok && fabsf(b[i] - w[i]) <= 0.125f * fabsf(w[i]);
        expect(ok, "quantlib_fp16_to_fp8_e4m3 / quantlib_fp8_to_fp16");
        quantlib_free(&qm);
    }

    HIP_OK(hipStreamSynchronize(stream));
    HIP_OK(hipStreamDestroy(stream));
    if (g_fail) {
        fprintf(stderr, "dropin caller: %d check(s) failed\n", g_fail);
        return 1;
    }
    printf("dropin caller: ok\n");
    return 0;
}
