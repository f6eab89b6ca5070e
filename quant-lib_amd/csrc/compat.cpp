// compat.cpp -- the reference's launcher names and KV-cache host API on top of
// the ql_* C ABI (declarations and behaviour notes in quantlib_compat.h).
//
// Host code only: it validates nothing beyond what the ql_* calls check and,
// like the reference, only the quantlib helpers that copy to the host (or grow
// the FP8 GEMM's dequantization buffer) synchronise.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <string.h>

#include <map>
#include <cstdlib>
#include <memory>
#include <mutex>
#include <utility>

#include <hip/hip_runtime_api.h>

#include "quantlib_amd.h"
#include "quantlib_compat.h"

namespace {

uint16_t* bits(__half* p) { return reinterpret_cast<uint16_t*>(p); }
const uint16_t* bits(const __half* p) { return reinterpret_cast<const uint16_t*>(p); }

// IEEE binary16 -> float (exact)
float half_to_float(uint16_t h) {
    const int e = (h >> 10) & 0x1F, m = h & 0x3FF;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 0x400), e - 25);
    return (h & 0x8000) ? -v : v;
}

}  // namespace

// kernels/rmsnorm.cu:51-57
void launch_rmsnorm(const float* x, const float* weight, float* out, int rows, int dim,
                    float eps, hipStream_t stream) {
    (void)ql_rmsnorm_f32(x, weight, out, rows, dim, eps, stream);
}

// kernels/rope.cu:44-50 -- interleaved pairs, position = row index.
void launch_rope(float* x, int seq_len, int n_heads, int head_dim, float theta,
                 hipStream_t stream) {
    (void)ql_rope_f32(x, nullptr, seq_len, n_heads, 0, head_dim, (int64_t)n_heads * head_dim, 0,
                      nullptr, 0, theta, QL_ROPE_INTERLEAVED, stream);
}

// kernels/feedforward.cu:27-35
void launch_swiglu(const float* gate, const float* up, float* out, int rows, int ffn_dim,
                   hipStream_t stream) {
    (void)ql_swiglu_f32(gate, up, out, rows, ffn_dim, stream);
}

// kernels/softmax.cu:88-94
void launch_softmax(const float* input, float* output, int rows, int cols, hipStream_t stream) {
    (void)ql_softmax_f32(input, output, rows, cols, stream);
}

// kernels/fp16_ops.cu:113-118
void launch_fp16_rmsnorm(const __half* x, const __half* w, __half* out, int rows, int dim,
                         float eps, hipStream_t stream) {
    (void)ql_rmsnorm_f16(bits(x), bits(w), bits(out), rows, dim, eps, stream);
}

// kernels/fp16_ops.cu:120-127
void launch_fp16_rope(__half* x, int seq_len, int n_heads, int head_dim, float theta,
                      hipStream_t stream) {
    (void)ql_rope_f16(bits(x), nullptr, seq_len, n_heads, 0, head_dim,
                      (int64_t)n_heads * head_dim, 0, nullptr, 0, theta, QL_ROPE_INTERLEAVED,
                      stream);
}

// kernels/fp16_ops.cu:129-135
void launch_fp16_swiglu(const __half* gate, const __half* up, __half* out, int rows,
                        int ffn_dim, hipStream_t stream) {
    (void)ql_swiglu_f16(bits(gate), bits(up), bits(out), rows, ffn_dim, stream);
}

// kernels/fp16_ops.cu:137-142
void launch_fp16_embed(const __half* table, __half* out, int token_id, int hidden_dim,
                       hipStream_t stream) {
    (void)ql_embed_token_f16(bits(table), token_id, hidden_dim, bits(out), stream);
}

// kernels/fp16_ops.cu:144-147
void launch_fp16_add(__half* x, const __half* y, int n, hipStream_t stream) {
    (void)ql_add_f16(bits(x), bits(y), n, stream);
}

// kernels/fp16_ops.cu:149-153
void launch_fp16_to_fp32(const __half* src, float* dst, int n, hipStream_t stream) {
    (void)ql_f16_to_f32(bits(src), dst, n, stream);
}

// src/quant_forward.cu:18-21
void launch_fp32_to_fp16(const float* src, __half* dst, int n, hipStream_t stream) {
    (void)ql_f32_to_f16(src, bits(dst), n, stream);
}

// kernels/flash_attention.cu:169-182
void launch_flash_attention(const __half* Q, const __half* K, const __half* V, __half* Out,
                            int seq_len, int n_heads, int n_kv_heads, int head_dim, int causal,
                            hipStream_t stream) {
    (void)ql_flash_attention_f16(bits(Q), bits(K), bits(V), bits(Out), seq_len, n_heads,
                                 n_kv_heads, head_dim, causal, stream);
}

// src/fp16_forward.cu:285-297 (argmax_kernel :259-283 on one block, then a
// synchronous copy of the index).  The reference's block reduction merges warp
// maxima with atomicMax on the float bits read as int, which orders negative
// maxima backwards and lets tied warps race; ql_argmax_f32 returns the first
// index of the true maximum.
int fp16_greedy_sample(const float* logits, int vocab_size, hipStream_t stream) {
    if (vocab_size <= 0) return 0;
    int32_t* d_out = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&d_out), sizeof(int32_t)) != hipSuccess) return -1;
    int32_t result = -1;
    hipError_t e = ql_argmax_f32(logits, 1, vocab_size, vocab_size, d_out, stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(&result, d_out, sizeof(result), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    (void)hipFree(d_out);
    return e == hipSuccess ? (int)result : -1;
}

// src/forward.cu:128-135
void add_residual(float* x, const float* d, int n, hipStream_t stream) {
    (void)ql_add_f32(x, d, n, stream);
}

// src/forward.cu:137-141, launched at :256-257
void launch_embed(float* out, const float* tbl, int tok, int hd, hipStream_t stream) {
    (void)ql_embed_token_f32(tbl, tok, hd, out, stream);
}

// src/fp16_forward.cu:148-164, launched at :194-199
void launch_fp16_kvcache_append(__half* k_cache, __half* v_cache, const __half* k_new,
                                const __half* v_new, int layer, int pos, int n_kv_heads,
                                int head_dim, int max_seq, int n_layers, hipStream_t stream) {
    (void)ql_kv_append_f16(bits(k_cache), bits(v_cache), bits(k_new), bits(v_new), layer, pos, 1,
                           n_kv_heads, head_dim, max_seq, n_layers, stream);
}

// ---- fp32 contiguous KV cache: src/kv_cache.cu:15-70 ----------------------------
// The reference exits the process on a failed allocation; this returns NULL.
KVCache* kvcache_create(int n_layers, int max_seq_len, int n_heads, int head_dim) {
    if (n_layers <= 0 || max_seq_len <= 0 || n_heads <= 0 || head_dim <= 0) return nullptr;
    KVCache* c = static_cast<KVCache*>(malloc(sizeof(KVCache)));
    if (!c) return nullptr;
    c->n_layers = n_layers;
    c->max_seq_len = max_seq_len;
    c->n_heads = n_heads;
    c->head_dim = head_dim;
    c->current_len = 0;
    c->k_cache = nullptr;
    c->v_cache = nullptr;
    const size_t bytes = (size_t)n_layers * max_seq_len * n_heads * head_dim * sizeof(float);
    if (hipMalloc(reinterpret_cast<void**>(&c->k_cache), bytes) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&c->v_cache), bytes) != hipSuccess ||
        hipMemset(c->k_cache, 0, bytes) != hipSuccess ||
        hipMemset(c->v_cache, 0, bytes) != hipSuccess) {
        kvcache_free(c);
        return nullptr;
    }
    return c;
}

void kvcache_free(KVCache* cache) {
    if (!cache) return;
    if (cache->k_cache) (void)hipFree(cache->k_cache);
    if (cache->v_cache) (void)hipFree(cache->v_cache);
    free(cache);
}

// Writes one layer's K,V slice at position current_len (src/kv_cache.cu:44-58),
// one kernel launch instead of two device-to-device copies.
void kvcache_append(KVCache* cache, int layer, const float* new_k, const float* new_v,
                    hipStream_t stream) {
    (void)ql_kv_append_f32(cache->k_cache, cache->v_cache, new_k, new_v, layer,
                           cache->current_len, 1, cache->n_heads, cache->head_dim,
                           cache->max_seq_len, cache->n_layers, stream);
}

float* kvcache_get_k(KVCache* cache, int layer) {
    const size_t stride = (size_t)cache->max_seq_len * cache->n_heads * cache->head_dim;
    return cache->k_cache + (size_t)layer * stride;
}

float* kvcache_get_v(KVCache* cache, int layer) {
    const size_t stride = (size_t)cache->max_seq_len * cache->n_heads * cache->head_dim;
    return cache->v_cache + (size_t)layer * stride;
}

// ---- fp16 contiguous KV cache: src/fp16_forward.cu:122-145 -----------------------
FP16KVCache* fp16_kvcache_create(int n_layers, int max_seq, int n_kv_heads, int head_dim) {
    if (n_layers <= 0 || max_seq <= 0 || n_kv_heads <= 0 || head_dim <= 0) return nullptr;
    FP16KVCache* c = static_cast<FP16KVCache*>(malloc(sizeof(FP16KVCache)));
    if (!c) return nullptr;
    c->n_layers = n_layers;
    c->max_seq = max_seq;
    c->n_kv_heads = n_kv_heads;
    c->head_dim = head_dim;
    c->current_len = 0;
    c->k_cache = nullptr;
    c->v_cache = nullptr;
    const size_t bytes = (size_t)n_layers * max_seq * n_kv_heads * head_dim * sizeof(__half);
    if (hipMalloc(reinterpret_cast<void**>(&c->k_cache), bytes) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&c->v_cache), bytes) != hipSuccess) {
        fp16_kvcache_free(c);
        return nullptr;
    }
    return c;
}

void fp16_kvcache_free(FP16KVCache* c) {
    if (!c) return;
    if (c->k_cache) (void)hipFree(c->k_cache);
    if (c->v_cache) (void)hipFree(c->v_cache);
    free(c);
}

// ---- paged KV cache: src/paged_kvcache.cu:16-98 ----------------------------------
// One contiguous pool per K and V, block i at pool + i*block_elems; device
// pointer tables k_blocks/v_blocks; LIFO free list initialised so that a fresh
// pool hands out 0, 1, 2, ...; per-sequence block tables filled with -1.
extern "C" PagedKVCache* paged_kv_create(int n_blocks, int n_layers, int n_kv_heads,
                                         int head_dim, int max_seqs, int max_blocks_per_seq) {
    if (n_blocks <= 0 || n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_seqs < 0 ||
        max_blocks_per_seq < 0)
        return nullptr;
    PagedKVCache* c = static_cast<PagedKVCache*>(calloc(1, sizeof(PagedKVCache)));
    if (!c) return nullptr;
    c->n_blocks = n_blocks;
    c->n_layers = n_layers;
    c->n_kv_heads = n_kv_heads;
    c->head_dim = head_dim;
    c->max_seqs = max_seqs;
    c->max_blocks_per_seq = max_blocks_per_seq;

    const size_t block_elems = (size_t)n_layers * PAGE_SIZE * n_kv_heads * head_dim;
    __half* k_pool = nullptr;
    __half* v_pool = nullptr;
    __half** hk = static_cast<__half**>(malloc(n_blocks * sizeof(__half*)));
    __half** hv = static_cast<__half**>(malloc(n_blocks * sizeof(__half*)));
    bool ok = hk && hv;
    ok = ok && hipMalloc(reinterpret_cast<void**>(&k_pool), block_elems * n_blocks * sizeof(__half)) == hipSuccess;
    ok = ok && hipMalloc(reinterpret_cast<void**>(&v_pool), block_elems * n_blocks * sizeof(__half)) == hipSuccess;
    if (ok) {
        for (int i = 0; i < n_blocks; ++i) {
            hk[i] = k_pool + (size_t)i * block_elems;
            hv[i] = v_pool + (size_t)i * block_elems;
        }
    }
    ok = ok && hipMalloc(reinterpret_cast<void**>(&c->k_blocks), n_blocks * sizeof(__half*)) == hipSuccess;
    ok = ok && hipMalloc(reinterpret_cast<void**>(&c->v_blocks), n_blocks * sizeof(__half*)) == hipSuccess;
    ok = ok && hipMemcpy(c->k_blocks, hk, n_blocks * sizeof(__half*), hipMemcpyHostToDevice) == hipSuccess;
    ok = ok && hipMemcpy(c->v_blocks, hv, n_blocks * sizeof(__half*), hipMemcpyHostToDevice) == hipSuccess;
    free(hk);
    free(hv);

    if (ok) {
        c->free_blocks = static_cast<int*>(malloc(n_blocks * sizeof(int)));
        c->block_tables = static_cast<int**>(calloc(max_seqs > 0 ? max_seqs : 1, sizeof(int*)));
        ok = c->free_blocks && c->block_tables;
    }
    if (ok) {
        for (int i = 0; i < n_blocks; ++i) c->free_blocks[i] = n_blocks - 1 - i;
        c->free_count = n_blocks;
        for (int s = 0; s < max_seqs && ok; ++s) {
            c->block_tables[s] = static_cast<int*>(malloc((max_blocks_per_seq > 0 ? max_blocks_per_seq : 1) * sizeof(int)));
            ok = c->block_tables[s] != nullptr;
            for (int j = 0; ok && j < max_blocks_per_seq; ++j) c->block_tables[s][j] = -1;
        }
    }
    if (!ok) {
        if (k_pool) (void)hipFree(k_pool);
        if (v_pool) (void)hipFree(v_pool);
        if (c->k_blocks) (void)hipFree(c->k_blocks);
        if (c->v_blocks) (void)hipFree(c->v_blocks);
        free(c->free_blocks);
        if (c->block_tables)
            for (int s = 0; s < max_seqs; ++s) free(c->block_tables[s]);
        free(c->block_tables);
        free(c);
        return nullptr;
    }
    return c;
}

extern "C" void paged_kv_free(PagedKVCache* cache) {
    if (!cache) return;
    // The pool bases are block 0's pointers (src/paged_kvcache.cu:70-78).
    __half* k_pool = nullptr;
    __half* v_pool = nullptr;
    if (hipMemcpy(&k_pool, cache->k_blocks, sizeof(__half*), hipMemcpyDeviceToHost) == hipSuccess &&
        k_pool)
        (void)hipFree(k_pool);
    if (hipMemcpy(&v_pool, cache->v_blocks, sizeof(__half*), hipMemcpyDeviceToHost) == hipSuccess &&
        v_pool)
        (void)hipFree(v_pool);
    (void)hipFree(cache->k_blocks);
    (void)hipFree(cache->v_blocks);
    free(cache->free_blocks);
    for (int s = 0; s < cache->max_seqs; ++s) free(cache->block_tables[s]);
    free(cache->block_tables);
    free(cache);
}

// Pops the LIFO free list; -1 when the pool is exhausted (src/paged_kvcache.cu:89-93).
extern "C" int paged_kv_allocate_block(PagedKVCache* cache) {
    if (cache->free_count == 0) return -1;
    cache->free_count--;
    return cache->free_blocks[cache->free_count];
}

// Pushes a block back (src/paged_kvcache.cu:95-98).  Unlike the reference, an
// index outside the pool or a push onto a full list is ignored instead of
// writing past the stack.
extern "C" void paged_kv_free_block(PagedKVCache* cache, int block_idx) {
    if (block_idx < 0 || block_idx >= cache->n_blocks || cache->free_count >= cache->n_blocks)
        return;
    cache->free_blocks[cache->free_count] = block_idx;
    cache->free_count++;
}

// ---- quantlib FP8 (quantlib_src/src/quantlib.cu:26-143, kernels/fp8_convert.cu:91-173) ----
namespace {

int fp8_format_of(const QuantMatrix* qm) {
    return (qm->format[0] == 'E' && qm->format[1] == '5') ? QL_FP8_E5M2 : QL_FP8_E4M3;
}

QuantMatrix fp16_to_fp8(const __half* src, int rows, int cols, QuantGranularity gran,
                        int group_size, int fmt, hipStream_t stream) {
    QuantMatrix qm;
    memset(&qm, 0, sizeof(qm));
    qm.rows = rows;
    qm.cols = cols;
    qm.bits = 8;
    snprintf(qm.format, sizeof(qm.format), "%s", fmt == QL_FP8_E4M3 ? "E4M3" : "E5M2");
    const long long n = (long long)rows * cols;
    // group_size as the reference stores it (quantlib_src/kernels/fp8_convert.cu:111-112)
    qm.params.granularity = gran;
    qm.params.group_size = gran == QUANT_PER_TENSOR ? (int)n : (gran == QUANT_PER_CHANNEL ? cols : group_size);
    int ns = 0;
    if (ql_fp8_num_scales(rows, cols, (int)gran, group_size, &ns) != hipSuccess || n <= 0) return qm;
    qm.params.n_scales = ns;
    if (hipMalloc(&qm.data, (size_t)n) != hipSuccess) {
        qm.data = nullptr;
        return qm;
    }
    if (hipMalloc(reinterpret_cast<void**>(&qm.params.scales), (size_t)ns * sizeof(float)) != hipSuccess) {
        (void)hipFree(qm.data);
        qm.data = nullptr;
        qm.params.scales = nullptr;
        return qm;
    }
    (void)ql_fp8_quantize(bits(src), rows, cols, fmt, (int)gran, group_size, QL_FP8_MODE_REFERENCE,
                          static_cast<uint8_t*>(qm.data), qm.params.scales, stream);
    return qm;
}

// quantlib_fp8_gemm's workspace (split-K partials, or the dequantized weights for
// M > 64): one buffer per (device of the stream, stream), grown on demand, so
// calls on different streams never share one.  Each buffer has its own lock,
// held until the call's kernels are enqueued: a concurrent call on the same
// stream that grows the buffer waits for the stream before freeing the old one,
// while calls on other streams go on.  g_ws_mu guards only the map, whose
// entries are never removed before exit (so a Workspace stays where it is);
// the buffers are freed at process exit (free_workspaces, registered with
// atexit after the HIP runtime has loaded, so it runs before the runtime's
// own teardown).
struct Workspace {
    std::mutex mu;
    void* p = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, std::unique_ptr<Workspace>> g_ws;
bool g_ws_atexit = false;

void free_workspaces() {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    for (auto& kv : g_ws) {
        if (kv.second->p) {
            int cur = -1;
            if (hipGetDevice(&cur) == hipSuccess && cur != kv.first.first) (void)hipSetDevice(kv.first.first);
            (void)hipFree(kv.second->p);
            if (cur >= 0 && cur != kv.first.first) (void)hipSetDevice(cur);
            kv.second->p = nullptr;
            kv.second->bytes = 0;
        }
    }
}

// The device a stream belongs to (the current device for the null stream).
hipError_t stream_device(hipStream_t stream, int* dev) {
    if (stream == nullptr) return hipGetDevice(dev);
    return hipStreamGetDevice(stream, dev);
}

Workspace* workspace_for(int dev, hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    if (!g_ws_atexit) {
        g_ws_atexit = std::atexit(free_workspaces) == 0;
    }
    std::unique_ptr<Workspace>& w = g_ws[std::make_pair(dev, stream)];
    if (!w) w.reset(new Workspace);
    return w.get();
}

}  // namespace

extern "C" QuantMatrix quantlib_fp16_to_fp8_e4m3(const __half* src, int rows, int cols,
                                                 QuantGranularity gran, int group_size,
                                                 hipStream_t stream) {
    return fp16_to_fp8(src, rows, cols, gran, group_size, QL_FP8_E4M3, stream);
}

extern "C" QuantMatrix quantlib_fp16_to_fp8_e5m2(const __half* src, int rows, int cols,
                                                 QuantGranularity gran, int group_size,
                                                 hipStream_t stream) {
    return fp16_to_fp8(src, rows, cols, gran, group_size, QL_FP8_E5M2, stream);
}

extern "C" void quantlib_fp8_to_fp16(const QuantMatrix* qm, __half* dst, hipStream_t stream) {
    if (!qm || qm->bits != 8) return;
    (void)ql_fp8_dequantize(static_cast<const uint8_t*>(qm->data), qm->params.scales, qm->rows, qm->cols,
                            fp8_format_of(qm), (int)qm->params.granularity, qm->params.group_size,
                            QL_FP8_MODE_REFERENCE, bits(dst), stream);
}

extern "C" void quantlib_fp8_gemm(const __half* A, const QuantMatrix* W, __half* C, int M, int N,
                                  int K, hipStream_t stream) {
    if (!W || W->bits != 8) return;
    void* ws = nullptr;
    size_t ws_bytes = 0, need = 0;
    if (ql_fp8_gemm_workspace_size(M, N, K, (int)W->params.granularity, W->params.group_size, &need) !=
        hipSuccess)
        return;
    auto run = [&]() {
        (void)ql_fp8_gemm_f16(bits(A), static_cast<const uint8_t*>(W->data), W->params.scales, M, N, K,
                              fp8_format_of(W), (int)W->params.granularity, W->params.group_size,
                              QL_FP8_MODE_REFERENCE, bits(C), ws, ws_bytes, stream);
    };
    if (need == 0) {   // no workspace: nothing shared, no lock
        run();
        return;
    }
    int dev = 0;
    if (stream_device(stream, &dev) != hipSuccess) return;
    Workspace& slot = *workspace_for(dev, stream);
    std::lock_guard<std::mutex> lock(slot.mu);
    if (slot.bytes < need) {
        // allocate on the stream's device, whatever device is current
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess) return;
        if (cur != dev && hipSetDevice(dev) != hipSuccess) return;
        if (slot.p) {
            (void)hipStreamSynchronize(stream);   // earlier calls on this stream still use it
            (void)hipFree(slot.p);
        }
        const hipError_t e = hipMalloc(&slot.p, need);
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess) {
            slot.p = nullptr;
            slot.bytes = 0;
            return;
        }
        slot.bytes = need;
    }
    ws = slot.p;
    ws_bytes = slot.bytes;
    run();
}

extern "C" void quantlib_free(QuantMatrix* qm) {
    if (!qm) return;
    if (qm->data) (void)hipFree(qm->data);
    if (qm->params.scales) (void)hipFree(qm->params.scales);
    if (qm->params.zeros) (void)hipFree(qm->params.zeros);
    qm->data = nullptr;
    qm->params.scales = nullptr;
    qm->params.zeros = nullptr;
}

extern "C" float quantlib_quant_error(const __half* original, const __half* dequantized,
                                      int n_elements) {
    if (n_elements <= 0) return 0.0f;
    uint16_t* a = static_cast<uint16_t*>(malloc((size_t)n_elements * 2));
    uint16_t* b = static_cast<uint16_t*>(malloc((size_t)n_elements * 2));
    float max_err = 0.0f;
    if (a && b && hipMemcpy(a, original, (size_t)n_elements * 2, hipMemcpyDeviceToHost) == hipSuccess &&
        hipMemcpy(b, dequantized, (size_t)n_elements * 2, hipMemcpyDeviceToHost) == hipSuccess) {
        for (int i = 0; i < n_elements; ++i) {
            const float e = fabsf(half_to_float(a[i]) - half_to_float(b[i]));
            if (e > max_err) max_err = e;
        }
    }
    free(a);
    free(b);
    return max_err;
}

extern "C" void quantlib_print_stats(const QuantMatrix* qm) {
    if (!qm) return;
    const size_t raw = (size_t)qm->rows * qm->cols * 2;
    const size_t quant = qm->bits == 8 ? (size_t)qm->rows * qm->cols : ((size_t)qm->rows * qm->cols + 1) / 2;
    printf("QuantMatrix [%s]  %d x %d  bits=%d\n", qm->format, qm->rows, qm->cols, qm->bits);
    printf("  FP16 size    : %.2f MB\n", raw / 1e6f);
    printf("  Quant size   : %.2f MB\n", quant / 1e6f);
    printf("  Compression  : %.2fx\n", quant ? (float)raw / quant : 0.0f);
    printf("  Scales       : %d  (granularity=%d  group=%d)\n", qm->params.n_scales,
           (int)qm->params.granularity, qm->params.group_size);
}
