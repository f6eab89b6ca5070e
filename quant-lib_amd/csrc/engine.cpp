// engine.cpp -- one fp16 decoder layer (and the logits of the sampled rows) for a
// batched step, composed from the library's kernels and hipBLASLt GEMMs.
//
// The layer order of fp16_layer_forward (src/fp16_forward.cu:167-223), with
// the reference's per-token, per-op launches replaced by one batched step over
// every row a ql_batcher plan lists (prefills and decodes together):
//
//   x += delta_in; y = rmsnorm(x) * attn_norm        ql_add_rmsnorm_f16 (fused)
//   qkv = y Wqkv^T                                    hipBLASLt (Q, K, V in one GEMM)
//   rope(q, k); k, v -> paged pool                    ql_rope_paged_kv_append_f16 (fused)
//   a = attention(q, paged K/V)                       ql_paged_attention_f16, the split
//                                                     decode for all-decode steps, or
//                                                     ql_attention_f16 on the QKV rows
//                                                     for one fresh prompt
//   x += a Wo^T; y = rmsnorm(x) * ffn_norm            hipBLASLt + ql_add_rmsnorm_f16
//   delta_out = swiglu(y Wg^T, y Wu^T) Wd^T           hipBLASLt x2, ql_swiglu_f16, hipBLASLt
//
// The MLP output is returned as delta_out and added by the next layer's fused
// add+RMSNorm (or by ql_engine_logits_f16 after the last layer).  Weights are
// row-major [out_features, in_features] fp16 (y = x W^T).  GEMMs accumulate in
// fp32 and write fp16 (ql_gemm_f16).  ql_engine_layer_fp8 is the same layer on
// FP8 weights (the reference's quantized forward, src/quant_forward.cu:57-129):
// each GEMM is ql_fp8_gemm_f16.  The engine owns its activation buffers, the
// split-decode workspace and (ql_engine_create_fp8) the FP8 GEMM workspace,
// allocated once at creation; the per-step calls allocate nothing (the GEMM
// library context is created on the first fp16 GEMM).
#include "quantlib_amd.h"

#include <new>

namespace {

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

}  // namespace

struct ql_engine {
    ql_layer_dims dims{};
    int max_rows = 0, max_seqs = 0, max_ctx = 0;
    void* arena = nullptr;
    uint16_t *y = nullptr, *qkv = nullptr, *attn = nullptr, *o = nullptr, *g = nullptr, *u = nullptr,
             *mid = nullptr;
    void* dec_ws = nullptr;
    size_t dec_ws_bytes = 0;
    void* fp8_ws = nullptr;        // FP8 GEMM workspace (ql_engine_create_fp8)
    size_t fp8_ws_bytes = 0;

    ~ql_engine() {
        if (arena) (void)hipFree(arena);
    }
};

namespace {

// the layer GEMMs: fp16 weights through hipBLASLt, FP8 weights through ql_fp8_gemm_f16
struct GemmF16 {
    const ql_layer_weights* w;
    hipError_t operator()(const ql_engine*, const uint16_t* x, int which, uint16_t* out, int M, int N, int K,
                          hipStream_t stream) const {
        const uint16_t* m[] = {w->wqkv, w->wo, w->w_gate, w->w_up, w->w_down};
        return ql_gemm_f16(x, m[which], out, M, N, K, stream);
    }
};

struct GemmFp8 {
    const ql_layer_weights_fp8* w;
    hipError_t operator()(const ql_engine* e, const uint16_t* x, int which, uint16_t* out, int M, int N,
                          int K, hipStream_t stream) const {
        const ql_fp8_weight* m[] = {&w->wqkv, &w->wo, &w->w_gate, &w->w_up, &w->w_down};
        return ql_fp8_gemm_f16(x, m[which]->codes, m[which]->scales, M, N, K, w->format, w->granularity,
                               w->group_size, w->mode, out, e->fp8_ws, e->fp8_ws_bytes, stream);
    }
};

enum { kWqkv = 0, kWo = 1, kWgate = 2, kWup = 3, kWdown = 4 };

}  // namespace

#define QL_TRY(expr)                          \
    do {                                      \
        const hipError_t e_ = (expr);         \
        if (e_ != hipSuccess) return e_;      \
    } while (0)

namespace {

hipError_t engine_create(const ql_layer_dims* d, int max_rows, int max_seqs, int max_ctx_len,
                         size_t fp8_ws_bytes, ql_engine** out) {
    if (!out || !d || max_rows <= 0 || max_seqs <= 0 || max_ctx_len < 0) return hipErrorInvalidValue;
    if (d->hidden <= 0 || d->n_heads <= 0 || d->n_kv_heads <= 0 || d->n_kv_heads > d->n_heads ||
        (d->head_dim != 64 && d->head_dim != 128) || d->ffn <= 0 || d->hidden % 8 || d->ffn % 8 ||
        !(d->rope_theta > 0.0f) || (d->rope_pairing != QL_ROPE_INTERLEAVED && d->rope_pairing != QL_ROPE_HALF))
        return hipErrorInvalidValue;
    *out = nullptr;
    ql_engine* e = new (std::nothrow) ql_engine();
    if (!e) return hipErrorOutOfMemory;
    e->dims = *d;
    e->max_rows = max_rows;
    e->max_seqs = max_seqs;
    e->max_ctx = max_ctx_len;
    const size_t R = (size_t)max_rows, D = (size_t)d->hidden, F = (size_t)d->ffn;
    const size_t Q = (size_t)d->n_heads * d->head_dim, KV = (size_t)d->n_kv_heads * d->head_dim;
    size_t ws = 0;
    if (ql_paged_decode_workspace_size(max_seqs, d->n_heads, d->n_kv_heads, d->head_dim, max_ctx_len, &ws) !=
        hipSuccess) {
        delete e;
        return hipErrorInvalidValue;
    }
    e->dec_ws_bytes = ws;
    const size_t sizes[] = {R * D, R * (Q + 2 * KV), R * Q, R * D, R * F, R * F, R * F};
    size_t total = 0;
    for (size_t s : sizes) total += align256(s * sizeof(uint16_t));
    total += align256(ws) + align256(fp8_ws_bytes);
    if (hipMalloc(&e->arena, total) != hipSuccess) {
        delete e;
        return hipErrorOutOfMemory;
    }
    char* p = static_cast<char*>(e->arena);
    uint16_t** bufs[] = {&e->y, &e->qkv, &e->attn, &e->o, &e->g, &e->u, &e->mid};
    for (int i = 0; i < 7; ++i) {
        *bufs[i] = reinterpret_cast<uint16_t*>(p);
        p += align256(sizes[i] * sizeof(uint16_t));
    }
    e->dec_ws = ws ? p : nullptr;
    p += align256(ws);
    e->fp8_ws = fp8_ws_bytes ? p : nullptr;
    e->fp8_ws_bytes = fp8_ws_bytes;
    *out = e;
    return hipSuccess;
}

}  // namespace

extern "C" hipError_t ql_engine_create(const ql_layer_dims* d, int max_rows, int max_seqs,
                                       int max_ctx_len, ql_engine** out) {
    return engine_create(d, max_rows, max_seqs, max_ctx_len, 0, out);
}

// the FP8 GEMM workspace: the largest any layer GEMM needs at any row count up to
// max_rows (split partials grow with the rows up to 64; above 64 rows, a
// dequantized copy of the weight matrix)
extern "C" hipError_t ql_engine_create_fp8(const ql_layer_dims* d, int max_rows, int max_seqs,
                                           int max_ctx_len, int granularity, int group_size,
                                           ql_engine** out) {
    if (!d || !out || max_rows <= 0) return hipErrorInvalidValue;
    const int H = d->n_heads, HK = d->n_kv_heads, HD = d->head_dim, D = d->hidden, F = d->ffn;
    const int shapes[5][2] = {{(H + 2 * HK) * HD, D}, {D, H * HD}, {F, D}, {F, D}, {D, F}};
    size_t need = 0;
    for (const auto& nk : shapes) {
        for (int m : {max_rows < 64 ? max_rows : 64, max_rows}) {
            size_t b = 0;
            const hipError_t st = ql_fp8_gemm_workspace_size(m, nk[0], nk[1], granularity, group_size, &b);
            if (st != hipSuccess) return st;
            if (b > need) need = b;
        }
    }
    return engine_create(d, max_rows, max_seqs, max_ctx_len, need, out);
}

extern "C" hipError_t ql_engine_destroy(ql_engine* e) {
    delete e;
    return hipSuccess;
}

namespace {

template <typename Gemm>
hipError_t layer_forward(ql_engine* e, const uint16_t* attn_norm, const uint16_t* ffn_norm, const Gemm& gemm,
                         int layer, uint16_t* x, const uint16_t* delta_in, uint16_t* delta_out,
                         const ql_step_device* s, hipStream_t stream) {
    const ql_layer_dims& d = e->dims;
    const int T = s->n_rows;
    const int H = d.n_heads, HK = d.n_kv_heads, HD = d.head_dim, D = d.hidden, F = d.ffn;
    const int QKV = (H + 2 * HK) * HD;
    // attention sublayer
    if (delta_in)
        QL_TRY(ql_add_rmsnorm_f16(x, delta_in, attn_norm, e->y, T, D, d.rms_eps, stream));
    else
        QL_TRY(ql_rmsnorm_f16(x, attn_norm, e->y, T, D, d.rms_eps, stream));
    QL_TRY(gemm(e, e->y, kWqkv, e->qkv, T, QKV, D, stream));
    uint16_t* q = e->qkv;
    uint16_t* k = e->qkv + (size_t)H * HD;
    const uint16_t* v = e->qkv + (size_t)(H + HK) * HD;
    QL_TRY(ql_rope_paged_kv_append_f16(q, k, v, T, H, HK, HD, QKV, QKV, QKV, s->positions, 0,
                                       d.rope_theta, d.rope_pairing, s->k_blocks, s->v_blocks,
                                       s->n_blocks, s->slot_mapping, layer, s->n_layers, stream));
    const uint16_t* const* kb = reinterpret_cast<const uint16_t* const*>(s->k_blocks);
    const uint16_t* const* vb = reinterpret_cast<const uint16_t* const*>(s->v_blocks);
    if (s->n_seqs == 1 && s->max_q_len == T && s->max_ctx_len == T && T > 1) {
        // one fresh prompt: its keys are exactly this step's rows, still in the QKV
        // buffer (rotated in place), so the contiguous kernel reads them through the
        // row stride instead of the pool (same arithmetic, no page lookups)
        QL_TRY(ql_attention_f16(q, k, v, e->attn, T, T, H, HK, HD, QKV, QKV, (int64_t)H * HD, 1, stream));
    } else if (s->max_q_len == 1 && T == s->n_seqs) {   // every sequence decodes: row i = sequence i
        QL_TRY(ql_paged_decode_attention_f16(q, e->attn, QKV, (int64_t)H * HD, s->n_seqs, s->ctx_lens,
                                             s->max_ctx_len, s->block_tables, s->max_blocks, kb, vb,
                                             s->n_blocks, layer, s->n_layers, H, HK, HD, e->dec_ws,
                                             e->dec_ws_bytes, stream));
    } else {
        QL_TRY(ql_paged_attention_f16(q, e->attn, QKV, (int64_t)H * HD, T, s->n_seqs, s->cu_q_lens,
                                      s->ctx_lens, s->max_q_len, s->block_tables, s->max_blocks, kb, vb,
                                      s->n_blocks, layer, s->n_layers, H, HK, HD, 1, stream));
    }
    QL_TRY(gemm(e, e->attn, kWo, e->o, T, D, H * HD, stream));
    // MLP sublayer
    QL_TRY(ql_add_rmsnorm_f16(x, e->o, ffn_norm, e->y, T, D, d.rms_eps, stream));
    QL_TRY(gemm(e, e->y, kWgate, e->g, T, F, D, stream));
    QL_TRY(gemm(e, e->y, kWup, e->u, T, F, D, stream));
    QL_TRY(ql_swiglu_f16(e->g, e->u, e->mid, T, F, stream));
    QL_TRY(gemm(e, e->mid, kWdown, delta_out, T, D, F, stream));
    return hipSuccess;
}

// checks shared by both layer kinds; *done = true for an empty step
hipError_t check_step(const ql_engine* e, int layer, const uint16_t* x, const uint16_t* delta_out,
                      const ql_step_device* s, bool* done) {
    *done = false;
    if (!e || !x || !delta_out || !s) return hipErrorInvalidValue;
    const int T = s->n_rows;
    if (T < 0 || T > e->max_rows || s->n_seqs < 0 || s->n_seqs > e->max_seqs ||
        s->max_ctx_len > e->max_ctx || layer < 0 || layer >= s->n_layers)
        return hipErrorInvalidValue;
    *done = T == 0;
    return hipSuccess;
}

}  // namespace

extern "C" hipError_t ql_engine_layer_f16(ql_engine* e, const ql_layer_weights* w, int layer,
                                          uint16_t* x, const uint16_t* delta_in, uint16_t* delta_out,
                                          const ql_step_device* s, hipStream_t stream) {
    bool done = false;
    QL_TRY(check_step(e, layer, x, delta_out, s, &done));
    if (!w) return hipErrorInvalidValue;
    if (done) return hipSuccess;
    if (!w->attn_norm || !w->wqkv || !w->wo || !w->ffn_norm || !w->w_gate || !w->w_up || !w->w_down)
        return hipErrorInvalidValue;
    return layer_forward(e, w->attn_norm, w->ffn_norm, GemmF16{w}, layer, x, delta_in, delta_out, s, stream);
}

extern "C" hipError_t ql_engine_layer_fp8(ql_engine* e, const ql_layer_weights_fp8* w, int layer,
                                          uint16_t* x, const uint16_t* delta_in, uint16_t* delta_out,
                                          const ql_step_device* s, hipStream_t stream) {
    bool done = false;
    QL_TRY(check_step(e, layer, x, delta_out, s, &done));
    if (!w) return hipErrorInvalidValue;
    if (done) return hipSuccess;
    const ql_fp8_weight* m[] = {&w->wqkv, &w->wo, &w->w_gate, &w->w_up, &w->w_down};
    if (!w->attn_norm || !w->ffn_norm) return hipErrorInvalidValue;
    for (const ql_fp8_weight* mm : m)
        if (!mm->codes || !mm->scales) return hipErrorInvalidValue;
    // the workspace reserved at creation must cover this step's GEMMs
    const ql_layer_dims& d = e->dims;
    const int T = s->n_rows;
    const int shapes[5][2] = {{(d.n_heads + 2 * d.n_kv_heads) * d.head_dim, d.hidden},
                              {d.hidden, d.n_heads * d.head_dim}, {d.ffn, d.hidden}, {d.ffn, d.hidden},
                              {d.hidden, d.ffn}};
    for (const auto& nk : shapes) {
        size_t b = 0;
        QL_TRY(ql_fp8_gemm_workspace_size(T, nk[0], nk[1], w->granularity, w->group_size, &b));
        if (b > e->fp8_ws_bytes) return hipErrorInvalidValue;
    }
    return layer_forward(e, w->attn_norm, w->ffn_norm, GemmFp8{w}, layer, x, delta_in, delta_out, s, stream);
}

extern "C" hipError_t ql_engine_logits_f16(ql_engine* e, uint16_t* x, const uint16_t* delta_in,
                                           const uint16_t* final_norm, const uint16_t* lm_head,
                                           int vocab, const int32_t* sample_rows, int n_sample,
                                           int n_rows, uint16_t* logits, int32_t* tokens,
                                           hipStream_t stream) {
    if (!e || !x || !final_norm || !lm_head || !sample_rows || !logits || vocab <= 0 || vocab % 8 ||
        n_sample < 0 || n_sample > e->max_rows || n_rows < 0 || n_rows > e->max_rows)
        return hipErrorInvalidValue;
    if (n_sample == 0) return hipSuccess;
    const int D = e->dims.hidden;
    // finish the residual stream of every row, then gather the rows to sample
    if (delta_in)
        QL_TRY(ql_add_rmsnorm_f16(x, delta_in, final_norm, e->y, n_rows, D, e->dims.rms_eps, stream));
    else
        QL_TRY(ql_rmsnorm_f16(x, final_norm, e->y, n_rows, D, e->dims.rms_eps, stream));
    QL_TRY(ql_embed_f16(e->y, sample_rows, n_sample, n_rows, D, e->o, stream));
    QL_TRY(ql_gemm_f16(e->o, lm_head, logits, n_sample, vocab, D, stream));
    if (tokens) QL_TRY(ql_argmax_f16(logits, n_sample, vocab, vocab, tokens, stream));
    return hipSuccess;
}

extern "C" hipError_t ql_engine_tune(ql_engine* e, int rows, hipStream_t stream) {
    if (!e || rows < 1 || rows > e->max_rows) return hipErrorInvalidValue;
    const ql_layer_dims& d = e->dims;
    const int qkv = (d.n_heads + 2 * d.n_kv_heads) * d.head_dim, att = d.n_heads * d.head_dim;
    const int shapes[4][2] = {{qkv, d.hidden}, {d.hidden, att}, {d.ffn, d.hidden}, {d.hidden, d.ffn}};
    for (const auto& sh : shapes) {
        const hipError_t r = ql_gemm_tune_f16(rows, sh[0], sh[1], stream);
        if (r != hipSuccess) return r;
    }
    return hipSuccess;
}

