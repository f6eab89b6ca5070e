// gather.hip -- token-embedding gather and paged KV-cache append for gfx950.
//
// Both are row copies addressed through an index: one wavefront per token
// reads the token's index once (a wavefront-uniform scalar load) and moves the
// row with 16-byte lane accesses, 64 lanes covering a contiguous 1 KiB span per
// instruction and up to 8 vectors per lane in flight.  Results are bit-exact
// copies.
#include "ql_common.hpp"
#include "quantlib_amd.h"

namespace {

using namespace ql;

constexpr int kRowUnroll = 8;

// Copy `nvec` W-element units from src to dst, one wavefront.
template <typename V>
__device__ __forceinline__ void wave_copy(V* __restrict__ dst, const V* __restrict__ src,
                                          int nvec, int lane) {
    for (int b = lane; b < nvec; b += kWave * kRowUnroll) {
        V r[kRowUnroll];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u)
            if (b + u * kWave < nvec) r[u] = src[b + u * kWave];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u)
            if (b + u * kWave < nvec) dst[b + u * kWave] = r[u];
    }
}

// out[t,:] = table[ids[t],:]  (src/forward.cu:137-141; kernels/fp16_ops.cu:81-89),
// batched over tokens.  An id outside [0, vocab) writes a zero row.
// With ids == NULL the single token `one_id` is gathered (the reference's
// one-token launchers pass the id by value).
template <typename D, int W>
__global__ __launch_bounds__(kBlock) void embed_rows(const D* __restrict__ table,
                                                     const int32_t* __restrict__ ids,
                                                     int one_id, int n_tokens, int vocab,
                                                     int dim, D* __restrict__ out) {
    using V = Vec<D, W>;
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (t >= n_tokens) return;
    const int id = ids ? ids[t] : one_id;
    const int nvec = dim / W;
    V* dst = reinterpret_cast<V*>(out + (size_t)t * dim);
    if (id < 0 || id >= vocab) {
        V z;
#pragma unroll
        for (int e = 0; e < W; ++e) z.v[e] = D(0);
        for (int i = lane; i < nvec; i += kWave) dst[i] = z;
        return;
    }
    wave_copy(dst, reinterpret_cast<const V*>(table + (size_t)id * dim), nvec, lane);
}

template <typename D>
hipError_t embed_dispatch(const D* table, const int32_t* ids, int one_id, int n_tokens,
                          int vocab, int dim, D* out, hipStream_t stream) {
    QL_CHECK_ARG(n_tokens >= 0 && vocab >= 0 && dim >= 0);
    if (n_tokens == 0 || dim == 0) return hipSuccess;
    QL_CHECK_ARG(table && out && (ids || n_tokens == 1));
    constexpr int W = vec16<D>();
    const unsigned grid = qlh::blocks_for(n_tokens, kBlock / kWave);
    if (dim % W == 0 && qlh::aligned16(table) && qlh::aligned16(out))
        hipLaunchKernelGGL((embed_rows<D, W>), dim3(grid), dim3(kBlock), 0, stream, table, ids,
                           one_id, n_tokens, vocab, dim, out);
    else
        hipLaunchKernelGGL((embed_rows<D, 1>), dim3(grid), dim3(kBlock), 0, stream, table, ids,
                           one_id, n_tokens, vocab, dim, out);
    return hipGetLastError();
}

// Paged append: token t's [kv] K and V runs go to
//   blocks[slot/16] + ((layer*16 + slot%16) * kv)
// (pool layout of src/paged_kvcache.cu:26-46, block [n_layers,16,H_kv,d]).
// Block pointers are read from the device table, so the 16-byte path is
// chosen per token from the actual addresses.
__global__ __launch_bounds__(kBlock) void paged_append_rows(
    _Float16* const* __restrict__ kb, _Float16* const* __restrict__ vb, int n_blocks,
    const int32_t* __restrict__ slots, const _Float16* __restrict__ kn,
    const _Float16* __restrict__ vn, int n_tokens, int layer, int kv) {
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (t >= n_tokens) return;
    const int slot = slots[t];
    if (slot < 0) return;
    const int b = slot / QL_PAGE_SIZE;
    const int o = slot % QL_PAGE_SIZE;
    if (b >= n_blocks) return;
    const size_t off = ((size_t)layer * QL_PAGE_SIZE + o) * (size_t)kv;
    _Float16* kd = kb[b] + off;
    _Float16* vd = vb[b] + off;
    const _Float16* ks = kn + (size_t)t * kv;
    const _Float16* vs = vn + (size_t)t * kv;
    const bool vec_ok = kv % 8 == 0 &&
                        (((uintptr_t)kd | (uintptr_t)vd | (uintptr_t)ks | (uintptr_t)vs) & 15) == 0;
    if (vec_ok) {
        using V = Vec<_Float16, 8>;
        const int nvec = kv / 8;
        // K and V interleaved in one pass: 2 x up to 4 vectors in flight per lane.
        for (int bi = lane; bi < nvec; bi += kWave * 4) {
            V rk[4], rv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (bi + u * kWave < nvec) {
                    rk[u] = reinterpret_cast<const V*>(ks)[bi + u * kWave];
                    rv[u] = reinterpret_cast<const V*>(vs)[bi + u * kWave];
                }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (bi + u * kWave < nvec) {
                    reinterpret_cast<V*>(kd)[bi + u * kWave] = rk[u];
                    reinterpret_cast<V*>(vd)[bi + u * kWave] = rv[u];
                }
        }
    } else {
        for (int i = lane; i < kv; i += kWave) {
            kd[i] = ks[i];
            vd[i] = vs[i];
        }
    }
}

}  // namespace

extern "C" int ql_version(void) { return 100; }

extern "C" hipError_t ql_embed_f32(const float* table, const int32_t* ids, int n_tokens,
                                   int vocab, int dim, float* out, hipStream_t stream) {
    QL_CHECK_ARG(ids || n_tokens == 0);
    return embed_dispatch<float>(table, ids, 0, n_tokens, vocab, dim, out, stream);
}

extern "C" hipError_t ql_embed_f16(const uint16_t* table, const int32_t* ids, int n_tokens,
                                   int vocab, int dim, uint16_t* out, hipStream_t stream) {
    QL_CHECK_ARG(ids || n_tokens == 0);
    return embed_dispatch<_Float16>(reinterpret_cast<const _Float16*>(table), ids, 0, n_tokens,
                                    vocab, dim, reinterpret_cast<_Float16*>(out), stream);
}

extern "C" hipError_t ql_embed_token_f32(const float* table, int token_id, int dim, float* out,
                                         hipStream_t stream) {
    return embed_dispatch<float>(table, nullptr, token_id, 1, 0x7fffffff, dim, out, stream);
}

extern "C" hipError_t ql_embed_token_f16(const uint16_t* table, int token_id, int dim,
                                         uint16_t* out, hipStream_t stream) {
    return embed_dispatch<_Float16>(reinterpret_cast<const _Float16*>(table), nullptr, token_id,
                                    1, 0x7fffffff, dim, reinterpret_cast<_Float16*>(out), stream);
}

extern "C" hipError_t ql_paged_kv_append_f16(uint16_t* const* k_blocks,
                                             uint16_t* const* v_blocks, int n_blocks,
                                             const int32_t* slot_mapping,
                                             const uint16_t* k_new, const uint16_t* v_new,
                                             int n_tokens, int layer, int n_layers,
                                             int n_kv_heads, int head_dim, hipStream_t stream) {
    QL_CHECK_ARG(n_tokens >= 0 && n_blocks >= 0 && n_kv_heads > 0 && head_dim > 0);
    QL_CHECK_ARG(n_layers > 0 && layer >= 0 && layer < n_layers);
    QL_CHECK_ARG((long long)n_kv_heads * head_dim <= (1LL << 30));
    if (n_tokens == 0 || n_blocks == 0) return hipSuccess;
    QL_CHECK_ARG(k_blocks && v_blocks && slot_mapping && k_new && v_new);
    const int kv = n_kv_heads * head_dim;
    hipLaunchKernelGGL(paged_append_rows, dim3(qlh::blocks_for(n_tokens, kBlock / kWave)),
                       dim3(kBlock), 0, stream,
                       reinterpret_cast<_Float16* const*>(k_blocks),
                       reinterpret_cast<_Float16* const*>(v_blocks), n_blocks, slot_mapping,
                       reinterpret_cast<const _Float16*>(k_new),
                       reinterpret_cast<const _Float16*>(v_new), n_tokens, layer, kv);
    return hipGetLastError();
}

extern "C" hipError_t ql_paged_slot_mapping(const int32_t* block_table, int n_table,
                                            int start_pos, int n_tokens, int32_t* slot_mapping) {
    QL_CHECK_ARG(n_tokens >= 0 && start_pos >= 0 && n_table >= 0);
    if (n_tokens == 0) return hipSuccess;
    QL_CHECK_ARG(block_table && slot_mapping);
    for (int i = 0; i < n_tokens; ++i) {
        const long long p = (long long)start_pos + i;
        const long long lb = p / QL_PAGE_SIZE;
        if (lb >= n_table) return hipErrorInvalidValue;
        const int32_t pb = block_table[lb];
        if (pb < 0 || pb > 0x7fffffff / QL_PAGE_SIZE - 1) return hipErrorInvalidValue;
        slot_mapping[i] = pb * QL_PAGE_SIZE + (int32_t)(p % QL_PAGE_SIZE);
    }
    return hipSuccess;
}
