// gather.hip -- token-embedding gather and paged KV-cache append for gfx950.
//
// Both are row copies addressed through an index, bit-exact.  A wavefront
// serves whole tokens with its token index made scalar, so the index reads
// (ids, slots, block pointers) are scalar loads, which neither wait for nor
// hold back the vector row loads; rows move with 16-byte nontemporal
// accesses, 64 lanes covering a contiguous 1 KiB span per instruction.  The
// paged append loads its source rows before resolving the slot (they do not
// depend on it), so the slot -> block pointer chain runs while they are in
// flight.
#include "ql_common.hpp"
#include "quantlib_amd.h"

namespace {

using namespace ql;

// Copies TPW rows of `nvec` V-units, one wavefront.  Lane r < TPW holds row
// r's source and destination addresses (0 = none); they are broadcast with
// cross-lane permutes so every load of the group can be in flight at once
// (UNR per lane per pass) instead of paying the index -> address -> data
// latency chain once per row.  A row with a destination but no source is
// zero-filled.
template <int TPW, int UNR, bool NT, typename V>
__device__ __forceinline__ void wave_rows_copy(unsigned long long src_l, unsigned long long dst_l,
                                               int nvec, int lane) {
    const int total = TPW * nvec;
    for (int base = 0; base < total; base += kWave * UNR) {
        V r[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int idx = base + u * kWave + lane;
            const int row = min(idx / nvec, TPW - 1);
            const unsigned long long sp = __shfl(src_l, row, kWave);
            if (idx < total && sp)
                r[u] = load<NT>(reinterpret_cast<const V*>(sp) + (idx - row * nvec));
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int idx = base + u * kWave + lane;
            const int row = min(idx / nvec, TPW - 1);
            const unsigned long long sp = __shfl(src_l, row, kWave);
            const unsigned long long dp = __shfl(dst_l, row, kWave);
            if (idx < total && dp) {
                V v;
                if (sp) {
                    v = r[u];
                } else {
#pragma unroll
                    for (int e = 0; e < (int)(sizeof(V) / 4); ++e)
                        reinterpret_cast<uint32_t*>(&v)[e] = 0u;
                }
                store<NT>(reinterpret_cast<V*>(dp) + (idx - row * nvec), v);
            }
        }
    }
}

// out[t,:] = table[ids[t],:]  (src/forward.cu:137-141; kernels/fp16_ops.cu:81-89),
// batched over tokens.  An id outside [0, vocab) writes a zero row.
// With ids == NULL the single token `one_id` is gathered (the reference's
// one-token launchers pass the id by value).
// Vector path (dim*sizeof(D) % 16 == 0 and 16-byte aligned table/out, checked
// by the host): one token per wavefront, its id by a scalar load, then the row
// in passes of UNR vectors per lane, every load of a pass issued before its
// stores.  Measured at C5 (8192 tokens x 4096, tables rotated past the MALL):
// 24.5 -> 22.7 us against resolving the ids with vector loads and cross-lane
// broadcasts.
template <typename D, int UNR>
__global__ __launch_bounds__(kBlock) void embed_rows_vec(const D* __restrict__ table,
                                                         const int32_t* __restrict__ ids,
                                                         int one_id, int n_tokens, int vocab,
                                                         int dim, D* __restrict__ out) {
    using V = Vec<char, 16>;
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * (kBlock / kWave) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    if (t >= n_tokens) return;  // wavefront-uniform
    const int id = ids ? ld_scalar(ids + t) : one_id;
    const bool ok = id >= 0 && id < vocab;   // wavefront-uniform
    const V* src = reinterpret_cast<const V*>(table + (size_t)(ok ? id : 0) * dim);
    V* dst = reinterpret_cast<V*>(out + (size_t)t * dim);
    const int nvec = dim * (int)sizeof(D) / 16;
    for (int base = 0; base < nvec; base += kWave * UNR) {
        // every lane loads (an index past the row re-reads its last vector): a
        // load under a per-lane test makes the compiler wait for it before the next
        V r[UNR];
        if (ok) {
#pragma unroll
            for (int u = 0; u < UNR; ++u) r[u] = load<true>(src + min(base + u * kWave + lane, nvec - 1));
        } else {
#pragma unroll
            for (int u = 0; u < UNR; ++u)
#pragma unroll
                for (int e = 0; e < 16; ++e) r[u].v[e] = 0;   // out-of-range id: a zero row
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int i = base + u * kWave + lane;
            if (i < nvec) store<true>(dst + i, r[u]);
        }
    }
}

// Any dim / offset: one wavefront per token, element copies.  (Covering aligned
// vectors realigned by a shift of two loads per output vector measured slower at
// 8192 x 4095 binary16: 31.3 against 26.8 us.)
template <typename D>
__global__ __launch_bounds__(kBlock) void embed_rows_scalar(const D* __restrict__ table,
                                                            const int32_t* __restrict__ ids,
                                                            int one_id, int n_tokens, int vocab,
                                                            int dim, D* __restrict__ out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (t >= n_tokens) return;
    const int id = ids ? ids[t] : one_id;
    const bool ok = id >= 0 && id < vocab;
    for (int i = lane; i < dim; i += kWave)
        out[(size_t)t * dim + i] = ok ? table[(size_t)id * dim + i] : D(0);
}

constexpr int kEmbedUNR = 8;   // 16-byte vectors per lane per pass (a 4096-wide fp16 row in one)

template <typename D>
hipError_t embed_dispatch(const D* table, const int32_t* ids, int one_id, int n_tokens,
                          int vocab, int dim, D* out, hipStream_t stream) {
    QL_CHECK_ARG(n_tokens >= 0 && vocab >= 0 && dim >= 0);
    if (n_tokens == 0 || dim == 0) return hipSuccess;
    QL_CHECK_ARG(table && out && (ids || n_tokens == 1));
    QL_CHECK_ARG(((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(out)) & (sizeof(D) - 1)) == 0);
    QL_CHECK_ARG((long long)dim * (long long)sizeof(D) < (1LL << 31));
    const int wpb = kBlock / kWave;
    if ((dim * (int)sizeof(D)) % 16 == 0 && qlh::aligned16(table) && qlh::aligned16(out)) {
        const unsigned grid = qlh::blocks_for(n_tokens, (long long)wpb);
        hipLaunchKernelGGL((embed_rows_vec<D, kEmbedUNR>), dim3(grid), dim3(kBlock), 0,
                           stream, table, ids, one_id, n_tokens, vocab, dim, out);
    } else {
        hipLaunchKernelGGL((embed_rows_scalar<D>), dim3(qlh::blocks_for(n_tokens, wpb)),
                           dim3(kBlock), 0, stream, table, ids, one_id, n_tokens, vocab, dim, out);
    }
    return hipGetLastError();
}

// Paged append: token t's [kv] K and V runs go to
//   blocks[slot/16] + ((layer*16 + slot%16) * kv)
// (pool layout of src/paged_kvcache.cu:26-46, block [n_layers,16,H_kv,d]).
// Vector path (kv % 8 == 0, 16-byte aligned k_new/v_new, checked by the host):
// TPW tokens per wavefront; lanes < TPW resolve slot -> block pointer, and a
// block pointer that is not 16-byte aligned sends that token through the
// element loop instead.
template <int TPW, int UNR>
__global__ __launch_bounds__(kBlock) void paged_append_vec(
    _Float16* const* __restrict__ kb, _Float16* const* __restrict__ vb, int n_blocks,
    const int32_t* __restrict__ slots, const _Float16* __restrict__ kn,
    const _Float16* __restrict__ vn, int n_tokens, int layer, int kv) {
    const int lane = threadIdx.x & (kWave - 1);
    const int t0 = (blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave) * TPW;
    if (t0 >= n_tokens) return;  // wavefront-uniform
    unsigned long long ks = 0, vs = 0, kd = 0, vd = 0;
    bool odd = false;  // destination not 16-byte aligned
    if (lane < TPW && t0 + lane < n_tokens) {
        const int t = t0 + lane;
        const int slot = slots[t];
        if (slot >= 0 && slot / QL_PAGE_SIZE < n_blocks) {
            const int b = slot / QL_PAGE_SIZE;
            const size_t off = ((size_t)layer * QL_PAGE_SIZE + slot % QL_PAGE_SIZE) * (size_t)kv;
            kd = reinterpret_cast<unsigned long long>(kb[b] + off);
            vd = reinterpret_cast<unsigned long long>(vb[b] + off);
            ks = reinterpret_cast<unsigned long long>(kn + (size_t)t * kv);
            vs = reinterpret_cast<unsigned long long>(vn + (size_t)t * kv);
            odd = ((kd | vd) & 15) != 0;
        }
    }
    if (__any(odd)) {
        // rare: some block base is misaligned -- element copies for those tokens
        for (int r = 0; r < TPW; ++r) {
            const bool rodd = __shfl((int)odd, r, kWave);
            if (!rodd) continue;
            _Float16* kdr = reinterpret_cast<_Float16*>(__shfl(kd, r, kWave));
            _Float16* vdr = reinterpret_cast<_Float16*>(__shfl(vd, r, kWave));
            const _Float16* ksr = reinterpret_cast<const _Float16*>(__shfl(ks, r, kWave));
            const _Float16* vsr = reinterpret_cast<const _Float16*>(__shfl(vs, r, kWave));
            for (int i = lane; i < kv; i += kWave) {
                kdr[i] = ksr[i];
                vdr[i] = vsr[i];
            }
        }
        if (odd) ks = vs = kd = vd = 0;
    }
    const int nvec = kv / 8;
    wave_rows_copy<TPW, UNR, true, Vec<char, 16>>(ks, kd, nvec, lane);
    wave_rows_copy<TPW, UNR, true, Vec<char, 16>>(vs, vd, nvec, lane);
}

// Rows-first variant for rows of up to 64*NV vectors (kv <= 512*NV): TPW tokens
// per wavefront, all their K and V source rows loaded first (they do not
// depend on the slot), then each token's slot and block pointers read with
// scalar loads while the rows are in flight, then the stores.  A block
// pointer that is not 16-byte aligned takes element stores for that token.
// Measured at C5 (8192 tokens x 8 heads x 128, K/V rotated past the MALL):
// 14.8 -> 12.6 us against the one-token, slot-first kernel above.
template <int TPW, int NV>
__global__ __launch_bounds__(kBlock) void paged_append_rows(
    _Float16* const* __restrict__ kb, _Float16* const* __restrict__ vb, int n_blocks,
    const int32_t* __restrict__ slots, const _Float16* __restrict__ kn,
    const _Float16* __restrict__ vn, int n_tokens, int layer, int kv) {
    using V = Vec<char, 16>;
    const int lane = threadIdx.x & (kWave - 1);
    const int t0 = (blockIdx.x * (kBlock / kWave) +
                    __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave))) * TPW;
    if (t0 >= n_tokens) return;  // wavefront-uniform
    const int nvec = kv / 8;
    V rk[TPW][NV], rv[TPW][NV];
    // every lane loads: indices past the row or the last token re-read valid
    // vectors (a load under a per-lane test makes the compiler wait for it
    // before issuing the next one)
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        const int t = min(t0 + j, n_tokens - 1);
        const V* ks = reinterpret_cast<const V*>(kn + (size_t)t * kv);
        const V* vs = reinterpret_cast<const V*>(vn + (size_t)t * kv);
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int i = min(lane + u * kWave, nvec - 1);
            rk[j][u] = load<true>(ks + i);
            rv[j][u] = load<true>(vs + i);
        }
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        if (t0 + j >= n_tokens) break;
        const int slot = ld_scalar(slots + t0 + j);
        if (slot < 0 || slot / QL_PAGE_SIZE >= n_blocks) continue;
        const size_t off = ((size_t)layer * QL_PAGE_SIZE + slot % QL_PAGE_SIZE) * (size_t)kv;
        _Float16* kd = ld_scalar(kb + slot / QL_PAGE_SIZE) + off;
        _Float16* vd = ld_scalar(vb + slot / QL_PAGE_SIZE) + off;
        const bool aligned = ((reinterpret_cast<uintptr_t>(kd) | reinterpret_cast<uintptr_t>(vd)) & 15) == 0;
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const int i = lane + u * kWave;
            if (i >= nvec) continue;
            if (aligned) {
                store<true>(reinterpret_cast<V*>(kd) + i, rk[j][u]);
                store<true>(reinterpret_cast<V*>(vd) + i, rv[j][u]);
            } else {   // a caller-provided pool with misaligned blocks: element stores
                const _Float16* ke = reinterpret_cast<const _Float16*>(&rk[j][u]);
                const _Float16* ve = reinterpret_cast<const _Float16*>(&rv[j][u]);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    kd[8 * i + e] = ke[e];
                    vd[8 * i + e] = ve[e];
                }
            }
        }
    }
}

// Any kv / alignment: one wavefront per token, element copies.
__global__ __launch_bounds__(kBlock) void paged_append_scalar(
    _Float16* const* __restrict__ kb, _Float16* const* __restrict__ vb, int n_blocks,
    const int32_t* __restrict__ slots, const _Float16* __restrict__ kn,
    const _Float16* __restrict__ vn, int n_tokens, int layer, int kv) {
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (t >= n_tokens) return;
    const int slot = slots[t];
    if (slot < 0 || slot / QL_PAGE_SIZE >= n_blocks) return;
    const int b = slot / QL_PAGE_SIZE;
    const size_t off = ((size_t)layer * QL_PAGE_SIZE + slot % QL_PAGE_SIZE) * (size_t)kv;
    for (int i = lane; i < kv; i += kWave) {
        kb[b][off + i] = kn[(size_t)t * kv + i];
        vb[b][off + i] = vn[(size_t)t * kv + i];
    }
}

constexpr int kPagedTPW = 1;   // tokens per wavefront of the wide-row kernel
constexpr int kPagedUNR = 2;
constexpr int kRowsTPW = 4;    // tokens per wavefront of the rows-first kernel (best of 1, 2, 4)

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
    const int wpb = kBlock / kWave;
    const bool vec_ok = kv % 8 == 0 && qlh::aligned16(k_new) && qlh::aligned16(v_new);
    if (vec_ok && kv <= 512 * 4) {
        const unsigned grid = qlh::blocks_for(n_tokens, (long long)wpb * kRowsTPW);
        auto* k_ = reinterpret_cast<_Float16* const*>(k_blocks);
        auto* v_ = reinterpret_cast<_Float16* const*>(v_blocks);
        auto* kn = reinterpret_cast<const _Float16*>(k_new);
        auto* vn = reinterpret_cast<const _Float16*>(v_new);
        if (kv <= 512)
            hipLaunchKernelGGL((paged_append_rows<kRowsTPW, 1>), dim3(grid), dim3(kBlock), 0, stream, k_, v_,
                               n_blocks, slot_mapping, kn, vn, n_tokens, layer, kv);
        else if (kv <= 1024)
            hipLaunchKernelGGL((paged_append_rows<kRowsTPW, 2>), dim3(grid), dim3(kBlock), 0, stream, k_, v_,
                               n_blocks, slot_mapping, kn, vn, n_tokens, layer, kv);
        else
            hipLaunchKernelGGL((paged_append_rows<kRowsTPW, 4>), dim3(grid), dim3(kBlock), 0, stream, k_, v_,
                               n_blocks, slot_mapping, kn, vn, n_tokens, layer, kv);
    } else if (vec_ok) {
        hipLaunchKernelGGL((paged_append_vec<kPagedTPW, kPagedUNR>),
                           dim3(qlh::blocks_for(n_tokens, (long long)wpb * kPagedTPW)), dim3(kBlock),
                           0, stream, reinterpret_cast<_Float16* const*>(k_blocks),
                           reinterpret_cast<_Float16* const*>(v_blocks), n_blocks, slot_mapping,
                           reinterpret_cast<const _Float16*>(k_new),
                           reinterpret_cast<const _Float16*>(v_new), n_tokens, layer, kv);
    } else {
        hipLaunchKernelGGL(paged_append_scalar, dim3(qlh::blocks_for(n_tokens, wpb)), dim3(kBlock),
                           0, stream, reinterpret_cast<_Float16* const*>(k_blocks),
                           reinterpret_cast<_Float16* const*>(v_blocks), n_blocks, slot_mapping,
                           reinterpret_cast<const _Float16*>(k_new),
                           reinterpret_cast<const _Float16*>(v_new), n_tokens, layer, kv);
    }
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
