// attention.hip -- fp16 flash attention with grouped-query heads on gfx950
// matrix cores, over contiguous K/V or the paged KV cache the append kernels
// write.
//
// Semantics follow launch_flash_attention / flash_attention_fp16_kernel
// (kernels/flash_attention.cu:29-182): per query head h the KV head is
// h * n_kv_heads / n_heads (:45); scores are (q . k) * scale with
// scale = 1/sqrtf(head_dim) (:173); keys after the query's position are
// masked when causal (:106); the softmax is the online (running max, running
// sum) form and the output is O / (l + 1e-8) (:161).  Generalisations: the
// queries may be the last q_len positions of a longer context (decode and
// chunked prefill), head_dim may be 64 or 128 (the reference's tiles hold 64),
// rows may be strided, and K/V may live in 16-token pages.
//
// Work decomposition.  One workgroup = 4 wavefronts = 128 consecutive queries
// of one query head; each wavefront owns 32 queries.  Keys stream through LDS
// in tiles of 64 (double-buffered: the next tile is fetched into registers
// while the current one is multiplied).  Per tile and wavefront:
//   S^T (64 keys x 32 queries) = K . Q^T    -- v_mfma_f32_32x32x16_f16
//   O^T (d x 32 queries)      += V^T . P^T
// Computing the transposed products makes every lane own one query column:
// the running max/sum are per lane, rescaling O is a per-lane multiply, and
// the P^T operand of the second product is the lane's own S^T registers
// narrowed to fp16 (no shuffles).  The contraction order of the keys inside
// one 16-key MFMA step is permuted identically in both operands, which the
// sum does not see.  V is stored transposed in LDS (d-major) so the V^T
// operand is two 8-byte LDS reads per MFMA.
//
// Precision: Q, K, V, P in fp16 (exact products), fp32 accumulation and
// softmax state; p = 2^(s*c - m*c) with c = scale*log2(e) from v_exp_f32, m a
// running offset that is raised only when a query's maximum grows by more than
// 2^8 (so p <= 256; the offset cancels in O/l); the row sum l adds the
// fp16-rounded p (v_dot2 with ones, fp32 accumulation), so O/l is an exact
// convex combination of the fp16 weights that multiplied V.
//
// Workgroups are mapped XCD-aware: ids go to the 8 XCDs round-robin, and each
// XCD is handed a contiguous run of query heads (and so of KV heads).
#include "ql_common.hpp"
#include "quantlib_amd.h"

#include <math.h>
#include <float.h>

namespace {

using namespace ql;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = kAttnWaves * kWave;   // 256
constexpr int kBQ = 32 * kAttnWaves;               // 128 queries per workgroup
constexpr int kBK = 64;                            // keys per tile

template <int HD>
struct Tile {
    static constexpr int KS = HD + 8;        // K row stride in LDS (halfs): +16 B breaks bank aliasing
    static constexpr int VS = kBK + 4;       // V^T row stride (halfs): +8 B
    static constexpr int K_ELEMS = kBK * KS;
    static constexpr int V_ELEMS = HD * VS;
    static constexpr int STAGE = K_ELEMS + V_ELEMS;
    static constexpr int KCH = HD / 8;       // 16-byte chunks per K/V row
    static constexpr int KLOADS = kBK * KCH / kAttnThreads;   // K chunks per thread
    static constexpr int KPT = HD / 32;      // keys per thread in the V loader (4 or 2)
    static constexpr int VGROUPS = kBK / KPT;                 // key groups (16 or 32)
    static_assert(KLOADS * kAttnThreads == kBK * KCH, "K tile split");
    static_assert(VGROUPS * KCH == kAttnThreads, "V tile split");
};

struct AttnArgs {
    const _Float16* q;
    _Float16* out;
    int64_t q_stride;        // elements between consecutive query rows
    int64_t o_stride;
    int n_heads, n_kv_heads;
    float cl2;               // scale * log2(e)
    int causal;
    // one sequence over contiguous K/V
    int q_len, kv_len;
    const _Float16* k;
    const _Float16* v;
    int64_t kv_stride;       // elements between consecutive key rows
    // paged K/V, several sequences
    const _Float16* const* kb;
    const _Float16* const* vb;
    int n_blocks;
    const int32_t* block_tables;   // [n_seqs, max_blocks]
    int max_blocks;
    const int32_t* cu_q;           // [n_seqs + 1] first query row of each sequence
    const int32_t* ctx_lens;       // [n_seqs] keys of each sequence
    int n_q_rows;                  // rows available in q / out
    int layer;
};

// Address of key row j (its d values are contiguous) for this KV head, or 0
// when the key has no backing block.
template <bool PAGED>
__device__ __forceinline__ uintptr_t key_row(const AttnArgs& a, const _Float16* base,
                                             const _Float16* const* blocks, const int32_t* table,
                                             int kvh, int j, int hd) {
    if constexpr (PAGED) {
        const int t = j >> 4;
        if (t >= a.max_blocks) return 0;
        const int b = table[t];
        if (b < 0 || b >= a.n_blocks) return 0;
        const size_t off = (((size_t)a.layer * QL_PAGE_SIZE + (j & (QL_PAGE_SIZE - 1))) *
                                (size_t)a.n_kv_heads + kvh) * hd;
        return reinterpret_cast<uintptr_t>(blocks[b] + off);
    } else {
        return reinterpret_cast<uintptr_t>(base + (size_t)j * a.kv_stride + (size_t)kvh * hd);
    }
}

typedef const __attribute__((address_space(1))) half8* GlobalHalf8Ptr;

// 16 bytes of chunk ch of a key row (row == 0: missing key -> zeros).  Loads
// always target a valid address (dummy stands in for a missing row) and the
// value is selected afterwards, so the fast path has no branches; loads are
// issued in the global address space so they count only against the vector
// memory counter (LDS waits do not wait for them).  A page pointer that is not
// 16-byte aligned (caller-provided pools) sends the wavefront through an
// element-wise path.
template <bool PAGED>
__device__ __forceinline__ half8 load_chunk(uintptr_t row, int ch, uintptr_t dummy) {
    const bool ok = row != 0;
    const uintptr_t src = (ok ? row : dummy) + 16 * (uintptr_t)ch;
    if constexpr (PAGED) {
        if (__any((src & 15) != 0)) {
            half8 r{};
            if (ok) {
                const _Float16* e = reinterpret_cast<const _Float16*>(src);
#pragma unroll
                for (int i = 0; i < 8; ++i) r[i] = e[i];
            }
            return r;
        }
    }
    const half8 x = *(GlobalHalf8Ptr)src;
    return ok ? x : half8{};
}

template <int HD, bool PAGED>
struct TileRegs {
    half8 k[Tile<HD>::KLOADS];
    half8 v[Tile<HD>::KPT];
};

// Fetch key tile [kv0, kv0+64) of this KV head into registers (keys at or
// beyond kv_len read as zeros; they are masked anyway).
template <int HD, bool PAGED>
__device__ __forceinline__ void fetch_tile(TileRegs<HD, PAGED>& r, const AttnArgs& a,
                                           const int32_t* table, int kvh, int kv0, int kv_len,
                                           uintptr_t dummy) {
    using T = Tile<HD>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < T::KLOADS; ++i) {
        const int idx = tid + kAttnThreads * i;
        const int key = idx / T::KCH, ch = idx % T::KCH;
        const int j = kv0 + key;
        const uintptr_t row = j < kv_len ? key_row<PAGED>(a, a.k, a.kb, table, kvh, j, HD) : 0;
        r.k[i] = load_chunk<PAGED>(row, ch, dummy);
    }
    const int g = tid % T::VGROUPS, ch = tid / T::VGROUPS;
#pragma unroll
    for (int i = 0; i < T::KPT; ++i) {
        const int j = kv0 + g * T::KPT + i;
        const uintptr_t row = j < kv_len ? key_row<PAGED>(a, a.v, a.vb, table, kvh, j, HD) : 0;
        r.v[i] = load_chunk<PAGED>(row, ch, dummy);
    }
}

// Registers -> LDS stage: K row-major [key][d], V transposed [d][key].
template <int HD, bool PAGED>
__device__ __forceinline__ void stash_tile(const TileRegs<HD, PAGED>& r, _Float16* sk, _Float16* sv) {
    using T = Tile<HD>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < T::KLOADS; ++i) {
        const int idx = tid + kAttnThreads * i;
        const int key = idx / T::KCH, ch = idx % T::KCH;
        *reinterpret_cast<half8*>(sk + key * T::KS + ch * 8) = r.k[i];
    }
    const int g = tid % T::VGROUPS, ch = tid / T::VGROUPS;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        _Float16* dst = sv + (ch * 8 + e) * T::VS + g * T::KPT;
        if constexpr (T::KPT == 4) {
            *reinterpret_cast<half4*>(dst) = half4{r.v[0][e], r.v[1][e], r.v[2][e], r.v[3][e]};
        } else {
            *reinterpret_cast<half2v*>(dst) = half2v{r.v[0][e], r.v[1][e]};
        }
    }
}

template <int HD, bool PAGED>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_fwd(AttnArgs a) {
    using T = Tile<HD>;
    constexpr int NKK = HD / 16;   // MFMA steps over d for S^T
    constexpr int NDB = HD / 32;   // 32-row blocks of O^T
    __shared__ _Float16 smem[2 * T::STAGE];

    // Work item (query head, query tile).  Consecutive workgroup ids go to the
    // 8 XCDs in turn; when the heads split evenly over the XCDs, each XCD is
    // given its own contiguous run of heads (so the K/V rows of their shared KV
    // heads stay in that XCD's L2).  Causal: heavy (late) query tiles first.
    const int n_qt = (int)gridDim.x / a.n_heads;
    int head, t;
    if (a.n_heads % 8 == 0) {
        const int hpx = a.n_heads / 8, xcd = (int)blockIdx.x & 7, j = (int)blockIdx.x >> 3;
        head = xcd * hpx + j % hpx;
        t = j / hpx;
    } else {
        head = (int)blockIdx.x % a.n_heads;
        t = (int)blockIdx.x / a.n_heads;
    }
    const int qt = a.causal ? n_qt - 1 - t : t;
    const int kvh = (int)(((long long)head * a.n_kv_heads) / a.n_heads);
    int q_begin = 0, q_len = a.q_len, kv_len = a.kv_len;
    const int32_t* table = nullptr;
    if constexpr (PAGED) {
        const int s = blockIdx.z;
        q_begin = a.cu_q[s];
        q_len = a.cu_q[s + 1] - q_begin;
        kv_len = a.ctx_lens[s];
        if (q_begin < 0 || q_len <= 0 || q_begin + q_len > a.n_q_rows) return;
        if (kv_len > a.max_blocks * QL_PAGE_SIZE) kv_len = a.max_blocks * QL_PAGE_SIZE;
        table = a.block_tables + (size_t)s * a.max_blocks;
    }
    const int q0 = qt * kBQ;
    if (q0 >= q_len) return;   // workgroup-uniform
    if (kv_len < 0) kv_len = 0;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int col = lane & 31;   // this lane's query within the wavefront
    const int hh = lane >> 5;    // which 8-wide half of an MFMA k-step the lane feeds
    const int qi = q0 + wave * 32 + col;     // query index within the sequence
    const int pos_base = kv_len - q_len;     // absolute position of query 0
    const int qpos = pos_base + qi;
    const bool q_valid = qi < q_len;

    // keys this workgroup needs
    int kv_hi = kv_len;
    if (a.causal) {
        const int last = pos_base + min(q_len, q0 + kBQ) - 1;
        kv_hi = min(kv_len, last + 1);
    }
    if (kv_hi < 0) kv_hi = 0;
    const int n_tiles = (kv_hi + kBK - 1) / kBK;
    const int wave_last_pos = pos_base + min(q0 + wave * 32 + 31, q_len - 1);
    const bool wave_has_q = q0 + wave * 32 < q_len;

    // Q^T operand: lane holds Q[query=col][d = 16*kk + 8*hh + 0..7]
    half8 qf[NKK];
    {
        const _Float16* qrow = a.q + (size_t)(q_begin + (q_valid ? qi : 0)) * a.q_stride + (size_t)head * HD;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
            qf[kk] = q_valid ? *reinterpret_cast<const half8*>(qrow + 16 * kk + 8 * hh) : half8{};
    }

    floatx16 o[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) o[i] = floatx16{};
    float m_run = -FLT_MAX, l_run = 0.0f;
    const float cl2 = a.cl2;

    // a valid, aligned address for the loads of missing key rows: this
    // sequence's first query row
    const uintptr_t dummy = reinterpret_cast<uintptr_t>(a.q + (size_t)q_begin * a.q_stride);
    TileRegs<HD, PAGED> regs;
    if (n_tiles > 0) {
        fetch_tile<HD, PAGED>(regs, a, table, kvh, 0, kv_len, dummy);
        stash_tile<HD, PAGED>(regs, smem, smem + T::K_ELEMS);
    }
    __syncthreads();

    for (int t = 0; t < n_tiles; ++t) {
        const int kv0 = t * kBK;
        const bool more = t + 1 < n_tiles;
        if (more) fetch_tile<HD, PAGED>(regs, a, table, kvh, kv0 + kBK, kv_len, dummy);
        const _Float16* sk = smem + (t & 1) * T::STAGE;
        const _Float16* sv = sk + T::K_ELEMS;

        // a wavefront with no queries, or whose queries all precede this tile,
        // has nothing to add
        const bool active = wave_has_q && (!a.causal || kv0 <= wave_last_pos);
        if (active) {
            floatx16 s[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                s[kb] = floatx16{};
                const _Float16* krow = sk + (kb * 32 + col) * T::KS + 8 * hh;
#pragma unroll
                for (int kk = 0; kk < NKK; ++kk) {
                    const half8 kf = *reinterpret_cast<const half8*>(krow + 16 * kk);
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[kk], s[kb], 0, 0, 0);
                }
            }
            // mask: lane holds S^T[key = kv0 + 32*kb + 8*(i/4) + 4*hh + i%4][query col]
            const bool need_mask = kv0 + kBK > kv_len || (a.causal && kv0 + kBK - 1 > pos_base + q0 + wave * 32);
            float mt = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    if (need_mask) {
                        const int j = kv0 + 32 * kb + 8 * (i >> 2) + 4 * hh + (i & 3);
                        const bool ok = j < kv_len && (!a.causal || j <= qpos);
                        s[kb][i] = ok ? s[kb][i] : -INFINITY;
                    }
                    mt = fmaxf(mt, s[kb][i]);
                }
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
            // Rescale only when some query's max grew by more than 2^8 in the
            // exponent: until then the stale offset keeps p <= 256 (exact
            // enough in binary16) and O/l is unchanged, since the offset cancels.
            const float m_cand = fmaxf(m_run, mt);
            if (__any((m_cand - m_run) * cl2 > 8.0f)) {
                const float alpha = __builtin_amdgcn_exp2f((m_run - m_cand) * cl2);
#pragma unroll
                for (int db = 0; db < NDB; ++db) o[db] *= alpha;
                l_run *= alpha;
                m_run = m_cand;
            }
            const float moff = m_run * cl2;
            half8 pf[2][2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[kb][i], cl2, -moff));
                    pf[kb][i >> 3][i & 7] = from_f32<_Float16>(p);
                }
            }
            // row sum of the binary16 weights, accumulated in fp32 (v_dot2 with ones)
            float lsum = l_run;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int e = 0; e < 8; e += 2)
                        lsum = __builtin_amdgcn_fdot2(half2v{pf[kb][c][e], pf[kb][c][e + 1]},
                                                      half2v{1.0f16, 1.0f16}, lsum, false);
            l_run = lsum;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const _Float16* vrow = sv + (db * 32 + col) * T::VS + 4 * hh;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const half4 lo = *reinterpret_cast<const half4*>(vrow + 32 * kb + 16 * c);
                        const half4 hi = *reinterpret_cast<const half4*>(vrow + 32 * kb + 16 * c + 8);
                        const half8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[kb][c], o[db], 0, 0, 0);
                    }
                }
            }
        }
        if (more) stash_tile<HD, PAGED>(regs, smem + ((t + 1) & 1) * T::STAGE,
                                        smem + ((t + 1) & 1) * T::STAGE + T::K_ELEMS);
        __syncthreads();
    }

    if (!q_valid) return;
    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    const float inv_den = 1.0f / (l_tot + 1e-8f);
    _Float16* orow = a.out + (size_t)(q_begin + qi) * a.o_stride + (size_t)head * HD;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            half4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = from_f32<_Float16>(o[db][4 * g + e] * inv_den);
            *reinterpret_cast<half4*>(orow + db * 32 + 8 * g + 4 * hh) = r;
        }
    }
}

float scale_log2e(int head_dim) {
    const float scale = 1.0f / sqrtf((float)head_dim);   // the reference's scale, fp32
    return (float)((double)scale * 1.4426950408889634);
}

template <bool PAGED>
hipError_t launch_attn(const AttnArgs& a, int head_dim, unsigned gx, unsigned gz, hipStream_t stream) {
    QL_CHECK_ARG((long long)gx * a.n_heads <= INT32_MAX);
    const dim3 grid(gx * (unsigned)a.n_heads, 1, gz);
    if (head_dim == 128) {
        hipLaunchKernelGGL((attn_fwd<128, PAGED>), grid, dim3(kAttnThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL((attn_fwd<64, PAGED>), grid, dim3(kAttnThreads), 0, stream, a);
    }
    return hipGetLastError();
}

bool aligned_rows(const void* p, int64_t stride) {
    return qlh::aligned16(p) && stride % 8 == 0;
}

}  // namespace

extern "C" hipError_t ql_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                       uint16_t* out, int q_len, int kv_len, int n_heads,
                                       int n_kv_heads, int head_dim, int64_t q_row_stride,
                                       int64_t kv_row_stride, int64_t out_row_stride, int causal,
                                       hipStream_t stream) {
    QL_CHECK_ARG(q_len >= 0 && kv_len >= 0 && n_heads > 0 && n_kv_heads > 0);
    QL_CHECK_ARG(n_kv_heads <= n_heads && n_heads <= 65535);
    QL_CHECK_ARG(head_dim == 64 || head_dim == 128);
    QL_CHECK_ARG(q_row_stride >= (int64_t)n_heads * head_dim);
    QL_CHECK_ARG(out_row_stride >= (int64_t)n_heads * head_dim);
    QL_CHECK_ARG(kv_row_stride >= (int64_t)n_kv_heads * head_dim);
    if (q_len == 0) return hipSuccess;
    QL_CHECK_ARG(q && out && (kv_len == 0 || (k && v)));
    QL_CHECK_ARG(aligned_rows(q, q_row_stride) && aligned_rows(out, out_row_stride));
    QL_CHECK_ARG(kv_len == 0 || (aligned_rows(k, kv_row_stride) && aligned_rows(v, kv_row_stride)));
    AttnArgs a{};
    a.q = reinterpret_cast<const _Float16*>(q);
    a.out = reinterpret_cast<_Float16*>(out);
    a.q_stride = q_row_stride;
    a.o_stride = out_row_stride;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.cl2 = scale_log2e(head_dim);
    a.causal = causal != 0;
    a.q_len = q_len;
    a.kv_len = kv_len;
    a.k = reinterpret_cast<const _Float16*>(k);
    a.v = reinterpret_cast<const _Float16*>(v);
    a.kv_stride = kv_row_stride;
    return launch_attn<false>(a, head_dim, qlh::blocks_for(q_len, kBQ), 1, stream);
}

extern "C" hipError_t ql_flash_attention_f16(const uint16_t* q, const uint16_t* k,
                                             const uint16_t* v, uint16_t* out, int seq_len,
                                             int n_heads, int n_kv_heads, int head_dim,
                                             int causal, hipStream_t stream) {
    QL_CHECK_ARG(n_heads > 0 && n_kv_heads > 0);
    const int64_t qs = (int64_t)n_heads * head_dim, ks = (int64_t)n_kv_heads * head_dim;
    return ql_attention_f16(q, k, v, out, seq_len, seq_len, n_heads, n_kv_heads, head_dim, qs, ks,
                            qs, causal, stream);
}

extern "C" hipError_t ql_paged_attention_f16(
    const uint16_t* q, uint16_t* out, int64_t q_row_stride, int64_t out_row_stride, int n_q_rows,
    int n_seqs, const int32_t* cu_q_lens, const int32_t* ctx_lens, int max_q_len,
    const int32_t* block_tables, int max_blocks_per_seq, const uint16_t* const* k_blocks,
    const uint16_t* const* v_blocks, int n_blocks, int layer, int n_layers, int n_heads,
    int n_kv_heads, int head_dim, int causal, hipStream_t stream) {
    QL_CHECK_ARG(n_seqs >= 0 && n_seqs <= 65535 && max_q_len >= 0 && n_q_rows >= 0);
    QL_CHECK_ARG(n_heads > 0 && n_kv_heads > 0 && n_kv_heads <= n_heads && n_heads <= 65535);
    QL_CHECK_ARG(head_dim == 64 || head_dim == 128);
    QL_CHECK_ARG(n_layers > 0 && layer >= 0 && layer < n_layers);
    QL_CHECK_ARG(max_blocks_per_seq >= 0 && max_blocks_per_seq <= (INT32_MAX / QL_PAGE_SIZE));
    QL_CHECK_ARG(n_blocks >= 0);
    QL_CHECK_ARG(q_row_stride >= (int64_t)n_heads * head_dim);
    QL_CHECK_ARG(out_row_stride >= (int64_t)n_heads * head_dim);
    if (n_seqs == 0 || max_q_len == 0 || n_q_rows == 0) return hipSuccess;
    QL_CHECK_ARG(q && out && cu_q_lens && ctx_lens);
    QL_CHECK_ARG(max_blocks_per_seq == 0 || (block_tables && k_blocks && v_blocks));
    QL_CHECK_ARG(aligned_rows(q, q_row_stride) && aligned_rows(out, out_row_stride));
    AttnArgs a{};
    a.q = reinterpret_cast<const _Float16*>(q);
    a.out = reinterpret_cast<_Float16*>(out);
    a.q_stride = q_row_stride;
    a.o_stride = out_row_stride;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.cl2 = scale_log2e(head_dim);
    a.causal = causal != 0;
    a.kb = reinterpret_cast<const _Float16* const*>(k_blocks);
    a.vb = reinterpret_cast<const _Float16* const*>(v_blocks);
    a.n_blocks = n_blocks;
    a.block_tables = block_tables;
    a.max_blocks = max_blocks_per_seq;
    a.cu_q = cu_q_lens;
    a.ctx_lens = ctx_lens;
    a.n_q_rows = n_q_rows;
    a.layer = layer;
    return launch_attn<true>(a, head_dim, qlh::blocks_for(max_q_len, kBQ), (unsigned)n_seqs, stream);
}
