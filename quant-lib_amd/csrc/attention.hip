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
// chunked prefill), head_dim may be 64 or 128 on the matrix cores (the
// reference's tiles hold 64) and any other value up to 64 on a vector-ALU
// kernel (attn_small), rows may be strided, and K/V may live in 16-token pages.
//
// Work decomposition (prefill).  One workgroup = 4 wavefronts = 128
// consecutive queries of one query head; each wavefront owns 32 queries.  Keys
// stream through LDS in tiles of 64, loaded straight from global memory into
// the other of two LDS stages while the current tile is multiplied.  Per tile
// and wavefront:
//   S^T (64 keys x 32 queries) = K . Q^T    -- v_mfma_f32_32x32x16_f16
//   O^T (d x 32 queries)      += V^T . P^T
// Computing the transposed products makes every lane own one query column:
// the running max/sum are per lane, rescaling O is a per-lane multiply, and
// the P^T operand of the second product is the lane's own S^T registers
// narrowed to fp16 (no shuffles).  The contraction order of the keys inside
// one 16-key MFMA step is permuted identically in both operands, which the
// sum does not see.  V stays row-major in LDS; the V^T operand is two
// transposing 8-byte LDS reads per MFMA.
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

#include <mutex>

// Key-split partials of ql_paged_decode_attention_f16_noalloc: a library-owned
// device array, one copy per GPU, reached through its device address (resolved
// once per device by hipGetSymbolAddress in decode_scratch()); host code never
// passes the array's name itself to a kernel or a copy.
constexpr size_t kDecodeScratchBytes = (size_t)QL_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kDecodeScratchBytes / sizeof(float)];

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

// Pair reductions across lanes l and l ^ 32 (l ^ 16) without an LDS round
// trip: gfx950's v_permlane32_swap (v_permlane16_swap) applied to a value and
// itself hands every lane both values of its pair, the lower half's first, so
// both lanes of a pair compute the same bits (__shfl_xor compiled to
// ds_bpermute plus a wait on every outstanding LDS read; measured 2-3% of the
// prefill kernel, bit-identical).
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

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
    // decode (one query row per sequence)
    int n_split;                   // key splits per (sequence, KV head)
    float* ws;                     // [n_seqs, n_heads, n_split, head_dim + 2] partials
    int hd;                        // head_dim (read by attn_small and the narrow prefill)
};

// Page bases of the consecutive 16-key pages of one decode step (up to 4): the
// address of (block, layer, slot 0, this KV head) for K and V, or 0 where the
// table entry is missing or out of range.  The lookups use VECTOR loads whose
// results are broadcast with v_readlane: scalar loads would share the LDS wait
// counter, so every LDS wait would also wait for the lookup.
struct Pages {
    uintptr_t k[4], v[4];
    bool misaligned;
};

__device__ __forceinline__ uintptr_t readlane64(uintptr_t x, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), l);
    return ((uintptr_t)hi << 32) | lo;
}

// Three-stage lookup of the page bases of COUNT consecutive pages: (1) lane p
// loads table entry first+p, (2) it loads the two block pointers, (3) the
// results are broadcast with v_readlane (decode).  Each stage's result is
// consumed one step later, at a point where the kernel waits for its K/V loads
// anyway, so the dependent table -> pointer chain never stalls the step in flight.
// A null block pointer in device memory: the pointer lookup of a missing table
// entry reads it, so the lookup is one unconditional load.
__device__ const _Float16* const kNoBlock = nullptr;
// Likewise an absent table entry: lanes past the pages wanted (or the table's
// end) read this instead, so the entry lookup is one unconditional load too.
__device__ const int32_t kNoEntry = -1;

template <bool PAGED, int COUNT>
struct PagePipe {
    int b = -1;                 // stage 1: table entry of page first + lane%4 (or -1)
    uintptr_t kp = 0, vp = 0;   // stage 2: block pointers as stored (0 = missing)

    // No branch around the load: with one, the compiler's wait before a later
    // use of any earlier load could not count the loads issued after it and
    // would wait for all of them.
    __device__ __forceinline__ void entries(const AttnArgs& a, const int32_t* table, int first) {
        if constexpr (PAGED) {
            const int p = (int)(threadIdx.x & 3);
            const int t = first + p;
            const bool ok = p < COUNT && t < a.max_blocks;
            typedef const int32_t __attribute__((address_space(1)))* GlobalEntryPtr;
            const int e = *(GlobalEntryPtr)(ok ? table + t : &kNoEntry);
            b = ok ? e : -1;
        }
    }
    // The loaded pointers are used only by bases(), one tile later: nothing here
    // consumes them, so no wait for these loads is placed before the next tile's work.
    __device__ __forceinline__ void pointers(const AttnArgs& a) {
        if constexpr (PAGED) {
            const bool ok = b >= 0 && b < a.n_blocks;
            typedef const _Float16* const __attribute__((address_space(1)))* GlobalBlockPtr;
            kp = reinterpret_cast<uintptr_t>(*(GlobalBlockPtr)(ok ? a.kb + b : &kNoBlock));
            vp = reinterpret_cast<uintptr_t>(*(GlobalBlockPtr)(ok ? a.vb + b : &kNoBlock));
        }
    }
    // page bases: (block, layer, slot 0, KV head kvh)
    __device__ __forceinline__ Pages bases(const AttnArgs& a, int kvh, int hd) const {
        Pages pg{};
        if constexpr (PAGED) {
            const uintptr_t head = ((uintptr_t)a.layer * QL_PAGE_SIZE * a.n_kv_heads + kvh) * hd * sizeof(_Float16);
            uintptr_t any = 0;
#pragma unroll
            for (int q = 0; q < COUNT; ++q) {
                const uintptr_t k = readlane64(kp, q), v = readlane64(vp, q);
                pg.k[q] = k ? k + head : 0;
                pg.v[q] = v ? v + head : 0;
                any |= pg.k[q] | pg.v[q];
            }
            pg.misaligned = (any & 15) != 0;
        }
        return pg;
    }
};

// The page lookups below are offset by divergent_zero(): a load whose address
// is uniform over the wavefront has its result moved to scalar registers right
// after it is issued, which waits for that load and for every load issued
// before it; offset by the zero, the lookups keep their results in vector
// registers until bases() moves them, after the tile's products.

// Lookup of the base of this wavefront's page of a prefill tile: (1) the table
// entry, (2) the two block pointers, (3) the head offset; each stage's result is
// consumed one tile later, where the kernel waits for its K/V loads anyway.
// Every lane loads the same addresses; bases() moves the result to scalar
// registers.
template <bool PAGED>
struct WavePagePipe {
    int b = -1;
    uintptr_t kp = 0, vp = 0;
    int z = 0;

    __device__ __forceinline__ void init() {
        if constexpr (PAGED) z = divergent_zero();
    }
    __device__ __forceinline__ void entry(const AttnArgs& a, const int32_t* table, int t) {
        if constexpr (PAGED) {
            typedef const int32_t __attribute__((address_space(1)))* GlobalEntryPtr;
            b = *(GlobalEntryPtr)((t < a.max_blocks ? table + t : &kNoEntry) + z);
        }
    }
    __device__ __forceinline__ void pointers(const AttnArgs& a) {
        if constexpr (PAGED) {
            const bool ok = b >= 0 && b < a.n_blocks;
            typedef const _Float16* const __attribute__((address_space(1)))* GlobalBlockPtr;
            kp = reinterpret_cast<uintptr_t>(*(GlobalBlockPtr)(ok ? a.kb + b : &kNoBlock));
            vp = reinterpret_cast<uintptr_t>(*(GlobalBlockPtr)(ok ? a.vb + b : &kNoBlock));
        }
    }
    __device__ __forceinline__ void bases(const AttnArgs& a, int kvh, int hd, uintptr_t& k, uintptr_t& v) const {
        if constexpr (PAGED) {
            const uintptr_t head = ((uintptr_t)a.layer * QL_PAGE_SIZE * a.n_kv_heads + kvh) * hd * sizeof(_Float16);
            const uintptr_t ks = readlane64(kp, 0), vs = readlane64(vp, 0);
            k = ks ? ks + head : 0;
            v = vs ? vs + head : 0;
        }
    }
};

typedef const __attribute__((address_space(1))) half8* GlobalHalf8Ptr;
typedef uint32_t u32x4g __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4g* GlobalU4Ptr;

// Streaming (nontemporal) 16-byte global load.
__device__ __forceinline__ half8 load_nt16(uintptr_t p) {
    return __builtin_bit_cast(half8, __builtin_nontemporal_load((GlobalU4Ptr)p));
}

// 16 bytes of chunk ch of a key row (row == 0: missing key -> zeros) for page
// pointers that are not 16-byte aligned (caller-provided pools): element-wise
// loads.  Used for a whole page, chosen once per wavefront.
__device__ __forceinline__ half8 load_chunk_unaligned(uintptr_t row, int ch) {
    half8 r{};
    if (row != 0) {
        // global address space: generic (flat) loads would also count against the
        // LDS counter, so every later LDS wait would wait for them
        const __attribute__((address_space(1))) _Float16* e =
            reinterpret_cast<const __attribute__((address_space(1))) _Float16*>(row + 16 * (uintptr_t)ch);
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = e[i];
    }
    return r;
}

// ---- prefill key tiles: global memory straight into LDS ------------------------------------
//
// gfx950's global_load_lds_dwordx4: lane l of one load instruction writes its 16
// bytes at the instruction's (wave-uniform) LDS base + 16*l, so no registers hold
// a tile in flight and nothing is copied from registers to LDS.  K and V tiles
// are stored row-major with unpadded rows; the 16-byte chunk c of key row r
// sits in slot c ^ tile_swz(r), so both the K fragment reads and the
// transposing V reads spread over all banks.  Keys at or past kv_len, and keys of a page missing
// from the block table, load a row of zeros (kZeroRow).
__device__ __attribute__((aligned(16))) _Float16 kZeroRow[128] = {};

// Chunk swizzle of key row r: a permutation of the row-number bits that sets the
// LDS bank group (the 16-byte slot within a 256-byte bank line).  K fragment
// reads (16 consecutive keys, one chunk each) need 16 (HD 64: 8 per row parity)
// distinct values over consecutive rows: any bit permutation gives that.  The
// transposing V reads of one instruction cover rows R + 0..3 (R = 4*hh mod 16)
// and 4 consecutive chunks (2 per 16-lane group): the row's low two bits go to
// the slot's high bits and hh to slot bit 1, so each 32-lane half of the
// instruction, whichever halves the hardware pairs, covers all 64 banks once.
// (HD 128 rows span one bank line; HD 64 rows two, split by the row parity.)
template <int HD>
__device__ __forceinline__ int tile_swz(int r) {
    if constexpr (HD == 128) return ((r & 3) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);
    const int t = (r >> 1) & 7;   // row pair within 16 rows
    return ((t & 1) << 2) | (t & 2) | ((t >> 2) & 1);
}

template <int HD>
struct KvTile {
    static constexpr int CH = HD / 8;                          // 16-byte chunks per key row
    static constexpr int ELEMS = kBK * HD;                     // one K (or V) tile, halfs
    static constexpr int LOADS = kBK * CH / kAttnThreads;      // chunks per thread per tile
    static constexpr int PAGE_SLOTS = QL_PAGE_SIZE * CH;       // slots of one 16-key page
    static_assert(LOADS * kAttnThreads == kBK * CH, "tile split");
    static_assert(PAGE_SLOTS % kWave == 0, "one load instruction stays inside one page");
    static_assert(HD <= 128, "kZeroRow covers one key row");
};

// Load i of a lane fills slot (i*4 + wave)*64 + lane of the stage, i.e. key row
// r = slot / CH, chunk (slot % CH) ^ tile_swz(r).
__device__ __forceinline__ void lds_load16(const void* src, _Float16* stage, int base_slot) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(stage + base_slot * 8), 16, 0,
                                     0);
}

// Paged tiles: wavefront w loads page w of the tile (key rows 16w .. 16w+15)
// with its LOADS instructions, so each wavefront needs the base of one page
// only and keeps it in its own registers.  Load i of a lane fills slot
// (w*LOADS + i)*64 + lane, i.e. key row r = slot / CH, chunk (slot % CH) ^
// tile_swz(r), row r % 16 of the page.  CHECKED: keys past kv_len and a missing
// page read kZeroRow.
template <int HD, bool CHECKED, bool NARROW = false>
__device__ __forceinline__ void load_wave_page(_Float16* sk, _Float16* sv, const AttnArgs& a, uintptr_t pk,
                                               uintptr_t pv, int kv0, int kv_len, int wave, int lane) {
    using T = KvTile<HD>;
    const int hd = NARROW ? a.hd : HD;
#pragma unroll
    for (int i = 0; i < T::LOADS; ++i) {
        const int base = (wave * T::LOADS + i) * kWave, slot = base + lane;
        const int r = slot / T::CH, c = (slot % T::CH) ^ tile_swz<HD>(r);
        const uintptr_t off =
            (uintptr_t)(r & (QL_PAGE_SIZE - 1)) * (uintptr_t)a.n_kv_heads * hd * sizeof(_Float16) + 16u * c;
        uintptr_t kg = pk + off, vg = pv + off;
        if constexpr (CHECKED || NARROW) {
            const uintptr_t zero = reinterpret_cast<uintptr_t>(kZeroRow) + 16u * c;
            const bool ok = (!CHECKED || kv0 + r < kv_len) && (!NARROW || c * 8 < hd);
            kg = ok && pk != 0 ? kg : zero;
            vg = ok && pv != 0 ? vg : zero;
        }
        lds_load16(reinterpret_cast<const void*>(kg), sk, base);
        lds_load16(reinterpret_cast<const void*>(vg), sv, base);
    }
}

// Issue the loads of key tile [kv0, kv0 + 64) of KV head kvh into sk (K) and sv
// (V).  Paged: pk / pv are the bases of this wavefront's page (0: missing); a
// full page takes the unchecked path, page bases that are not 16-byte aligned
// (caller-provided pools) element-wise loads and LDS stores.  Each branch is
// uniform over the wavefront.
// NARROW (HD 64): heads of a.hd < 64 elements (a multiple of 8); the 16-byte
// chunks past a.hd load the zero row, so the tile holds the heads zero-padded to 64.
template <int HD, bool PAGED, bool NARROW = false>
__device__ __forceinline__ void load_tile(_Float16* sk, _Float16* sv, const AttnArgs& a, uintptr_t pk,
                                          uintptr_t pv, int kvh, int kv0, int kv_len, int wave, int lane) {
    using T = KvTile<HD>;
    if constexpr (!PAGED) {   // rows 16-byte aligned (checked by the entry points)
        const int hd = NARROW ? a.hd : HD;
#pragma unroll
        for (int i = 0; i < T::LOADS; ++i) {
            const int base = (i * kAttnWaves + wave) * kWave, slot = base + lane;
            const int r = slot / T::CH, c = (slot % T::CH) ^ tile_swz<HD>(r);
            const int j = kv0 + r;
            const size_t off = (size_t)j * (size_t)a.kv_stride + (size_t)kvh * hd + (size_t)c * 8;
            const bool ok = j < kv_len && (!NARROW || c * 8 < hd);
            lds_load16(ok ? a.k + off : kZeroRow + c * 8, sk, base);
            lds_load16(ok ? a.v + off : kZeroRow + c * 8, sv, base);
        }
    } else if (((pk | pv) & 15) != 0) {
        const int hd = NARROW ? a.hd : HD;
#pragma unroll
        for (int i = 0; i < T::LOADS; ++i) {
            const int slot = (wave * T::LOADS + i) * kWave + lane;
            const int r = slot / T::CH, c = (slot % T::CH) ^ tile_swz<HD>(r);
            const uintptr_t off =
                (uintptr_t)(r & (QL_PAGE_SIZE - 1)) * (uintptr_t)a.n_kv_heads * hd * sizeof(_Float16) + 16u * c;
            const uintptr_t zero = reinterpret_cast<uintptr_t>(kZeroRow) + 16u * c;
            const bool ok = kv0 + r < kv_len && (!NARROW || c * 8 < hd);
            *reinterpret_cast<half8*>(sk + slot * 8) = load_chunk_unaligned(ok && pk != 0 ? pk + off : zero, 0);
            *reinterpret_cast<half8*>(sv + slot * 8) = load_chunk_unaligned(ok && pv != 0 ? pv + off : zero, 0);
        }
    } else if (kv0 + (wave + 1) * QL_PAGE_SIZE <= kv_len && pk != 0 && pv != 0) {
        load_wave_page<HD, false, NARROW>(sk, sv, a, pk, pv, kv0, kv_len, wave, lane);
    } else {
        load_wave_page<HD, true, NARROW>(sk, sv, a, pk, pv, kv0, kv_len, wave, lane);
    }
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at their maxima): this thread's
// direct-to-LDS loads have landed.
__device__ __forceinline__ void wait_tile_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

typedef short short4v __attribute__((ext_vector_type(4)));

// Transposing LDS read (ds_read_b64_tr_b16): in each 16-lane group, lane i
// receives element i%4 of the 8 bytes addressed by lanes 4e + i/4, e = 0..3.
__device__ __forceinline__ half4 lds_read_tr4(const _Float16* p) {
    const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) short4v*)(p));
    return __builtin_bit_cast(half4, r);
}

// Work item of a prefill workgroup: (query head, query tile).  Consecutive
// workgroup ids go to the 8 XCDs in turn; when the heads split evenly over the
// XCDs, each XCD is given its own contiguous run of heads (so the K/V rows of
// their shared KV heads stay in that XCD's L2).  Causal: heavy (late) query
// tiles first.
__device__ __forceinline__ void prefill_item(const AttnArgs& a, int& head, int& qt) {
    const int n_qt = (int)gridDim.x / a.n_heads;
    int t;
    if (a.n_heads % 8 == 0) {
        const int hpx = a.n_heads / 8, xcd = (int)blockIdx.x & 7, j = (int)blockIdx.x >> 3;
        head = xcd * hpx + j % hpx;
        t = j / hpx;
    } else {
        head = (int)blockIdx.x % a.n_heads;
        t = (int)blockIdx.x / a.n_heads;
    }
    qt = a.causal ? n_qt - 1 - t : t;
}

// Q^T operand: lane holds Q[query][d = 16*kk + 8*hh + 0..7] (zeros past the last query).
template <int HD>
__device__ __forceinline__ void load_q_operand(half8 (&qf)[HD / 16], const _Float16* qrow, bool valid, int hh,
                                               int hd = HD) {
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk)
        qf[kk] = valid && 16 * kk + 8 * hh < hd ? *reinterpret_cast<const half8*>(qrow + 16 * kk + 8 * hh) : half8{};
}

// One wavefront's online-softmax step over a 64-key tile, given its scores
// s[kb] = S^T block kb (lane holds S^T[key = kv0 + 32*kb + 8*(i/4) + 4*hh + i%4]
// [its query]): masks keys past kv_len and (causal) after the query, raises the
// running maximum when needed, forms the binary16 weights, adds their fp32 sum to
// l_run and accumulates P V into O^T.  v_operand(db, kb, c) returns the V^T
// operand of rows d = 32*db + 0..31 over the keys of pf[kb][c].
template <int HD, class VOperand>
__device__ __forceinline__ void softmax_pv(floatx16 (&s)[2], floatx16 (&o)[HD / 32], float& m_run, float& l_run,
                                           float cl2, bool causal, int kv0, int kv_len, int qpos,
                                           int wave_first_pos, int hh, VOperand v_operand) {
    constexpr int NDB = HD / 32;
    const bool need_mask = kv0 + kBK > kv_len || (causal && kv0 + kBK - 1 > wave_first_pos);
    if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int j = kv0 + 32 * kb + 8 * (i >> 2) + 4 * hh + (i & 3);
                const bool ok = j < kv_len && (!causal || j <= qpos);
                s[kb][i] = ok ? s[kb][i] : -INFINITY;
            }
        }
    }
    // maximum as a tree: four independent chains of eight, then combined
    float mq[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        mq[c] = fmaxf(s[c >> 1][8 * (c & 1)], s[c >> 1][8 * (c & 1) + 1]);
#pragma unroll
        for (int i = 2; i < 8; ++i) mq[c] = fmaxf(mq[c], s[c >> 1][8 * (c & 1) + i]);
    }
    float mt = fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]));
    mt = max_xor32(mt);
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
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int c = 0; c < 2; ++c)
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v_operand(db, kb, c), pf[kb][c], o[db], 0, 0, 0);
        }
    }
}

// O = O^T / l for the lane's query (both 8-key halves of the sum combined).
template <int HD>
__device__ __forceinline__ void store_o(const floatx16 (&o)[HD / 32], float l_run, _Float16* orow, int hh,
                                        int hd = HD) {
    const float l_tot = sum_xor32(l_run);
    const float inv_den = 1.0f / (l_tot + 1e-8f);
#pragma unroll
    for (int db = 0; db < HD / 32; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            half4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = from_f32<_Float16>(o[db][4 * g + e] * inv_den);
            if (db * 32 + 8 * g + 4 * hh < hd)   // narrow heads (a multiple of 8): whole 4-element runs
                *reinterpret_cast<half4*>(orow + db * 32 + 8 * g + 4 * hh) = r;
        }
    }
}

// One prefill workgroup: 128 queries of one query head against every key they
// see, in 64-key tiles through two LDS stages.  The stages are two distinct
// arrays and the tile loop is unrolled by two, so no wait for the loads into
// one stage is placed before the reads of the other.  Paged K/V: wavefront w
// loads page w of each tile, and the base of its page of tile t+2 is looked up
// (WavePagePipe) while tile t is multiplied.
template <int HD, bool PAGED, bool NARROW = false>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_fwd(AttnArgs a) {
    using T = KvTile<HD>;
    constexpr int NKK = HD / 16;   // MFMA steps over d for S^T
    constexpr int NDB = HD / 32;   // 32-row blocks of O^T
    __shared__ __attribute__((aligned(16))) _Float16 sk0[T::ELEMS];
    __shared__ __attribute__((aligned(16))) _Float16 sv0[T::ELEMS];
    __shared__ __attribute__((aligned(16))) _Float16 sk1[T::ELEMS];
    __shared__ __attribute__((aligned(16))) _Float16 sv1[T::ELEMS];

    int head, qt;
    prefill_item(a, head, qt);
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
    // paged: a scalar wave index makes load_tile's page choice scalar (the
    // compiler's register allocation measured best this way for each layout)
    const int wave = PAGED ? __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave) : (int)threadIdx.x / kWave;
    const int col = lane & 31;   // this lane's query within the wavefront
    const int hh = lane >> 5;    // which 8-wide half of an MFMA k-step the lane feeds
    const int qi = q0 + wave * 32 + col;     // query index within the sequence
    const int pos_base = kv_len - q_len;     // absolute position of query 0
    const int qpos = pos_base + qi;
    const bool q_valid = qi < q_len;

    // keys this workgroup needs
    int kv_hi = kv_len;
    if (a.causal) kv_hi = min(kv_len, pos_base + min(q_len, q0 + kBQ));
    if (kv_hi < 0) kv_hi = 0;
    const int n_tiles = (kv_hi + kBK - 1) / kBK;
    const int wave_first_pos = pos_base + q0 + wave * 32;
    const int wave_last_pos = pos_base + min(q0 + wave * 32 + 31, q_len - 1);
    const bool wave_has_q = q0 + wave * 32 < q_len;

    half8 qf[NKK];
    const int hd = NARROW ? a.hd : HD;   // the heads' width in memory
    load_q_operand<HD>(qf, a.q + (size_t)(q_begin + (q_valid ? qi : 0)) * a.q_stride + (size_t)head * hd,
                       q_valid, hh, hd);
    floatx16 o[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) o[i] = floatx16{};
    float m_run = -FLT_MAX, l_run = 0.0f;
    const int s16 = lane & 15, grp = (lane >> 4) & 1;

    // S^T = K . Q^T and the online-softmax step of one tile held in (sk, sv); a
    // wavefront with no queries, or whose queries all precede the tile, skips it
    auto compute = [&](const _Float16* sk, const _Float16* sv, int kv0) {
        if (!(wave_has_q && (!a.causal || kv0 <= wave_last_pos))) return;
        // Contiguous K/V: the two 32-key blocks' products in turn, each step's K
        // fragments read ahead of its products (PF steps ahead; with them read just
        // before, every product waited for an LDS round trip): HD 128 prefetches two
        // steps, in an order pinned by scheduling groups (the compiler otherwise
        // sinks the reads back); HD 64 one step, which keeps its occupancy at 3
        // wavefronts per SIMD.  Measured on MI355X, same process, bit-identical:
        // C5 prefill 592.7 -> 577.7 us (611.5 -> 600.8 on a slower box), 4096
        // tokens at HD 64 101.8 -> 97.4 us.  The paged kernel measured no gain
        // (635.9 -> 639.7 us) and keeps the plain loop (PF = 0).
        constexpr int PF = PAGED ? 0 : (HD == 128 ? 2 : 1);
        floatx16 s[2];
        const _Float16* krow0 = sk + col * HD;
        const _Float16* krow1 = sk + (32 + col) * HD;
        const int sw0 = tile_swz<HD>(col), sw1 = tile_swz<HD>(32 + col);
        auto kfrag = [&](const _Float16* krow, int sw, int kk) {
            return *reinterpret_cast<const half8*>(krow + 8 * ((2 * kk + hh) ^ sw));
        };
        s[0] = floatx16{};
        s[1] = floatx16{};
        if constexpr (PF == 0) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const _Float16* krow = kb ? krow1 : krow0;
                const int sw = kb ? sw1 : sw0;
#pragma unroll
                for (int kk = 0; kk < NKK; ++kk)
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfrag(krow, sw, kk), qf[kk], s[kb], 0, 0, 0);
            }
        } else if constexpr (PF == 1) {
            half8 ka = kfrag(krow0, sw0, 0), kb = kfrag(krow1, sw1, 0);
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk) {
                half8 na{}, nb{};
                if (kk + 1 < NKK) {
                    na = kfrag(krow0, sw0, kk + 1);
                    nb = kfrag(krow1, sw1, kk + 1);
                }
                s[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qf[kk], s[0], 0, 0, 0);
                s[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb, qf[kk], s[1], 0, 0, 0);
                ka = na;
                kb = nb;
            }
        } else {
            half8 ka[NKK], kb2[NKK];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kk = 0; kk < PF; ++kk) {
                ka[kk] = kfrag(krow0, sw0, kk);
                kb2[kk] = kfrag(krow1, sw1, kk);
            }
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk) {
                if (kk + PF < NKK) {
                    ka[kk + PF] = kfrag(krow0, sw0, kk + PF);
                    kb2[kk + PF] = kfrag(krow1, sw1, kk + PF);
                }
                s[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[kk], qf[kk], s[0], 0, 0, 0);
                s[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kb2[kk], qf[kk], s[1], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * PF, 0);   // DS reads of the first steps
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk) {
                if (kk + PF < NKK) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // DS reads
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                       // MFMA
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // V^T operand: lane s16 of its 16-lane group addresses V[key r][d .. d+3] with
        // key r = 32*kb + 16*c + 4*hh + s16/4 (+8 for the upper half) and
        // d = 32*db + 16*grp + 4*(s16%4); the transposing read hands each lane its column.
        softmax_pv<HD>(s, o, m_run, l_run, a.cl2, a.causal, kv0, kv_len, qpos, wave_first_pos, hh,
                       [&](int db, int kb, int c) {
                           const int d = 32 * db + 16 * grp + 4 * (s16 & 3);
                           const int r0 = 32 * kb + 16 * c + 4 * hh + (s16 >> 2), r1 = r0 + 8;
                           const half4 lo = lds_read_tr4(sv + r0 * HD + 8 * ((d >> 3) ^ tile_swz<HD>(r0)) + (d & 7));
                           const half4 hi = lds_read_tr4(sv + r1 * HD + 8 * ((d >> 3) ^ tile_swz<HD>(r1)) + (d & 7));
                           return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                       });
    };

    constexpr int kTilePages = kBK / QL_PAGE_SIZE;
    static_assert(kTilePages == kAttnWaves && KvTile<HD>::PAGE_SLOTS == KvTile<HD>::LOADS * kWave,
                  "one page per wavefront");
    WavePagePipe<PAGED> pp;
    pp.init();
    uintptr_t pgk = 0, pgv = 0;   // this wavefront's page of the next tile (paged)
    if (n_tiles > 0) {
        uintptr_t k0 = 0, v0 = 0;
        pp.entry(a, table, wave);
        pp.pointers(a);
        pp.bases(a, kvh, hd, k0, v0);
        if (n_tiles > 1) {
            pp.entry(a, table, kTilePages + wave);
            pp.pointers(a);
            pp.bases(a, kvh, hd, pgk, pgv);
        }
        if (n_tiles > 2) pp.entry(a, table, 2 * kTilePages + wave);
        load_tile<HD, PAGED, NARROW>(sk0, sv0, a, k0, v0, kvh, 0, kv_len, wave, lane);
    }
    wait_tile_loads();
    __syncthreads();
    // tile t sits in (sk, sv); tile t+1 is loaded into (nk, nv) meanwhile
    auto step = [&](int t, const _Float16* sk, const _Float16* sv, _Float16* nk, _Float16* nv) {
        const int kv0 = t * kBK;
        if (t + 1 < n_tiles) load_tile<HD, PAGED, NARROW>(nk, nv, a, pgk, pgv, kvh, kv0 + kBK, kv_len, wave, lane);
        if (t + 2 < n_tiles) pp.pointers(a);                                    // tile t+2
        if (t + 3 < n_tiles) pp.entry(a, table, (t + 3) * kTilePages + wave);   // tile t+3
        compute(sk, sv, kv0);
        if (t + 2 < n_tiles) pp.bases(a, kvh, hd, pgk, pgv);
        wait_tile_loads();
        __syncthreads();
    };
    for (int t = 0; t < n_tiles; t += 2) {
        step(t, sk0, sv0, sk1, sv1);
        if (t + 1 >= n_tiles) break;
        step(t + 1, sk1, sv1, sk0, sv0);
    }

    if (!q_valid) return;
    store_o<HD>(o, l_run, a.out + (size_t)(q_begin + qi) * a.o_stride + (size_t)head * hd, hh, hd);
}

// ---- decode: one query row per sequence ------------------------------------------------
//
// One workgroup = (sequence, KV head, key split, chunk of <= 16 query heads).
// The query heads that share the KV head are the 16 columns of
// v_mfma_f32_16x16x32_f16 products, so each K/V row is read once for all of
// them.  The 4 wavefronts stream disjoint 32-key steps of the split.  K and V
// rows are loaded whole: each load instruction covers complete 256-byte head
// rows (16 lanes per row), which streams the pool's interleaved head rows
// markedly faster than the MFMA fragment shape (16 rows x 64 bytes).  The
// rows are double-buffered in registers, then re-laid through wavefront-private
// LDS areas: K row-major with 16-byte slots XOR-swizzled by key (conflict-free
// fragment reads), V transposed (LDS operations of one wavefront complete in
// order, so no barrier is needed there).  S^T = K.Q^T and O^T += V^T.P^T as in the prefill kernel; the
// wavefronts are merged through LDS at the end.  With several splits the
// merged partial (offset m, sum l, unnormalised O) goes to the workspace and
// attn_decode_combine finishes each row.
constexpr int kDecStep = 32;

typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int HD>
struct Dec {
    static constexpr int VS = kDecStep + 4;          // V^T row stride in LDS (halfs)
    static constexpr int VBUF = HD * VS;              // one V^T stage (halfs)
    static constexpr int KBUF = kDecStep * HD;        // one K stage (halfs), swizzled rows
    static constexpr int WAVE_V = VBUF + KBUF;        // LDS per wavefront (halfs)
    static constexpr int NKK = HD / 32;               // k-steps over d for S^T
    static constexpr int NDB = HD / 16;               // 16-row blocks of O^T
    static constexpr int CH = HD / 8;                 // 16-byte chunks per row
    static constexpr int KPL = HD / 16;               // K/V keys per lane per step
    static constexpr int KG = kWave / CH;             // key groups in the V loader
    static_assert(KG * KPL == kDecStep, "K/V step split");
    static_assert(KPL % 4 == 0, "V^T writes are 4 keys wide");
    static constexpr int PART = kAttnWaves * 16 * (HD + 2);   // floats of the merge area
    static constexpr int SMEM_BYTES =
        kAttnWaves * WAVE_V * 2 > PART * 4 ? kAttnWaves * WAVE_V * 2 : PART * 4;
};

// Rows of one step as loaded: chunk lane%CH of keys KPL*(lane/CH) + i.  A key
// with no backing row (past the split's end, or its page missing from the block
// table) was loaded from the dummy row and is zeroed when staged; on a page that
// is not 16-byte aligned every row was, and staging re-reads the rows element by
// element (dec_rows says which, from the step's first key and its pages).
template <int HD>
struct DecK {
    half8 k[Dec<HD>::KPL];
};
template <int HD>
struct DecV {
    half8 v[Dec<HD>::KPL];
};

// Per-lane constants of the decode loaders: byte offset of the lane's K/V chunk
// from its page base (paged) or from the step's first key row (contiguous), and
// the page of the lane's keys.
template <int HD, bool PAGED>
struct DecPlan {
    using T = Dec<HD>;
    uint32_t row_bytes;   // uniform
    uint32_t v_off;       // the lane's first key; key i adds i * row_bytes
    int v_page;
    int key;              // the lane's first key in the step

    // hd: the heads' width in memory (HD, or a narrower contiguous head, decode
    // with the chunks past it zero)
    __device__ __forceinline__ DecPlan(const AttnArgs& a, int kvh, int lane, int hd = HD) {
        row_bytes = PAGED ? (uint32_t)(a.n_kv_heads * hd * sizeof(_Float16))
                          : (uint32_t)(a.kv_stride * sizeof(_Float16));
        const uint32_t head_bytes = PAGED ? 0u : (uint32_t)(kvh * hd * sizeof(_Float16));
        const int ch = lane % T::CH, kg = lane / T::CH;
        key = T::KPL * kg;   // its KPL keys stay inside one page
        v_page = key >> 4;
        v_off = (uint32_t)(PAGED ? (key & 15) : key) * row_bytes + head_bytes + 16u * ch;
    }
};

// The 16 bytes at p for a page pointer that is not 16-byte aligned (caller-
// provided pools): element-wise loads in the global address space (generic
// loads would also count against the LDS counter).
__device__ __forceinline__ half8 load8_unaligned(uintptr_t p) {
    const __attribute__((address_space(1))) _Float16* e =
        reinterpret_cast<const __attribute__((address_space(1))) _Float16*>(p);
    half8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = e[i];
    return r;
}

// K stage: row `key` holds its 16-byte chunk c in slot kt_slot(key, c).  Fragment
// reads (16 lanes = keys 16*kb .. +15, one chunk) then hit 16 distinct bank groups:
// 256-byte rows alias every bank, so the slot varies with key & 15; 128-byte rows
// alternate bank halves, so it varies with (key >> 1) & 7.
template <int HD>
__device__ __forceinline__ int kt_slot(int key, int c) {
    return HD == 128 ? (c ^ (key & 15)) : (c ^ ((key >> 1) & 7));
}

// A step whose 32 keys all exist on present, aligned pages: nothing to zero or
// re-read at staging.
template <bool PAGED>
__device__ __forceinline__ bool dec_full(const uintptr_t* pages, bool misaligned, int k0, int k_end) {
    bool full = k0 + kDecStep <= k_end;
    if constexpr (PAGED) full = full && !misaligned && pages[0] && pages[1];
    return full;
}

// The lane's chunk of its first key in the step at k0 (0 = no page), and which
// of its KPL keys have a row (bit i).
template <int HD, bool PAGED>
__device__ __forceinline__ uintptr_t dec_rows(const AttnArgs& a, const DecPlan<HD, PAGED>& plan,
                                              const uintptr_t* pages, const _Float16* base, int k0,
                                              int k_end, uint32_t& live) {
    using T = Dec<HD>;
    uintptr_t b;
    if constexpr (PAGED) {
        (void)base;
        b = plan.v_page == 0 ? pages[0] : pages[1];
    } else {
        (void)pages;
        b = reinterpret_cast<uintptr_t>(base) + (uintptr_t)k0 * (uintptr_t)a.kv_stride * sizeof(_Float16);
    }
    const int n_in = k_end - (k0 + plan.key);
    uint32_t in = 0;
#pragma unroll
    for (int i = 0; i < T::KPL; ++i) in |= (uint32_t)(i < n_in) << i;
    live = b ? in : 0u;
    return b ? b + plan.v_off : 0;
}

template <int HD, bool PAGED>
__device__ __forceinline__ void dec_stage_k(DecK<HD>& r, _Float16* sk, const AttnArgs& a,
                                            const DecPlan<HD, PAGED>& plan, const Pages& pg, int k0,
                                            int k_end, int lane, int hd = HD) {
    using T = Dec<HD>;
    const int ch = lane % T::CH, kg = lane / T::CH;
    if (!dec_full<PAGED>(pg.k, pg.misaligned, k0, k_end)) {   // wavefront-uniform
        uint32_t live;
        const uintptr_t row = dec_rows<HD, PAGED>(a, plan, pg.k, a.k, k0, k_end, live);
#pragma unroll
        for (int i = 0; i < T::KPL; ++i) {
            if (PAGED && pg.misaligned && ((live >> i) & 1) && ch * 8 < hd)   // chunks past a narrow head stay zero
                r.k[i] = load8_unaligned(row + (uintptr_t)i * plan.row_bytes);
            if (!((live >> i) & 1)) r.k[i] = half8{};
        }
    }
#pragma unroll
    for (int i = 0; i < T::KPL; ++i) {
        const int key = T::KPL * kg + i;
        *reinterpret_cast<half8*>(sk + key * HD + 8 * kt_slot<HD>(key, ch)) = r.k[i];
    }
}

// K and V rows of one step.  Every step issues the same 2*KPL loads, back to
// back and nontemporal (each row is read by one workgroup), with no branch:
// a lane whose page is missing or misaligned reads its chunk of the dummy row
// KPL times; keys past the end read a row that exists (the rest of their page,
// or for contiguous K/V the last key's row), and staging zeroes or re-reads
// them.  (With the checked loads of the last step and of missing pages as a
// separate branch, the compiler's wait before the first product of every step,
// at the join of the two paths, waited for 13 of the 16 rows just issued for
// the next step.)
// NARROW (contiguous HD 64, heads of hd < 64): lanes whose chunk lies past the
// head read the zero row instead, so the staged K and V are the heads zero-padded.
template <int HD, bool PAGED, bool NARROW = false>
__device__ __forceinline__ void dec_fetch_kv(DecK<HD>& rk, DecV<HD>& rv, const AttnArgs& a,
                                             const DecPlan<HD, PAGED>& plan, const Pages& pg,
                                             int k0, int k_end, uintptr_t dummy, int lane, int hd = HD) {
    using T = Dec<HD>;
    uint32_t klive, vlive;
    const uintptr_t krow = dec_rows<HD, PAGED>(a, plan, pg.k, a.k, k0, k_end, klive);
    const uintptr_t vrow = dec_rows<HD, PAGED>(a, plan, pg.v, a.v, k0, k_end, vlive);
    const bool mis = PAGED && pg.misaligned;
    const int n_in = k_end - (k0 + plan.key);
    // rows a lane may read: all KPL of its page (paged), up to the last key (contiguous)
    const int last = PAGED ? T::KPL - 1 : (n_in > 0 ? min(n_in, T::KPL) - 1 : 0);
    const bool kok = krow != 0 && !mis && (PAGED || n_in > 0);
    const bool vok = vrow != 0 && !mis && (PAGED || n_in > 0);
    const bool pad = NARROW && (lane % T::CH) * 8 >= hd;
    const uintptr_t dchunk = pad ? reinterpret_cast<uintptr_t>(kZeroRow) + 16u * (uint32_t)(lane % T::CH)
                                 : dummy + 16u * (uint32_t)(lane % T::CH);
    const uintptr_t kb = kok && !pad ? krow : dchunk, vb = vok && !pad ? vrow : dchunk;
    const uint32_t ks = kok && !pad ? plan.row_bytes : 0u, vs = vok && !pad ? plan.row_bytes : 0u;
    (void)klive;
    (void)vlive;
#pragma unroll
    for (int i = 0; i < T::KPL; ++i) rk.k[i] = load_nt16(kb + (uintptr_t)((uint32_t)min(i, last) * ks));
#pragma unroll
    for (int i = 0; i < T::KPL; ++i) rv.v[i] = load_nt16(vb + (uintptr_t)((uint32_t)min(i, last) * vs));
}

// V^T stage: row d, keys KPL*kg + i.  The 8-byte unit u (4 keys) of row r is
// stored at unit u ^ ((r >> 4) & 7): with the 72-byte row stride both these
// 4-key writes and the operand reads of dec_step hit 16 distinct bank pairs
// per 16 lanes.
__device__ __forceinline__ int vt_unit(int r, int u) { return u ^ ((r >> 4) & 7); }

template <int HD, bool PAGED>
__device__ __forceinline__ void dec_stage_v(DecV<HD>& r, _Float16* sv, const AttnArgs& a,
                                            const DecPlan<HD, PAGED>& plan, const Pages& pg, int k0,
                                            int k_end, int lane, int hd = HD) {
    using T = Dec<HD>;
    const int ch = lane % T::CH, kg = lane / T::CH;
    if (!dec_full<PAGED>(pg.v, pg.misaligned, k0, k_end)) {   // wavefront-uniform
        uint32_t live;
        const uintptr_t row = dec_rows<HD, PAGED>(a, plan, pg.v, a.v, k0, k_end, live);
#pragma unroll
        for (int i = 0; i < T::KPL; ++i) {
            if (PAGED && pg.misaligned && ((live >> i) & 1) && ch * 8 < hd)   // chunks past a narrow head stay zero
                r.v[i] = load8_unaligned(row + (uintptr_t)i * plan.row_bytes);
            if (!((live >> i) & 1)) r.v[i] = half8{};
        }
    }
#pragma unroll
    for (int i = 0; i < T::KPL; i += 4)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int row = ch * 8 + e;
            *reinterpret_cast<half4*>(sv + row * T::VS + 4 * vt_unit(row, (T::KPL * kg + i) >> 2)) =
                half4{r.v[i][e], r.v[i + 1][e], r.v[i + 2][e], r.v[i + 3][e]};
        }
}

struct DecState {
    float m_run, l_run;
};

// One 32-key step: K staged at sk (row-major, swizzled), V^T staged at sv.
template <int HD>
__device__ __forceinline__ void dec_step(const _Float16* sk, const half8* qf, floatx4* o,
                                         DecState& st, const _Float16* sv, int k0, int k_end,
                                         int lane, float cl2) {
    using T = Dec<HD>;
    const int col = lane & 15, hq = lane >> 4;
    floatx4 sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        sc[kb] = floatx4{};
        const int key = 16 * kb + col;
#pragma unroll
        for (int kk = 0; kk < T::NKK; ++kk) {
            // A operand: key, d = 32*kk + 8*hq .. +8 (chunk 4*kk + hq)
            const half8 kf = *reinterpret_cast<const half8*>(sk + key * HD + 8 * kt_slot<HD>(key, 4 * kk + hq));
            sc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[kk], sc[kb], 0, 0, 0);
        }
    }
    // lane holds S^T[key = k0 + 16*kb + 4*hq + i][column col]
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (k0 + kDecStep > k_end) {
                const int j = k0 + 16 * kb + 4 * hq + i;
                sc[kb][i] = j < k_end ? sc[kb][i] : -INFINITY;
            }
            mt = fmaxf(mt, sc[kb][i]);
        }
    mt = max_xor32(max_xor16(mt));
    const float m_cand = fmaxf(st.m_run, mt);
    if (__any((m_cand - st.m_run) * cl2 > 8.0f)) {
        const float alpha = __builtin_amdgcn_exp2f((st.m_run - m_cand) * cl2);
#pragma unroll
        for (int db = 0; db < T::NDB; ++db) o[db] *= alpha;
        st.l_run *= alpha;
        st.m_run = m_cand;
    }
    const float moff = st.m_run * cl2;
    half8 pf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            pf[4 * kb + i] = from_f32<_Float16>(__builtin_amdgcn_exp2f(fmaf(sc[kb][i], cl2, -moff)));
    float lsum = st.l_run;
#pragma unroll
    for (int e = 0; e < 8; e += 2)
        lsum = __builtin_amdgcn_fdot2(half2v{pf[e], pf[e + 1]}, half2v{1.0f16, 1.0f16}, lsum, false);
    st.l_run = lsum;
    // O^T[d][col] += V^T[d][keys] P^T[keys][col]; MFMA k index 8*hq + e maps to
    // key 4*hq + e (e < 4) and 16 + 4*hq + e - 4 (e >= 4), as in pf
#pragma unroll
    for (int db = 0; db < T::NDB; ++db) {
        const int row = 16 * db + col;
        const _Float16* vrow = sv + row * T::VS;
        const half4 lo = *reinterpret_cast<const half4*>(vrow + 4 * vt_unit(row, hq));
        const half4 hi = *reinterpret_cast<const half4*>(vrow + 4 * vt_unit(row, 4 + hq));
        const half8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf, o[db], 0, 0, 0);
    }
}

// Query row, key count and block table of sequence s; false = nothing to do.
template <bool PAGED>
__device__ __forceinline__ bool dec_sequence(const AttnArgs& a, int s, int& q_row, int& kv_len,
                                             const int32_t*& table) {
    q_row = 0;
    kv_len = a.kv_len;
    table = nullptr;
    if constexpr (PAGED) {
        q_row = s;
        if (a.cu_q) {
            q_row = a.cu_q[s];
            if (a.cu_q[s + 1] - q_row != 1) return false;
        }
        if (q_row < 0 || q_row >= a.n_q_rows) return false;
        kv_len = a.ctx_lens[s];
        if (kv_len > a.max_blocks * QL_PAGE_SIZE) kv_len = a.max_blocks * QL_PAGE_SIZE;
        table = a.block_tables + (size_t)s * a.max_blocks;
    }
    if (kv_len < 0) kv_len = 0;
    return true;
}

// NARROW: contiguous K/V with heads of a.hd < 64 (a multiple of 8) on the HD 64
// kernel, zero-padded, one key split.
template <int HD, bool PAGED, bool NARROW = false>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_decode(AttnArgs a) {
    using T = Dec<HD>;
    __shared__ __attribute__((aligned(16))) char smem_raw[T::SMEM_BYTES];
    const int s = blockIdx.z, kvh = blockIdx.y;
    const int sp = (int)blockIdx.x % a.n_split, cg = (int)blockIdx.x / a.n_split;
    // query heads h with h*n_kv_heads/n_heads == kvh: [ceil(kvh*H/Hkv), ceil((kvh+1)*H/Hkv))
    const long long H = a.n_heads, HK = a.n_kv_heads;
    const int h_lo = (int)((kvh * H + HK - 1) / HK);
    const int h_hi = (int)(((kvh + 1) * H + HK - 1) / HK);
    const int hb = h_lo + 16 * cg;
    const int G = min(h_hi, hb + 16) - hb;
    if (G <= 0) return;   // workgroup-uniform
    int q_row, kv_len;
    const int32_t* table;
    if (!dec_sequence<PAGED>(a, s, q_row, kv_len, table)) return;
    const int per = (kv_len + a.n_split - 1) / a.n_split;
    const int chunk = (per + kAttnWaves * kDecStep - 1) / (kAttnWaves * kDecStep) * (kAttnWaves * kDecStep);
    const int k_begin = sp * chunk;
    const int k_end = min(kv_len, k_begin + chunk);
    const int n_steps = k_end > k_begin ? (k_end - k_begin + kDecStep - 1) / kDecStep : 0;

    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int col = lane & 15, hq = lane >> 4;
    const bool col_ok = col < G;
    const int hd = NARROW ? a.hd : HD;   // the heads' width in memory
    half8 qf[T::NKK];
    {
        const _Float16* qrow = a.q + (size_t)q_row * a.q_stride + (size_t)(hb + (col_ok ? col : 0)) * hd;
#pragma unroll
        for (int kk = 0; kk < T::NKK; ++kk)
            qf[kk] = col_ok && 32 * kk + 8 * hq < hd ? *reinterpret_cast<const half8*>(qrow + 32 * kk + 8 * hq)
                                                     : half8{};
    }
    floatx4 o[T::NDB];
#pragma unroll
    for (int i = 0; i < T::NDB; ++i) o[i] = floatx4{};
    DecState st{-FLT_MAX, 0.0f};
    const float cl2 = a.cl2;
    _Float16* sv = reinterpret_cast<_Float16*>(smem_raw) + wave * T::WAVE_V;
    _Float16* sk = sv + T::VBUF;
    const uintptr_t dummy = reinterpret_cast<uintptr_t>(a.q + (size_t)q_row * a.q_stride);

    // wavefront w takes steps w, w+4, w+8, ...: each step stages its K rows
    // (loaded one step earlier) into LDS, then reuses those registers for the
    // next step's K rows; V goes through one register set and is staged as soon
    // as the step has read the previous stage; page bases flow through the
    // 3-stage lookup, one step per stage
    constexpr int kStride = kAttnWaves * kDecStep;
    constexpr int kStepPages = kDecStep / QL_PAGE_SIZE;
    DecK<HD> kr;
    DecV<HD> vr;
    const DecPlan<HD, PAGED> plan(a, kvh, lane, hd);
    PagePipe<PAGED, kStepPages> pp;
    int step = wave;
    Pages pg_next{};
    Pages pg_k{};   // pages of the K rows in kr
    auto page_of = [&](int sidx) { return (k_begin + sidx * kDecStep) >> 4; };
    if (step < n_steps) {
        const int k0 = k_begin + step * kDecStep;
        pp.entries(a, table, page_of(step));
        pp.pointers(a);
        const Pages pg = pp.bases(a, kvh, hd);
        pg_k = pg;
        if (step + kAttnWaves < n_steps) {
            pp.entries(a, table, page_of(step + kAttnWaves));
            pp.pointers(a);
            pg_next = pp.bases(a, kvh, hd);
        }
        if (step + 2 * kAttnWaves < n_steps) pp.entries(a, table, page_of(step + 2 * kAttnWaves));
        dec_fetch_kv<HD, PAGED, NARROW>(kr, vr, a, plan, pg, k0, k_end, dummy, lane, hd);
        dec_stage_v<HD, PAGED>(vr, sv, a, plan, pg, k0, k_end, lane, hd);
    }
    // one step: stage its K rows, prefetch the wavefront's next step into the
    // registers, multiply, then stage the next step's V rows
    // Every load of a step is issued unconditionally (lookups for steps past the
    // end read valid table entries or the null entry, the last step's prefetch
    // reads the dummy row): with a branch around any of them the compiler could
    // not count the loads issued after this step's V rows, and its wait for those
    // rows would wait for the next step's rows too.
    auto run_step = [&]() -> bool {
        const int k0 = k_begin + step * kDecStep;
        const bool more = step + kAttnWaves < n_steps;
        dec_stage_k<HD, PAGED>(kr, sk, a, plan, pg_k, k0, k_end, lane, hd);   // after the previous step's K reads (in order)
        // page lookups first: issued after the K/V rows, their waits would also
        // wait for the rows
        pp.pointers(a);
        pp.entries(a, table, page_of(step + 3 * kAttnWaves));
        dec_fetch_kv<HD, PAGED, NARROW>(kr, vr, a, plan, pg_next, k0 + kStride, k_end, dummy, lane, hd);
        dec_step<HD>(sk, qf, o, st, sv, k0, k_end, lane, cl2);
        if (!more) return false;
        dec_stage_v<HD, PAGED>(vr, sv, a, plan, pg_next, k0 + kStride, k_end, lane, hd);    // after this step's V^T reads (in order)
        pg_k = pg_next;
        if (step + 2 * kAttnWaves < n_steps) pg_next = pp.bases(a, kvh, hd);
        step += kAttnWaves;
        return true;
    };
    while (step < n_steps)
        if (!run_step()) break;

    // merge the wavefronts: the 4 lanes of a column share m_run, so their sums add
    const float l_tot = sum_xor32(sum_xor16(st.l_run));
    __syncthreads();   // every wavefront is done with its V^T staging
    float* part = reinterpret_cast<float*>(smem_raw);   // [wave][column][HD + 2]
    {
        float* pw = part + (wave * 16 + col) * (HD + 2);
#pragma unroll
        for (int db = 0; db < T::NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) pw[16 * db + 4 * hq + i] = o[db][i];
        if (hq == 0) {
            pw[HD] = st.m_run;
            pw[HD + 1] = l_tot;
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < G * HD; e += kAttnThreads) {
        const int c = e / HD, d = e % HD;
        float mstar = -FLT_MAX;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) mstar = fmaxf(mstar, part[(w * 16 + c) * (HD + 2) + HD]);
        float acc = 0.0f, lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float* pp = part + (w * 16 + c) * (HD + 2);
            const float f = __builtin_amdgcn_exp2f((pp[HD] - mstar) * cl2);
            acc = fmaf(f, pp[d], acc);
            lsum = fmaf(f, pp[HD + 1], lsum);
        }
        const int h = hb + c;
        if (NARROW || a.n_split == 1) {   // narrow heads: one split, columns past the head dropped
            if (d < hd)
                a.out[(size_t)q_row * a.o_stride + (size_t)h * hd + d] = from_f32<_Float16>(acc / (lsum + 1e-8f));
        } else {
            float* w = a.ws + (((size_t)s * a.n_heads + h) * a.n_split + sp) * (HD + 2);
            w[d] = acc;
            if (d == 0) {
                w[HD] = mstar;
                w[HD + 1] = lsum;
            }
        }
    }
}

// Finish split decode rows: out = sum_s 2^((m_s - m*)c) O_s / (sum_s 2^((m_s - m*)c) l_s + 1e-8).
// One workgroup per (sequence, head): thread s < n_split reads split s's (m, l),
// the weights go through LDS, then thread d sums its column with independent loads.
constexpr int kMaxSplits = 128;

template <int HD, bool PAGED>
__global__ __launch_bounds__(kMaxSplits) void attn_decode_combine(AttnArgs a) {
    __shared__ float wsc[kMaxSplits];
    __shared__ float red[kMaxSplits];
    __shared__ float lden;
    const int h = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
    int q_row, kv_len;
    const int32_t* table;
    if (!dec_sequence<PAGED>(a, s, q_row, kv_len, table)) return;
    const int ns = a.n_split;
    const float* w = a.ws + ((size_t)s * a.n_heads + h) * ns * (HD + 2);
    const float m_s = tid < ns ? w[tid * (HD + 2) + HD] : -FLT_MAX;
    const float l_s = tid < ns ? w[tid * (HD + 2) + HD + 1] : 0.0f;
    red[tid] = m_s;
    __syncthreads();
    for (int o = kMaxSplits / 2; o > 0; o >>= 1) {
        if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
        __syncthreads();
    }
    const float mstar = red[0];
    __syncthreads();
    const float f = __builtin_amdgcn_exp2f((m_s - mstar) * a.cl2);
    wsc[tid] = tid < ns ? f : 0.0f;
    red[tid] = tid < ns ? f * l_s : 0.0f;
    __syncthreads();
    for (int o = kMaxSplits / 2; o > 0; o >>= 1) {
        if (tid < o) red[tid] += red[tid + o];
        __syncthreads();
    }
    if (tid == 0) lden = red[0] + 1e-8f;
    __syncthreads();
    for (int d = tid; d < HD; d += kMaxSplits) {
        float acc = 0.0f;
#pragma unroll 8
        for (int sp = 0; sp < ns; ++sp) acc = fmaf(wsc[sp], w[sp * (HD + 2) + d], acc);
        a.out[(size_t)q_row * a.o_stride + (size_t)h * HD + d] = from_f32<_Float16>(acc / lden);
    }
}

// ---- any other head_dim up to 64 ------------------------------------------------------
//
// The reference kernel's tiles hold head_dim <= 64 and take any such value
// (kernels/flash_attention.cu:25-27,64-66); the matrix-core kernels above take
// 64 and 128 with 16-byte rows.  This kernel covers the rest of that range, 1 ..
// 63, at any row alignment: one workgroup = 256 consecutive queries of one
// query head, one query per lane.  Key tiles of 64 rows are staged through LDS
// as binary16, zero-padded to HDP (16, 32 or 64) columns, one element per load
// (no alignment assumed), and every lane reads the same LDS row (a broadcast).
// A lane keeps its query, running max, running sum and output row in
// registers; scores, probabilities and sums are fp32 (the probabilities are
// not rounded to binary16 as in the matrix-core kernels).  Masking, the GQA
// map, the paged lookups (a missing page reads as zero keys), the sequence
// checks and O / (l + 1e-8) are those of attn_fwd and attn_decode.
constexpr int kSmallThreads = 256;
constexpr int kSmallBK = 64;   // keys per LDS tile
constexpr int kSmallSub = 32;  // keys per online-softmax update (bounds the score registers)

template <int HDP, bool PAGED>
__global__ __launch_bounds__(kSmallThreads) void attn_small(AttnArgs a) {
    static_assert(HDP % 8 == 0 && HDP <= 64, "LDS rows are read 8 halfs at a time");
    __shared__ __attribute__((aligned(16))) _Float16 sk[kSmallBK * HDP];
    __shared__ __attribute__((aligned(16))) _Float16 sv[kSmallBK * HDP];
    const int hd = a.hd;
    const int head = (int)blockIdx.x % a.n_heads, qt = (int)blockIdx.x / a.n_heads;
    const int kvh = (int)(((long long)head * a.n_kv_heads) / a.n_heads);
    int q_begin = 0, q_len = a.q_len, kv_len = a.kv_len;
    const int32_t* table = nullptr;
    if constexpr (PAGED) {
        const int s = blockIdx.z;
        if (a.cu_q) {
            q_begin = a.cu_q[s];
            q_len = a.cu_q[s + 1] - q_begin;
        } else {   // decode: sequence s owns query row s
            q_begin = s;
            q_len = 1;
        }
        kv_len = a.ctx_lens[s];
        if (q_begin < 0 || q_len <= 0 || q_begin + q_len > a.n_q_rows) return;   // workgroup-uniform
        if (kv_len > a.max_blocks * QL_PAGE_SIZE) kv_len = a.max_blocks * QL_PAGE_SIZE;
        table = a.block_tables + (size_t)s * a.max_blocks;
    }
    if (kv_len < 0) kv_len = 0;
    const int q0 = qt * kSmallThreads;
    if (q0 >= q_len) return;   // workgroup-uniform

    const int tid = threadIdx.x;
    const int qi = q0 + tid;
    const bool q_valid = qi < q_len;
    const int pos_base = kv_len - q_len;   // absolute position of query 0
    // keys this workgroup needs, and the last key this lane's query sees
    int kv_hi = kv_len;
    if (a.causal) kv_hi = min(kv_len, pos_base + min(q_len, q0 + kSmallThreads));
    const int last = a.causal ? min(pos_base + qi, kv_len - 1) : kv_len - 1;

    float q[HDP], o[HDP];
    {
        const _Float16* qrow = a.q + (size_t)(q_begin + (q_valid ? qi : 0)) * a.q_stride + (size_t)head * hd;
#pragma unroll
        for (int d = 0; d < HDP; ++d) {
            q[d] = q_valid && d < hd ? (float)qrow[d] : 0.0f;
            o[d] = 0.0f;
        }
    }
    float m_run = -INFINITY, l_run = 0.0f;
    const float cl2 = a.cl2;

    for (int kv0 = 0; kv0 < kv_hi; kv0 += kSmallBK) {
        __syncthreads();   // every lane has read the previous tile
        for (int i = tid; i < kSmallBK * HDP; i += kSmallThreads) {
            const int r = i / HDP, c = i % HDP, key = kv0 + r;
            _Float16 kx = 0, vx = 0;
            if (c < hd && key < kv_len) {
                const _Float16* kp = nullptr;
                const _Float16* vp = nullptr;
                if constexpr (PAGED) {
                    const int b = table[key / QL_PAGE_SIZE];
                    if (b >= 0 && b < a.n_blocks) {
                        const size_t off =
                            (((size_t)a.layer * QL_PAGE_SIZE + key % QL_PAGE_SIZE) * a.n_kv_heads + kvh) * hd + c;
                        const _Float16* kb = a.kb[b];
                        const _Float16* vb = a.vb[b];
                        kp = kb ? kb + off : nullptr;
                        vp = vb ? vb + off : nullptr;
                    }
                } else {
                    const size_t off = (size_t)key * a.kv_stride + (size_t)kvh * hd + c;
                    kp = a.k + off;
                    vp = a.v + off;
                }
                if (kp) kx = *kp;
                if (vp) vx = *vp;
            }
            sk[i] = kx;
            sv[i] = vx;
        }
        __syncthreads();
        if (!q_valid) continue;
#pragma unroll 1
        for (int j0 = kv0; j0 < kv0 + kSmallBK && j0 <= last; j0 += kSmallSub) {
            const _Float16* kt = sk + (j0 - kv0) * HDP;
            const _Float16* vt = sv + (j0 - kv0) * HDP;
            float s[kSmallSub];
            float m_sub = -INFINITY;
#pragma unroll
            for (int j = 0; j < kSmallSub; ++j) {
                float acc = 0.0f;
#pragma unroll
                for (int c = 0; c < HDP / 8; ++c) {
                    const half8 k8 = *reinterpret_cast<const half8*>(kt + j * HDP + 8 * c);
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc = fmaf(q[8 * c + e], (float)k8[e], acc);
                }
                s[j] = j0 + j <= last ? acc : -INFINITY;
                m_sub = fmaxf(m_sub, s[j]);
            }
            // m_sub is finite: key j0 <= last is visible
            const float m_new = fmaxf(m_run, m_sub);
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * cl2);   // 0 on the first update
            l_run *= alpha;
#pragma unroll
            for (int d = 0; d < HDP; ++d) o[d] *= alpha;
#pragma unroll
            for (int j = 0; j < kSmallSub; ++j) {
                const float p = __builtin_amdgcn_exp2f((s[j] - m_new) * cl2);   // 0 for masked keys
                l_run += p;
#pragma unroll
                for (int c = 0; c < HDP / 8; ++c) {
                    const half8 v8 = *reinterpret_cast<const half8*>(vt + j * HDP + 8 * c);
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[8 * c + e] = fmaf(p, (float)v8[e], o[8 * c + e]);
                }
            }
            m_run = m_new;
        }
    }
    if (!q_valid) return;
    const float inv_den = 1.0f / (l_run + 1e-8f);
    _Float16* orow = a.out + (size_t)(q_begin + qi) * a.o_stride + (size_t)head * hd;
#pragma unroll
    for (int d = 0; d < HDP; ++d)
        if (d < hd) orow[d] = from_f32<_Float16>(o[d] * inv_den);
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
    } else if (head_dim == 64) {
        hipLaunchKernelGGL((attn_fwd<64, PAGED>), grid, dim3(kAttnThreads), 0, stream, a);
    } else {   // narrow heads, zero-padded to 64 in the tiles
        hipLaunchKernelGGL((attn_fwd<64, PAGED, true>), grid, dim3(kAttnThreads), 0, stream, a);
    }
    return hipGetLastError();
}

bool aligned_rows(const void* p, int64_t stride) {
    return qlh::aligned16(p) && stride % 8 == 0;
}

// head_dim 64 and 128 run the matrix-core kernels, as does a prefill over narrower
// heads of a multiple of 8 (zero-padded to 64 in the tiles); every other value up to
// 64 (the reference kernel's range) runs attn_small.
bool mfma_hd(int head_dim) { return head_dim == 64 || head_dim == 128; }
bool narrow_hd(int head_dim) { return head_dim < 64 && head_dim % 8 == 0; }
bool valid_hd(int head_dim) { return head_dim == 128 || (head_dim >= 1 && head_dim <= 64); }

// attn_small over n_seqs sequences of at most max_q_len queries (grid z = n_seqs).
template <bool PAGED>
hipError_t launch_small(const AttnArgs& a, int max_q_len, unsigned n_seqs, hipStream_t stream) {
    const long long gx = (long long)qlh::blocks_for(max_q_len, kSmallThreads) * a.n_heads;
    QL_CHECK_ARG(gx <= INT32_MAX && n_seqs <= 65535);
    const dim3 grid((unsigned)gx, 1, n_seqs);
    if (a.hd <= 16)
        hipLaunchKernelGGL((attn_small<16, PAGED>), grid, dim3(kSmallThreads), 0, stream, a);
    else if (a.hd <= 32)
        hipLaunchKernelGGL((attn_small<32, PAGED>), grid, dim3(kSmallThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((attn_small<64, PAGED>), grid, dim3(kSmallThreads), 0, stream, a);
    return hipGetLastError();
}

// Decode launch shape: chunks of <= 16 query heads per KV head, and key splits
// so that about 512 workgroups are in flight (2 per CU), each split covering
// at least 256 keys.
int dec_col_chunks(int n_heads, int n_kv_heads) {
    const int gmax = (n_heads + n_kv_heads - 1) / n_kv_heads;
    return (gmax + 15) / 16;
}

int dec_splits(int n_seqs, int n_kv_heads, int n_cg, int max_ctx) {
    const long long base = (long long)n_seqs * n_kv_heads * n_cg;
    const long long want = (512 + base - 1) / base;
    const long long cap = ((long long)max_ctx + 255) / 256;
    long long n = want < cap ? want : cap;
    if (n > kMaxSplits) n = kMaxSplits;
    return n < 1 ? 1 : (int)n;
}

size_t dec_ws_bytes(int n_seqs, int n_heads, int head_dim, int n_split) {
    return n_split > 1 ? (size_t)n_seqs * n_heads * n_split * (head_dim + 2) * sizeof(float) : 0;
}

template <bool PAGED>
hipError_t launch_decode(const AttnArgs& a, int head_dim, int n_seqs, hipStream_t stream) {
    const int n_cg = dec_col_chunks(a.n_heads, a.n_kv_heads);
    QL_CHECK_ARG((long long)a.n_split * n_cg <= INT32_MAX);
    const dim3 grid((unsigned)(a.n_split * n_cg), (unsigned)a.n_kv_heads, (unsigned)n_seqs);
    const dim3 cgrid((unsigned)a.n_heads, (unsigned)n_seqs);
    if (head_dim == 128) {
        hipLaunchKernelGGL((attn_decode<128, PAGED>), grid, dim3(kAttnThreads), 0, stream, a);
        if (a.n_split > 1)
            hipLaunchKernelGGL((attn_decode_combine<128, PAGED>), cgrid, dim3(kMaxSplits), 0, stream, a);
    } else if (head_dim == 64) {
        hipLaunchKernelGGL((attn_decode<64, PAGED>), grid, dim3(kAttnThreads), 0, stream, a);
        if (a.n_split > 1)
            hipLaunchKernelGGL((attn_decode_combine<64, PAGED>), cgrid, dim3(kMaxSplits), 0, stream, a);
    } else {   // narrow heads: one split (the caller sets n_split = 1)
        QL_CHECK_ARG(a.n_split == 1);
        hipLaunchKernelGGL((attn_decode<64, PAGED, true>), grid, dim3(kAttnThreads), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace

extern "C" hipError_t ql_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                       uint16_t* out, int q_len, int kv_len, int n_heads,
                                       int n_kv_heads, int head_dim, int64_t q_row_stride,
                                       int64_t kv_row_stride, int64_t out_row_stride, int causal,
                                       hipStream_t stream) {
    QL_CHECK_ARG(q_len >= 0 && kv_len >= 0 && n_heads > 0 && n_kv_heads > 0);
    QL_CHECK_ARG(n_kv_heads <= n_heads && n_heads <= 65535);
    QL_CHECK_ARG(valid_hd(head_dim));
    QL_CHECK_ARG(q_row_stride >= (int64_t)n_heads * head_dim);
    QL_CHECK_ARG(out_row_stride >= (int64_t)n_heads * head_dim);
    QL_CHECK_ARG(kv_row_stride >= (int64_t)n_kv_heads * head_dim);
    QL_CHECK_ARG(kv_row_stride < (int64_t)1 << 24);   // 64 key rows span < 4 GiB (32-bit offsets)
    if (q_len == 0) return hipSuccess;
    QL_CHECK_ARG(q && out && (kv_len == 0 || (k && v)));
    if (mfma_hd(head_dim)) {
        QL_CHECK_ARG(aligned_rows(q, q_row_stride) && aligned_rows(out, out_row_stride));
        QL_CHECK_ARG(kv_len == 0 || (aligned_rows(k, kv_row_stride) && aligned_rows(v, kv_row_stride)));
    }
    // narrow heads (a multiple of 8 below 64) with 16-byte aligned rows: the
    // head_dim-64 matrix-core kernel with the heads zero-padded in its tiles
    const bool narrow = narrow_hd(head_dim) && aligned_rows(q, q_row_stride) &&
                        aligned_rows(out, out_row_stride) &&
                        (kv_len == 0 || (aligned_rows(k, kv_row_stride) && aligned_rows(v, kv_row_stride)));
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
    a.hd = head_dim;
    if (narrow && q_len > 1) return launch_attn<false>(a, head_dim, qlh::blocks_for(q_len, kBQ), 1, stream);
    if (!mfma_hd(head_dim) && !narrow) return launch_small<false>(a, q_len, 1, stream);
    if (q_len == 1) {   // decode: the query heads of a KV head share one pass over K/V
        a.n_split = 1;
        return launch_decode<false>(a, head_dim, 1, stream);
    }
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
    QL_CHECK_ARG(valid_hd(head_dim));
    QL_CHECK_ARG(n_layers > 0 && layer >= 0 && layer < n_layers);
    QL_CHECK_ARG(max_blocks_per_seq >= 0 && max_blocks_per_seq <= (INT32_MAX / QL_PAGE_SIZE));
    QL_CHECK_ARG(n_blocks >= 0);
    QL_CHECK_ARG(q_row_stride >= (int64_t)n_heads * head_dim);
    QL_CHECK_ARG(out_row_stride >= (int64_t)n_heads * head_dim);
    if (n_seqs == 0 || max_q_len == 0 || n_q_rows == 0) return hipSuccess;
    QL_CHECK_ARG(q && out && cu_q_lens && ctx_lens);
    QL_CHECK_ARG(max_blocks_per_seq == 0 || (block_tables && k_blocks && v_blocks));
    if (mfma_hd(head_dim)) QL_CHECK_ARG(aligned_rows(q, q_row_stride) && aligned_rows(out, out_row_stride));
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
    a.hd = head_dim;
    // narrow heads (a multiple of 8 below 64) with aligned rows: the head_dim-64
    // kernels, zero-padded (the decode in one key split)
    const bool narrow = narrow_hd(head_dim) && aligned_rows(q, q_row_stride) && aligned_rows(out, out_row_stride);
    if (!mfma_hd(head_dim) && !narrow) return launch_small<true>(a, max_q_len, (unsigned)n_seqs, stream);
    if (max_q_len == 1) {   // every sequence decodes one token
        a.n_split = 1;
        return launch_decode<true>(a, head_dim, n_seqs, stream);
    }
    return launch_attn<true>(a, head_dim, qlh::blocks_for(max_q_len, kBQ), (unsigned)n_seqs, stream);
}

extern "C" hipError_t ql_paged_decode_workspace_size(int n_seqs, int n_heads, int n_kv_heads,
                                                     int head_dim, int max_ctx_len, size_t* bytes) {
    QL_CHECK_ARG(bytes && n_seqs >= 0 && n_heads > 0 && n_kv_heads > 0 && n_kv_heads <= n_heads);
    QL_CHECK_ARG(valid_hd(head_dim) && max_ctx_len >= 0);
    *bytes = 0;
    if (n_seqs == 0 || !mfma_hd(head_dim)) return hipSuccess;   // attn_small: one pass, no workspace
    const int n_split = dec_splits(n_seqs, n_kv_heads, dec_col_chunks(n_heads, n_kv_heads), max_ctx_len);
    *bytes = dec_ws_bytes(n_seqs, n_heads, head_dim, n_split);
    return hipSuccess;
}

extern "C" hipError_t ql_decode_attention_workspace_size(int n_heads, int n_kv_heads, int head_dim,
                                                         int kv_len, size_t* bytes) {
    QL_CHECK_ARG(bytes && n_heads > 0 && n_kv_heads > 0 && n_kv_heads <= n_heads);
    QL_CHECK_ARG(valid_hd(head_dim) && kv_len >= 0);
    *bytes = 0;
    if (!mfma_hd(head_dim)) return hipSuccess;   // attn_small: one pass, no workspace
    const int n_split = dec_splits(1, n_kv_heads, dec_col_chunks(n_heads, n_kv_heads), kv_len);
    *bytes = dec_ws_bytes(1, n_heads, head_dim, n_split);
    return hipSuccess;
}

extern "C" hipError_t ql_decode_attention_f16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                              uint16_t* out, int kv_len, int n_heads, int n_kv_heads,
                                              int head_dim, int64_t kv_row_stride, void* workspace,
                                              size_t workspace_bytes, hipStream_t stream) {
    QL_CHECK_ARG(kv_len >= 0 && n_heads > 0 && n_kv_heads > 0);
    QL_CHECK_ARG(n_kv_heads <= n_heads && n_heads <= 65535);
    QL_CHECK_ARG(valid_hd(head_dim));
    QL_CHECK_ARG(kv_row_stride >= (int64_t)n_kv_heads * head_dim);
    QL_CHECK_ARG(kv_row_stride < (int64_t)1 << 24);   // as ql_attention_f16
    QL_CHECK_ARG(workspace_bytes == 0 || workspace);
    QL_CHECK_ARG(q && out && (kv_len == 0 || (k && v)));
    const int64_t qs = (int64_t)n_heads * head_dim;
    if (mfma_hd(head_dim)) {
        QL_CHECK_ARG(aligned_rows(q, qs) && aligned_rows(out, qs));
        QL_CHECK_ARG(kv_len == 0 || (aligned_rows(k, kv_row_stride) && aligned_rows(v, kv_row_stride)));
    }
    AttnArgs a{};
    a.q = reinterpret_cast<const _Float16*>(q);
    a.out = reinterpret_cast<_Float16*>(out);
    a.q_stride = qs;
    a.o_stride = qs;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.cl2 = scale_log2e(head_dim);
    a.causal = 1;
    a.q_len = 1;
    a.kv_len = kv_len;
    a.k = reinterpret_cast<const _Float16*>(k);
    a.v = reinterpret_cast<const _Float16*>(v);
    a.kv_stride = kv_row_stride;
    a.hd = head_dim;
    if (narrow_hd(head_dim) && aligned_rows(q, qs) && aligned_rows(out, qs) &&
        (kv_len == 0 || (aligned_rows(k, kv_row_stride) && aligned_rows(v, kv_row_stride)))) {
        a.n_split = 1;   // narrow heads on the head_dim-64 kernel, zero-padded: one pass, no workspace
        return launch_decode<false>(a, head_dim, 1, stream);
    }
    if (!mfma_hd(head_dim)) return launch_small<false>(a, 1, 1, stream);
    // as many key splits as wanted and the workspace holds (1 = no workspace used)
    int n_split = dec_splits(1, n_kv_heads, dec_col_chunks(n_heads, n_kv_heads), kv_len);
    while (n_split > 1 && dec_ws_bytes(1, n_heads, head_dim, n_split) > workspace_bytes) --n_split;
    QL_CHECK_ARG(n_split == 1 || qlh::aligned16(workspace));
    a.n_split = n_split;
    a.ws = n_split > 1 ? static_cast<float*>(workspace) : nullptr;
    return launch_decode<false>(a, head_dim, 1, stream);
}

namespace {

constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kScratchMaxDevices] = {};

// Device address of `scratch` on the device of `stream` (the current device
// for the null stream), where the kernels reading it run: looked up on the
// first call per device, with that device made current for the lookup, and
// kept for the process.
hipError_t decode_scratch(hipStream_t stream, void** addr) {
    int dev = -1;
    const hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kScratchMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        int cur = -1;
        hipError_t r = hipGetDevice(&cur);
        if (r != hipSuccess) return r;
        if (cur != dev && (r = hipSetDevice(dev)) != hipSuccess) return r;
        void* p = nullptr;
        r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (r != hipSuccess) return r;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_addr[dev] = p;
    }
    *addr = g_scratch_addr[dev];
    return hipSuccess;
}

// Shared body of the split decode entry points.  from_scratch: run exactly the
// split the workspace query sizes, with its partials in `scratch`, or refuse
// when they would not fit; otherwise as many splits as `workspace` holds.
hipError_t paged_decode(
    const uint16_t* q, uint16_t* out, int64_t q_row_stride, int64_t out_row_stride, int n_seqs,
    const int32_t* ctx_lens, int max_ctx_len, const int32_t* block_tables, int max_blocks_per_seq,
    const uint16_t* const* k_blocks, const uint16_t* const* v_blocks, int n_blocks, int layer,
    int n_layers, int n_heads, int n_kv_heads, int head_dim, void* workspace,
    size_t workspace_bytes, bool from_scratch, hipStream_t stream) {
    QL_CHECK_ARG(n_seqs >= 0 && n_seqs <= 65535 && max_ctx_len >= 0);
    QL_CHECK_ARG(n_heads > 0 && n_kv_heads > 0 && n_kv_heads <= n_heads && n_heads <= 65535);
    QL_CHECK_ARG(valid_hd(head_dim));
    QL_CHECK_ARG(n_layers > 0 && layer >= 0 && layer < n_layers);
    QL_CHECK_ARG(max_blocks_per_seq >= 0 && max_blocks_per_seq <= (INT32_MAX / QL_PAGE_SIZE));
    QL_CHECK_ARG(n_blocks >= 0);
    QL_CHECK_ARG(q_row_stride >= (int64_t)n_heads * head_dim);
    QL_CHECK_ARG(out_row_stride >= (int64_t)n_heads * head_dim);
    QL_CHECK_ARG(workspace_bytes == 0 || workspace);
    if (n_seqs == 0) return hipSuccess;
    QL_CHECK_ARG(q && out && ctx_lens);
    QL_CHECK_ARG(max_blocks_per_seq == 0 || (block_tables && k_blocks && v_blocks));
    if (mfma_hd(head_dim)) QL_CHECK_ARG(aligned_rows(q, q_row_stride) && aligned_rows(out, out_row_stride));
    AttnArgs a{};
    a.q = reinterpret_cast<const _Float16*>(q);
    a.out = reinterpret_cast<_Float16*>(out);
    a.q_stride = q_row_stride;
    a.o_stride = out_row_stride;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.cl2 = scale_log2e(head_dim);
    a.causal = 1;
    a.kb = reinterpret_cast<const _Float16* const*>(k_blocks);
    a.vb = reinterpret_cast<const _Float16* const*>(v_blocks);
    a.n_blocks = n_blocks;
    a.block_tables = block_tables;
    a.max_blocks = max_blocks_per_seq;
    a.cu_q = nullptr;   // sequence s owns query row s
    a.ctx_lens = ctx_lens;
    a.n_q_rows = n_seqs;
    a.layer = layer;
    a.hd = head_dim;
    if (narrow_hd(head_dim) && aligned_rows(q, q_row_stride) && aligned_rows(out, out_row_stride)) {
        a.n_split = 1;   // narrow heads on the head_dim-64 kernel, zero-padded: one pass, no workspace
        return launch_decode<true>(a, head_dim, n_seqs, stream);
    }
    if (!mfma_hd(head_dim)) return launch_small<true>(a, 1, (unsigned)n_seqs, stream);   // no split
    int n_split = dec_splits(n_seqs, n_kv_heads, dec_col_chunks(n_heads, n_kv_heads), max_ctx_len);
    if (from_scratch) {
        QL_CHECK_ARG(dec_ws_bytes(n_seqs, n_heads, head_dim, n_split) <= kDecodeScratchBytes);
        if (n_split > 1) {
            const hipError_t e = decode_scratch(stream, &workspace);
            if (e != hipSuccess) return e;
        }
    } else {
        // as many key splits as wanted and the workspace holds (1 = no workspace used)
        while (n_split > 1 && dec_ws_bytes(n_seqs, n_heads, head_dim, n_split) > workspace_bytes) --n_split;
    }
    a.n_split = n_split;
    a.ws = n_split > 1 ? static_cast<float*>(workspace) : nullptr;
    return launch_decode<true>(a, head_dim, n_seqs, stream);
}

}  // namespace

extern "C" hipError_t ql_paged_decode_attention_f16(
    const uint16_t* q, uint16_t* out, int64_t q_row_stride, int64_t out_row_stride, int n_seqs,
    const int32_t* ctx_lens, int max_ctx_len, const int32_t* block_tables, int max_blocks_per_seq,
    const uint16_t* const* k_blocks, const uint16_t* const* v_blocks, int n_blocks, int layer,
    int n_layers, int n_heads, int n_kv_heads, int head_dim, void* workspace,
    size_t workspace_bytes, hipStream_t stream) {
    return paged_decode(q, out, q_row_stride, out_row_stride, n_seqs, ctx_lens, max_ctx_len,
                        block_tables, max_blocks_per_seq, k_blocks, v_blocks, n_blocks, layer,
                        n_layers, n_heads, n_kv_heads, head_dim, workspace, workspace_bytes, false,
                        stream);
}

extern "C" hipError_t ql_paged_decode_attention_f16_noalloc(
    const uint16_t* q, uint16_t* out, int64_t q_row_stride, int64_t out_row_stride, int n_seqs,
    const int32_t* ctx_lens, int max_ctx_len, const int32_t* block_tables, int max_blocks_per_seq,
    const uint16_t* const* k_blocks, const uint16_t* const* v_blocks, int n_blocks, int layer,
    int n_layers, int n_heads, int n_kv_heads, int head_dim, hipStream_t stream) {
    return paged_decode(q, out, q_row_stride, out_row_stride, n_seqs, ctx_lens, max_ctx_len,
                        block_tables, max_blocks_per_seq, k_blocks, v_blocks, n_blocks, layer,
                        n_layers, n_heads, n_kv_heads, head_dim, nullptr, 0, true, stream);
}
