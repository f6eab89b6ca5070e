// rope.hip -- rotary position embedding on Q and K (GQA head counts) in one
// launch, in place, for gfx950.
//
// Arithmetic per pair i of a head at position pos (kernels/rope.cu:35-41,
// kernels/fp16_ops.cu:54-62), with the transcendental steps made accurate so a
// CPU restatement can reproduce them:
//   e   = (2i) / d                       fp32 division, as the reference
//   inv = 1 / (float)pow(theta, e)       pow in fp64, rounded to fp32
//   a   = (float)pos * inv               fp32
//   c   = cos(a), s = sin(a)             evaluated in fp64 and rounded to fp32
//                                        (bit-identical to the CPU restatement; a
//                                        1-ulp fp32 sincos would move outputs that
//                                        cancel to near zero by binary16 steps)
//   y0  = fma(x0, c, -(x1*s)),  y1 = fma(x0, s, x1*c)
// Pairing: interleaved (2i, 2i+1) as the reference, or rotate-half (i, i+d/2).
//
// Fast path (d/2 <= 128 pairs, 16-byte aligned rows; a wavefront pass takes as many
// whole heads' 16-byte chunks as fit its 64 lanes): inv_freq is computed once per call on the host (the same libm
// pow the CPU restatement uses) and passed by value.  One wavefront serves a
// (token, group of heads): every lane first issues the loads of all 16-byte
// chunks it owns (at most MAXU, or MAXU pairs of chunks for rotate-half), then
// evaluates the trig of pair `lane` while they are in flight; the values are
// redistributed with cross-lane permutes so each pair's sincos is computed once
// per token and group.  Every wavefront access is a contiguous, coalesced
// 16-byte-per-lane span, streamed with nontemporal hints.
#include <math.h>

#include <algorithm>

#include "ql_common.hpp"
#include "quantlib_amd.h"

namespace {

using namespace ql;

template <int N>
struct InvFreqN {
    float v[N];
};
using InvFreq = InvFreqN<64>;   // up to 64 pairs (head_dim 128)

// inv_freq of pair i, host side, in the order of kernels/rope.cu:35.
float host_inv_freq(int pair, int d, float theta) {
    const float e = (2.0f * (float)pair) / (float)d;
    const float p = (float)pow((double)theta, (double)e);
    return 1.0f / p;
}

__device__ __forceinline__ float dev_inv_freq(int pair, int d, float theta) {
    const float e = (2.0f * (float)pair) / (float)d;
    const float p = (float)pow((double)theta, (double)e);
    return 1.0f / p;
}

__device__ __forceinline__ void trig(float a, float& c, float& s) {
    double sd, cd;
    sincos((double)a, &sd, &cd);
    c = (float)cd;
    s = (float)sd;
}

__device__ __forceinline__ void rotate(float x0, float x1, float c, float s, float& y0,
                                       float& y1) {
    y0 = fmaf(x0, c, -(x1 * s));
    y1 = fmaf(x0, s, x1 * c);
}

// Where the fused variants put K and V: nothing (plain RoPE), the paged pool
// (block pointer tables + slot mapping), or the contiguous cache
// [n_layers, max_seq, n_kv_heads, head_dim] at positions pos0 + t.
enum CacheKind { kNoCache = 0, kPagedCache = 1, kContigCache = 2 };

template <typename D>
struct KvDst {
    D* const* kb;           // paged: per-block K / V base pointers (device)
    D* const* vb;
    const int32_t* slots;   // paged: slot of each token (block*16 + offset), <0 = skip
    int n_blocks;
    D* kc;                  // contiguous: cache bases
    D* vc;
    int pos0;
    int max_seq;
    const D* v;             // new V rows [n_tokens, v_row_stride]
    long long vs;
    int layer;
    int skip_k_inplace;     // 1: rotated K goes to the cache only, k is left as read
};

// Cache row of token t for the current layer (K and V), or nullptr to skip.
template <typename D, int CACHE>
__device__ __forceinline__ void cache_rows(const KvDst<D>& kv, int t, int kvw, D*& kd, D*& vd) {
    kd = vd = nullptr;
    if constexpr (CACHE == kPagedCache) {
        const int slot = ld_scalar(kv.slots + t);
        if (slot >= 0 && slot / QL_PAGE_SIZE < kv.n_blocks) {
            const int b = slot / QL_PAGE_SIZE;
            const size_t off = ((size_t)kv.layer * QL_PAGE_SIZE + slot % QL_PAGE_SIZE) * (size_t)kvw;
            kd = ld_scalar(kv.kb + b) + off;
            vd = ld_scalar(kv.vb + b) + off;
        }
    } else if constexpr (CACHE == kContigCache) {
        const size_t off = ((size_t)kv.layer * kv.max_seq + kv.pos0 + t) * (size_t)kvw;
        kd = kv.kc + off;
        vd = kv.vc + off;
    }
}

// Store a W-element chunk to a cache row that may not be 16-byte aligned
// (paged block pointers come from a device table).
template <typename D, typename V>
__device__ __forceinline__ void store_cache(D* dst, const V& v, bool aligned) {
    if (aligned) {
        store<true>(reinterpret_cast<V*>(dst), v);
    } else {
#pragma unroll
        for (int e = 0; e < (int)(sizeof(V) / sizeof(D)); ++e) dst[e] = v.v[e];
    }
}

// Heads of a token, in order: hq Q heads, hk K heads, then (fused variants)
// hk V heads that are copied to the cache unrotated.
// NP: the pairs the inv_freq table holds (64, or 128 for head_dim up to 256: each
// lane then evaluates the angles of pairs lane and lane + 64).
template <typename D, int PAIRING, int MAXU, int CACHE, int NP = 64>
__global__ __launch_bounds__(kBlock) void rope_fast(D* q, D* k, int n_tokens, int hq, int hk,
                                                    int d, long long qs, long long ks,
                                                    const int32_t* __restrict__ positions,
                                                    int pos_offset, InvFreqN<NP> inv,
                                                    int heads_per_wave, KvDst<D> kv) {
    constexpr int W = vec16<D>();
    constexpr int PPS = PAIRING == QL_ROPE_INTERLEAVED ? W / 2 : W;  // pairs per slot
    constexpr bool HALF = PAIRING == QL_ROPE_HALF;
    using V = Vec<D, W>;

    const int lane = threadIdx.x & (kWave - 1);
    // token index made scalar: its position, slot and block pointers are then
    // read with scalar loads, whose waits do not wait for the row loads
    const int t = blockIdx.x * (kBlock / kWave) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    if (t >= n_tokens) return;  // wavefront-uniform; no barriers below
    const int npairs = d >> 1;
    const int S = npairs / PPS;        // slots per head (<= 64)
    const int SPW = (kWave / S) * S;   // slots per wavefront pass: whole heads, lanes past it idle
    const int j = lane % S;
    const int hrot = hq + hk;                          // heads that rotate
    const int htot = hrot + (CACHE != kNoCache ? hk : 0);
    const int h0 = blockIdx.y * heads_per_wave;
    const int h1 = min(htot, h0 + heads_per_wave);
    const int nslots = (h1 - h0) * S;  // <= SPW * MAXU (host guarantees)
    D* qt = q ? q + (long long)t * qs : nullptr;
    D* kt = k ? k + (long long)t * ks : nullptr;
    const D* vt = CACHE != kNoCache ? kv.v + (long long)t * kv.vs : nullptr;

    D* kd = nullptr;
    D* vd = nullptr;
    bool cache_aligned = true;
    if constexpr (CACHE != kNoCache) {
        cache_rows<D, CACHE>(kv, t, hk * d, kd, vd);
        cache_aligned = ((reinterpret_cast<uintptr_t>(kd) | reinterpret_cast<uintptr_t>(vd)) & 15) == 0;
    }

    V lo[MAXU];
    V hi[HALF ? MAXU : 1];
    D* src[MAXU];
    int hs[MAXU];
    // Every lane loads (slots past the group, and idle lanes, re-read the group's last
    // slot's row, in bounds): a load under a per-lane test makes the compiler wait for
    // it before issuing the next one.
#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
        const int sl = lane + u * SPW;
        const bool valid = lane < SPW && sl < nslots;
        const int h = h0 + min(sl, nslots - 1) / S;
        // Selected as integer addresses: the equivalent nested pointer
        // select crashes this toolchain's optimizer.
        const uintptr_t head =
            h < hq ? reinterpret_cast<uintptr_t>(qt) + sizeof(D) * (size_t)h * d
                   : (h < hrot ? reinterpret_cast<uintptr_t>(kt) + sizeof(D) * (size_t)(h - hq) * d
                               : reinterpret_cast<uintptr_t>(vt) + sizeof(D) * (size_t)(h - hrot) * d);
        D* const p = reinterpret_cast<D*>(head) + j * W;
        lo[u] = load<true>(reinterpret_cast<const V*>(p));
        if constexpr (HALF) hi[u] = load<true>(reinterpret_cast<const V*>(p + npairs));
        src[u] = valid ? p : nullptr;
        hs[u] = valid ? h : -1;
    }

    float c[PPS], s[PPS];
    if (h0 < hrot) {  // wavefront-uniform: this group has heads to rotate
        const int pos = positions ? ld_scalar(positions + t) : pos_offset + t;
        float c_own, s_own;
        trig((float)pos * inv.v[lane % npairs], c_own, s_own);
        if constexpr (NP == 64) {
#pragma unroll
            for (int e = 0; e < PPS; ++e) {
                c[e] = __shfl(c_own, j * PPS + e, kWave);
                s[e] = __shfl(s_own, j * PPS + e, kWave);
            }
        } else {   // pairs 64 .. npairs - 1 from the second angle
            float c_hi, s_hi;
            trig((float)pos * inv.v[64 + lane % (npairs - 64)], c_hi, s_hi);
#pragma unroll
            for (int e = 0; e < PPS; ++e) {
                const int pi = j * PPS + e;
                const float cl = __shfl(c_own, pi & 63, kWave), sl = __shfl(s_own, pi & 63, kWave);
                const float ch = __shfl(c_hi, pi & 63, kWave), sh = __shfl(s_hi, pi & 63, kWave);
                c[e] = pi < 64 ? cl : ch;
                s[e] = pi < 64 ? sl : sh;
            }
        }
    }

#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
        if (!src[u]) continue;
        const int h = hs[u];
        if (CACHE != kNoCache && h >= hrot) {  // V head: copy into the cache
            if (vd) {
                D* dst = vd + (h - hrot) * d + j * W;
                store_cache<D>(dst, lo[u], cache_aligned);
                if constexpr (HALF) store_cache<D>(dst + npairs, hi[u], cache_aligned);
            }
            continue;
        }
        V ylo, yhi;
        if constexpr (!HALF) {
#pragma unroll
            for (int e = 0; e < PPS; ++e) {
                float y0, y1;
                rotate(to_f32(lo[u].v[2 * e]), to_f32(lo[u].v[2 * e + 1]), c[e], s[e], y0, y1);
                ylo.v[2 * e] = from_f32<D>(y0);
                ylo.v[2 * e + 1] = from_f32<D>(y1);
            }
            if (!(CACHE != kNoCache && h >= hq && kv.skip_k_inplace))
                store<true>(reinterpret_cast<V*>(src[u]), ylo);
        } else {
#pragma unroll
            for (int e = 0; e < PPS; ++e) {
                float y0, y1;
                rotate(to_f32(lo[u].v[e]), to_f32(hi[u].v[e]), c[e], s[e], y0, y1);
                ylo.v[e] = from_f32<D>(y0);
                yhi.v[e] = from_f32<D>(y1);
            }
            if (!(CACHE != kNoCache && h >= hq && kv.skip_k_inplace)) {
                store<true>(reinterpret_cast<V*>(src[u]), ylo);
                store<true>(reinterpret_cast<V*>(src[u] + npairs), yhi);
            }
        }
        if (CACHE != kNoCache && h >= hq && kd) {  // rotated K also goes to the cache
            D* dst = kd + (h - hq) * d + j * W;
            store_cache<D>(dst, ylo, cache_aligned);
            if constexpr (HALF) store_cache<D>(dst + npairs, yhi, cache_aligned);
        }
    }
}

// Any even head_dim (<= 2048), any alignment: one wavefront per token, lane =
// pair index (strided), trig once per (token, pair), then every head; fused
// variants then copy the token's V row (and the rotated K row) to the cache.
template <typename D, int PAIRING, int CACHE>
__global__ __launch_bounds__(kBlock) void rope_generic(D* q, D* k, int n_tokens, int hq, int hk,
                                                       int d, long long qs, long long ks,
                                                       const int32_t* __restrict__ positions,
                                                       int pos_offset, float theta,
                                                       KvDst<D> kv) {
    const int lane = threadIdx.x & (kWave - 1);
    // token index made scalar: its position, slot and block pointers are then
    // read with scalar loads, whose waits do not wait for the row loads
    const int t = blockIdx.x * (kBlock / kWave) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    if (t >= n_tokens) return;
    const int npairs = d >> 1;
    const int pos = positions ? ld_scalar(positions + t) : pos_offset + t;
    D* kd = nullptr;
    D* vd = nullptr;
    if constexpr (CACHE != kNoCache) cache_rows<D, CACHE>(kv, t, hk * d, kd, vd);
    for (int p = lane; p < npairs; p += kWave) {
        float c, s;
        trig((float)pos * dev_inv_freq(p, d, theta), c, s);
        const int i0 = PAIRING == QL_ROPE_INTERLEAVED ? 2 * p : p;
        const int i1 = PAIRING == QL_ROPE_INTERLEAVED ? 2 * p + 1 : p + npairs;
        for (int h = 0; h < hq + hk; ++h) {
            D* head = h < hq ? q + (long long)t * qs + (long long)h * d
                             : k + (long long)t * ks + (long long)(h - hq) * d;
            float y0, y1;
            rotate(to_f32(head[i0]), to_f32(head[i1]), c, s, y0, y1);
            if (!(CACHE != kNoCache && h >= hq && kv.skip_k_inplace)) {
                head[i0] = from_f32<D>(y0);
                head[i1] = from_f32<D>(y1);
            }
            if (CACHE != kNoCache && h >= hq && kd) {
                kd[(h - hq) * d + i0] = from_f32<D>(y0);
                kd[(h - hq) * d + i1] = from_f32<D>(y1);
            }
        }
    }
    if constexpr (CACHE != kNoCache) {
        if (vd) {
            const D* vt = kv.v + (long long)t * kv.vs;
            for (int i = lane; i < hk * d; i += kWave) vd[i] = vt[i];
        }
    }
}

// Rows starting at p every stride_bytes are all 16-byte aligned (or p is unused).
inline bool rows_aligned16(const void* p, int64_t stride_bytes) {
    return !p || (qlh::aligned16(p) && stride_bytes % 16 == 0);
}

// Plane kernel for the common head sizes (HD = 64 or 128, compile time): each
// workgroup takes one plane -- Q, K or (fused variants) V -- and a group of its
// heads, so every branch on the head type is uniform over the workgroup and
// all address arithmetic is shifts.  V planes only copy into the cache and
// skip the trig.  Groups: gq over Q, gk over K, gk over V.  Grid: mix == 0 puts
// the plane groups along blockIdx.y (each plane streams its own buffer); mix > 0
// is one row of workgroups in which every `mix` token blocks of one plane group
// are followed by the same token blocks of the next group, so Q, K and V rows
// that interleave in one buffer (a fused QKV projection's output) are read
// together.
template <typename D, int PAIRING, int HD, int MAXU, int CACHE>
__global__ __launch_bounds__(kBlock) void rope_planes(D* q, D* k, int n_tokens, int hq, int hk,
                                                      long long qs, long long ks,
                                                      const int32_t* __restrict__ positions,
                                                      int pos_offset, InvFreq inv, int gq, int gk,
                                                      int hpw_q, int hpw_k, KvDst<D> kv, int mix) {
    constexpr int W = vec16<D>();
    constexpr bool HALF = PAIRING == QL_ROPE_HALF;
    constexpr int NP = HD / 2;                                  // pairs per head
    constexpr int PPS = HALF ? W : W / 2;                       // pairs per slot
    constexpr int S = NP / PPS;                                 // slots per head
    static_assert(S >= 1 && 64 % S == 0, "head chunks must tile a wavefront");
    using V = Vec<D, W>;

    const int lane = threadIdx.x & (kWave - 1);
    // token index made scalar: its position, slot and block pointers are then
    // read with scalar loads, whose waits do not wait for the row loads
    int tb = (int)blockIdx.x, gy = (int)blockIdx.y;   // token block, plane group
    if (mix > 0) {
        const int span = (gq + gk + (CACHE != kNoCache ? gk : 0)) * mix;
        const int c = tb / span, r = tb - c * span;
        gy = r / mix;
        tb = c * mix + (r - gy * mix);
    }
    const int t = tb * (kBlock / kWave) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    if (t >= n_tokens) return;  // wavefront-uniform; no barriers below
    const int j = lane % S;

    // plane and head range of this workgroup (uniform)
    const int plane = gy < gq ? 0 : (gy < gq + gk ? 1 : 2);    // 0 Q, 1 K, 2 V
    const int g = plane == 0 ? gy : (plane == 1 ? gy - gq : gy - gq - gk);
    const int hpw = plane == 0 ? hpw_q : hpw_k;
    const int nh = plane == 0 ? hq : hk;
    const int h0 = g * hpw;
    const int h1 = min(nh, h0 + hpw);
    const int nslots = (h1 - h0) * S;
    D* row = plane == 0 ? q + (long long)t * qs
           : (plane == 1 ? k + (long long)t * ks : const_cast<D*>(kv.v) + (long long)t * kv.vs);
    // the same row base made scalar for the write-through buffer stores (the
    // loads keep `row`: a pointer rebuilt from integers would make them FLAT
    // accesses, which also count against the scalar-load counter)
    D* const row_s = uniform(row);

    // The per-lane inv_freq read goes first (vector loads retire in issue
    // order, so the trig's wait for it then does not wait for the rows), and
    // every lane loads (slots past the group re-read its last chunk): a load
    // under a per-lane test makes the compiler wait for it before the next.
    const float inv_l = inv.v[lane % NP];
    asm volatile("" ::: "memory");   // keep the row loads after it
    V lo[MAXU];
    V hi[HALF ? MAXU : 1];
#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
        const int sl = min(lane + u * kWave, nslots - 1);
        const V* p = reinterpret_cast<const V*>(row + (h0 + sl / S) * HD + j * W);
        lo[u] = load<true>(p);
        if constexpr (HALF) hi[u] = load<true>(reinterpret_cast<const V*>(reinterpret_cast<const D*>(p) + NP));
    }

    D* kd = nullptr;
    D* vd = nullptr;
    bool cache_aligned = true;
    if constexpr (CACHE != kNoCache) {
        if (plane != 0) {
            cache_rows<D, CACHE>(kv, t, hk * HD, kd, vd);
            kd = uniform(kd);
            vd = uniform(vd);
            cache_aligned = ((reinterpret_cast<uintptr_t>(kd) | reinterpret_cast<uintptr_t>(vd)) & 15) == 0;
        }
        if (plane == 2) {  // V: copy the rows into the cache, no rotation
            if (vd) {
#pragma unroll
                for (int u = 0; u < MAXU; ++u) {
                    const int sl = lane + u * kWave;
                    if (sl < nslots) {
                        const int off = (h0 + sl / S) * HD + j * W;
                        if (cache_aligned) {
                            store_wt(vd, (uint32_t)off * sizeof(D), lo[u]);
                            if constexpr (HALF) store_wt(vd, (uint32_t)(off + NP) * sizeof(D), hi[u]);
                        } else {
                            store_cache<D>(vd + off, lo[u], false);
                            if constexpr (HALF) store_cache<D>(vd + off + NP, hi[u], false);
                        }
                    }
                }
            }
            return;
        }
    }

    const int pos = positions ? ld_scalar(positions + t) : pos_offset + t;
    float c_own, s_own;
    trig((float)pos * inv_l, c_own, s_own);
    float c[PPS], s[PPS];
#pragma unroll
    for (int e = 0; e < PPS; ++e) {
        c[e] = __shfl(c_own, j * PPS + e, kWave);
        s[e] = __shfl(s_own, j * PPS + e, kWave);
    }

#pragma unroll
    for (int u = 0; u < MAXU; ++u) {
        const int sl = lane + u * kWave;
        if (sl >= nslots) continue;
        const int off = (h0 + sl / S) * HD + j * W;
        V ylo, yhi;
        if constexpr (!HALF) {
#pragma unroll
            for (int e = 0; e < PPS; ++e) {
                float y0, y1;
                rotate(to_f32(lo[u].v[2 * e]), to_f32(lo[u].v[2 * e + 1]), c[e], s[e], y0, y1);
                ylo.v[2 * e] = from_f32<D>(y0);
                ylo.v[2 * e + 1] = from_f32<D>(y1);
            }
            if (!(CACHE != kNoCache && plane == 1 && kv.skip_k_inplace))
                store_wt(row_s, (uint32_t)off * sizeof(D), ylo);
        } else {
#pragma unroll
            for (int e = 0; e < PPS; ++e) {
                float y0, y1;
                rotate(to_f32(lo[u].v[e]), to_f32(hi[u].v[e]), c[e], s[e], y0, y1);
                ylo.v[e] = from_f32<D>(y0);
                yhi.v[e] = from_f32<D>(y1);
            }
            if (!(CACHE != kNoCache && plane == 1 && kv.skip_k_inplace)) {
                store_wt(row_s, (uint32_t)off * sizeof(D), ylo);
                store_wt(row_s, (uint32_t)(off + NP) * sizeof(D), yhi);
            }
        }
        if constexpr (CACHE != kNoCache) {
            if (plane == 1 && kd) {
                if (cache_aligned) {
                    store_wt(kd, (uint32_t)off * sizeof(D), ylo);
                    if constexpr (HALF) store_wt(kd, (uint32_t)(off + NP) * sizeof(D), yhi);
                } else {
                    store_cache<D>(kd + off, ylo, false);
                    if constexpr (HALF) store_cache<D>(kd + off + NP, yhi, false);
                }
            }
        }
    }
}

// Exchange a 16-byte chunk with the lane 8 places away inside its 16-lane row
// (lane i <-> lane i^8): the rotate-half partner when a head row is 16 chunks.
template <typename V>
__device__ __forceinline__ V swap8(const V& a) {
    static_assert(sizeof(V) == 16, "16-byte chunks");
    const u32x4 x = __builtin_bit_cast(u32x4, a);
    u32x4 r;
    // DPP row_ror:8 -- lane i of each 16-lane row reads lane (i + 8) mod 16
    r.x = __builtin_amdgcn_mov_dpp((int)x.x, 0x128, 0xF, 0xF, false);
    r.y = __builtin_amdgcn_mov_dpp((int)x.y, 0x128, 0xF, 0xF, false);
    r.z = __builtin_amdgcn_mov_dpp((int)x.z, 0x128, 0xF, 0xF, false);
    r.w = __builtin_amdgcn_mov_dpp((int)x.w, 0x128, 0xF, 0xF, false);
    return __builtin_bit_cast(V, r);
}

typedef const __attribute__((address_space(1))) u32x4 g_u32x4;

// RoPE without a cache for 256-byte head rows (binary16 head_dim 128): a
// token's Q head rows, then its K head rows, are walked in 1 KiB units of four
// rows, kUnitsPerWave units per wavefront, consecutive wavefronts of the grid
// per token (no barriers).  Lane l of a unit owns chunk l%16 of head row l/16,
// so every load and store instruction is one contiguous 1 KiB span of a row
// (or whole 256 B rows where a unit straddles Q and K).  A rotate-half pair
// (i, i+64) lies in chunks c and c^8 of the same row: each lane takes its
// partner's chunk with one DPP row rotation and computes its own half of the
// pair.  Measured at C5 (Q 32 heads, K 8 heads, 8192 tokens): 5-6% faster
// than the plane kernel; with the paged cache (rows of three planes) and for
// binary32 head_dim 64 the plane kernel stays faster, so only this case uses it.
constexpr int kUnitsPerWave = 2;
constexpr int kUnitBlock = 64;

template <int PAIRING>
__global__ __launch_bounds__(kUnitBlock) void rope_units(_Float16* q, _Float16* k, int n_tokens,
                                                         int hq, int hk, int wpt, long long qs,
                                                         long long ks,
                                                         const int32_t* __restrict__ positions,
                                                         int pos_offset, InvFreq inv) {
    using D = _Float16;
    using V = Vec<D, 8>;
    constexpr int U = kUnitsPerWave;
    constexpr int NP = 64;                     // pairs per 128-wide head
    constexpr bool HALF = PAIRING == QL_ROPE_HALF;
    constexpr int PPL = HALF ? 8 : 4;          // pairs a lane's chunk touches

    // wavefront index made scalar: everything indexed by the token (its
    // position, the row bases) is then read with scalar loads, on the counter
    // the row loads do not use
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    const long long g = (long long)blockIdx.x * (kUnitBlock / kWave) + wid;
    const int t = (int)(g / wpt);
    if (t >= n_tokens) return;                 // wavefront-uniform; no barriers below
    const int u0 = (int)(g - (long long)t * wpt) * U;
    const int lane = threadIdx.x & (kWave - 1);
    const int c = lane & 15;                   // chunk in the head row
    const int htot = hq + hk;
    D* qt = q ? q + (long long)t * qs : nullptr;
    D* kt = k ? k + (long long)t * ks : nullptr;

    // The one per-lane read besides the rows (inv_freq of this lane's pair) is
    // issued first: vector loads retire in issue order, so waiting for it does
    // not wait for the rows.
    const float inv_l = inv.v[lane % NP];
    asm volatile("" ::: "memory");             // keep the row loads after it

    // Every lane loads (lanes past the last head re-read the last head's row
    // and store nothing): with no branch around the loads, the wait before the
    // trig covers the inv_freq read alone.
    V x[U];
    uintptr_t row[U];
    bool live[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
        const int hl = ((u0 + i) << 2) + (lane >> 4);
        live[i] = hl < htot;
        const int h = live[i] ? hl : htot - 1;
        // rows selected as integer addresses (see rope_fast), loaded in the
        // global address space (a generic load would also count against the
        // LDS counter, so the cross-lane reads below would wait for it)
        row[i] = h < hq ? reinterpret_cast<uintptr_t>(qt) + 256 * (size_t)h
                        : reinterpret_cast<uintptr_t>(kt) + 256 * (size_t)(h - hq);
        x[i] = __builtin_bit_cast(V, __builtin_nontemporal_load(
                                         reinterpret_cast<g_u32x4*>(row[i] + 16 * (size_t)c)));
    }

    const int pos = positions ? ld_scalar(positions + t) : pos_offset + t;
    float c_own, s_own;
    trig((float)pos * inv_l, c_own, s_own);
    const int p0 = HALF ? (c & 7) * 8 : c * 4;  // first pair of this lane's chunk
    float cs[PPL], sn[PPL];
#pragma unroll
    for (int e = 0; e < PPL; ++e) {
        cs[e] = __shfl(c_own, p0 + e, kWave);
        sn[e] = __shfl(s_own, p0 + e, kWave);
    }

    // the unit's rows come from Q and K: the stores go out from the wavefront's
    // scalar Q or K row base (write-through buffer stores, as the plane kernel)
    D* qrow = uniform(qt);
    D* krow = uniform(kt);
#pragma unroll
    for (int i = 0; i < U; ++i) {
        const V p = HALF ? swap8(x[i]) : x[i];  // every lane joins the exchange
        V y;
        if constexpr (HALF) {
            const bool lo = c < 8;              // lo lanes hold x0, hi lanes x1
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float a = to_f32(x[i].v[e]), b = to_f32(p.v[e]);
                float y0, y1;
                rotate(lo ? a : b, lo ? b : a, cs[e], sn[e], y0, y1);
                y.v[e] = from_f32<D>(lo ? y0 : y1);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float y0, y1;
                rotate(to_f32(x[i].v[2 * e]), to_f32(x[i].v[2 * e + 1]), cs[e], sn[e], y0, y1);
                y.v[2 * e] = from_f32<D>(y0);
                y.v[2 * e + 1] = from_f32<D>(y1);
            }
        }
        if (live[i]) {
            const int h = ((u0 + i) << 2) + (lane >> 4);
            if (h < hq) store_wt(qrow, (uint32_t)(256 * h + 16 * c), y);
            else store_wt(krow, (uint32_t)(256 * (h - hq) + 16 * c), y);
        }
    }
}

// Launch the plane kernel: groups per plane chosen so a lane owns at most
// MAXU chunks and there are enough wavefronts to fill the device.
template <typename D, int PAIRING, int HD, int CACHE>
hipError_t launch_planes(D* q, D* k, int n_tokens, int hq, int hk, long long qs, long long ks,
                         const int32_t* positions, int pos_offset, const InvFreq& inv,
                         const KvDst<D>& kv, int mix, hipStream_t stream) {
    constexpr int W = vec16<D>();
    constexpr int S = (HD / 2) / (PAIRING == QL_ROPE_HALF ? W : W / 2);
    // a rotate-half slot is two 16-byte chunks, an interleaved slot one: keep
    // 2 KiB per lane-set in flight either way
    constexpr int MAXU = PAIRING == QL_ROPE_HALF ? 2 : 4;
    const int hcap = (kWave * MAXU) / S;  // heads per wavefront at most
    const int hpw_q = hq > 0 ? (hq < hcap ? hq : hcap) : 1;
    const int hpw_k = hk > 0 ? (hk < hcap ? hk : hcap) : 1;
    const int gq = hq > 0 ? (hq + hpw_q - 1) / hpw_q : 0;
    const int gk = hk > 0 ? (hk + hpw_k - 1) / hpw_k : 0;
    const int gy = gq + gk + (CACHE != kNoCache ? gk : 0);
    const unsigned gx = qlh::blocks_for(n_tokens, kBlock / kWave);
    dim3 grid(gx, gy);
    if (mix > 0) {
        const long long n = ((long long)gx + mix - 1) / mix * mix * gy;
        QL_CHECK_ARG(n <= 0x7fffffffLL);
        grid = dim3((unsigned)n, 1);
    }
    hipLaunchKernelGGL((rope_planes<D, PAIRING, HD, MAXU, CACHE>), grid, dim3(kBlock), 0, stream, q, k,
                       n_tokens, hq, hk, qs, ks, positions, pos_offset, inv, gq, gk, hpw_q, hpw_k, kv, mix);
    return hipGetLastError();
}

template <typename D, int CACHE>
hipError_t launch_planes_hd(int d, int pairing, D* q, D* k, int n_tokens, int hq, int hk,
                            long long qs, long long ks, const int32_t* positions, int pos_offset,
                            const InvFreq& inv, const KvDst<D>& kv, int mix, hipStream_t stream) {
    if (d == 128) {
        if constexpr (CACHE == kNoCache && sizeof(D) == 2) {
            return hipErrorInvalidValue;   // binary16 head_dim 128 without a cache runs rope_units
        } else {
            if (pairing == QL_ROPE_HALF)
                return launch_planes<D, QL_ROPE_HALF, 128, CACHE>(q, k, n_tokens, hq, hk, qs, ks,
                                                                  positions, pos_offset, inv, kv, mix,
                                                                  stream);
            return launch_planes<D, QL_ROPE_INTERLEAVED, 128, CACHE>(q, k, n_tokens, hq, hk, qs,
                                                                     ks, positions, pos_offset,
                                                                     inv, kv, mix, stream);
        }
    }
    if (pairing == QL_ROPE_HALF)
        return launch_planes<D, QL_ROPE_HALF, 64, CACHE>(q, k, n_tokens, hq, hk, qs, ks, positions,
                                                         pos_offset, inv, kv, mix, stream);
    return launch_planes<D, QL_ROPE_INTERLEAVED, 64, CACHE>(q, k, n_tokens, hq, hk, qs, ks,
                                                            positions, pos_offset, inv, kv, mix, stream);
}

// Token blocks per plane group of the plane kernel's interleaved grid (mix > 0),
// used when the Q, K (and V) rows interleave in one buffer: equal row strides and
// every plane's first row inside one row's span, as in a fused QKV projection's
// output.  Measured on MI355X, fused RoPE + paged append at 8192 tokens, Q 32 and
// K 8 heads of 128 in 12 KiB QKV rows: planes along y 43.1 us, interleaved every
// 1 / 4 / 16 token blocks 39.0 / 38.2 / 37.8 us; on separate Q, K, V buffers the
// planes along y stay faster (36.0 against 36.7-37.6 us).  Bit-identical either way.
constexpr int kRopeMixBlocks = 16;

template <typename D>
int rope_mix(const D* q, const D* k, const D* v, long long qs, long long ks, long long vs) {
    if (!q || !k || qs != ks || (v && vs != qs)) return 0;
    uintptr_t lo = reinterpret_cast<uintptr_t>(q), hi = lo;
    for (const D* p : {k, v}) {
        if (!p) continue;
        lo = std::min(lo, reinterpret_cast<uintptr_t>(p));
        hi = std::max(hi, reinterpret_cast<uintptr_t>(p));
    }
    return hi - lo < (uintptr_t)qs * sizeof(D) ? kRopeMixBlocks : 0;
}

constexpr int kRopeMaxU = 4;        // chunks (or chunk pairs) per lane
constexpr int kRopeTargetWaves = 16384;

// rope_fast's launch: heads per wavefront at most kRopeMaxU passes of the whole heads
// that fit 64 lanes, split further while tokens alone give fewer than
// kRopeTargetWaves wavefronts.
template <typename D, int CACHE, int NP>
hipError_t launch_fast_heads(D* q, D* k, int n_tokens, int hq, int hk, int d, int64_t qs, int64_t ks,
                             const int32_t* positions, int pos_offset, const InvFreqN<NP>& inv, int pairing,
                             int slots, unsigned gx, const KvDst<D>& kv, hipStream_t stream) {
    const int htot = hq + hk + (CACHE != kNoCache ? hk : 0);
    const int hcap = (kWave / slots) * kRopeMaxU;   // whole heads per wavefront pass
    int groups = (kRopeTargetWaves + n_tokens - 1) / n_tokens;
    groups = groups < 1 ? 1 : (groups > htot ? htot : groups);
    int hpw = (htot + groups - 1) / groups;
    hpw = hpw > hcap ? hcap : hpw;
    groups = (htot + hpw - 1) / hpw;
    if (pairing == QL_ROPE_INTERLEAVED)
        hipLaunchKernelGGL((rope_fast<D, QL_ROPE_INTERLEAVED, kRopeMaxU, CACHE, NP>), dim3(gx, groups),
                           dim3(kBlock), 0, stream, q, k, n_tokens, hq, hk, d, (long long)qs, (long long)ks,
                           positions, pos_offset, inv, hpw, kv);
    else
        hipLaunchKernelGGL((rope_fast<D, QL_ROPE_HALF, kRopeMaxU, CACHE, NP>), dim3(gx, groups), dim3(kBlock), 0,
                           stream, q, k, n_tokens, hq, hk, d, (long long)qs, (long long)ks, positions, pos_offset,
                           inv, hpw, kv);
    return hipGetLastError();
}

template <typename D, int CACHE>
hipError_t rope_dispatch(D* q, D* k, int n_tokens, int hq, int hk, int d, int64_t qs,
                         int64_t ks, const int32_t* positions, int pos_offset, float theta,
                         int pairing, KvDst<D> kv, hipStream_t stream) {
    QL_CHECK_ARG(n_tokens >= 0 && hq >= 0 && hk >= 0);
    QL_CHECK_ARG(pairing == QL_ROPE_INTERLEAVED || pairing == QL_ROPE_HALF);
    QL_CHECK_ARG(d > 0 && d % 2 == 0 && d <= 2048);
    if (CACHE != kNoCache) {
        QL_CHECK_ARG(k && kv.v && hk > 0 && kv.vs >= (int64_t)hk * d);
    }
    if (!q) hq = 0;
    if (!k) hk = 0;
    if (n_tokens == 0 || hq + hk == 0) return hipSuccess;
    QL_CHECK_ARG(!q || qs >= (int64_t)hq * d);
    QL_CHECK_ARG(!k || ks >= (int64_t)hk * d);
    QL_CHECK_ARG(theta > 0.0f);

    constexpr int W = vec16<D>();
    const int npairs = d / 2;
    const int pps = pairing == QL_ROPE_INTERLEAVED ? W / 2 : W;
    const int slots = npairs % pps == 0 ? npairs / pps : 0;
    const bool tile_ok = npairs <= 128 && slots > 0;
    bool align_ok = rows_aligned16(q, qs * (int64_t)sizeof(D)) &&
                    rows_aligned16(k, ks * (int64_t)sizeof(D)) && (d * (int)sizeof(D)) % 16 == 0;
    if (CACHE != kNoCache) align_ok = align_ok && rows_aligned16(kv.v, kv.vs * (int64_t)sizeof(D));
    if (CACHE == kContigCache)
        align_ok = align_ok && qlh::aligned16(kv.kc) && qlh::aligned16(kv.vc);
    const int tok_per_block = kBlock / kWave;
    const unsigned gx = qlh::blocks_for(n_tokens, tok_per_block);
    if (tile_ok && align_ok) {
        InvFreq inv;
        for (int i = 0; i < 64; ++i) inv.v[i] = i < npairs ? host_inv_freq(i, d, theta) : 0.0f;
        if (npairs > 64) {   // head_dim 130 .. 256: the vector path with a 128-pair table
            InvFreqN<128> inv2;
            for (int i = 0; i < 128; ++i) inv2.v[i] = i < npairs ? host_inv_freq(i, d, theta) : 0.0f;
            return launch_fast_heads<D, CACHE, 128>(q, k, n_tokens, hq, hk, d, qs, ks, positions, pos_offset,
                                                    inv2, pairing, slots, gx, kv, stream);
        }
        if constexpr (CACHE == kNoCache && sizeof(D) == 2) {
            if (d == 128) {
                const int units = (hq + hk + 3) / 4;
                const int wpt = (units + kUnitsPerWave - 1) / kUnitsPerWave;
                const long long waves = (long long)n_tokens * wpt;
                const long long blocks = (waves + kUnitBlock / kWave - 1) / (kUnitBlock / kWave);
                QL_CHECK_ARG(blocks <= 0x7fffffffLL);
                if (pairing == QL_ROPE_HALF)
                    hipLaunchKernelGGL((rope_units<QL_ROPE_HALF>), dim3((unsigned)blocks),
                                       dim3(kUnitBlock), 0, stream, q, k, n_tokens, hq, hk, wpt,
                                       (long long)qs, (long long)ks, positions, pos_offset, inv);
                else
                    hipLaunchKernelGGL((rope_units<QL_ROPE_INTERLEAVED>), dim3((unsigned)blocks),
                                       dim3(kUnitBlock), 0, stream, q, k, n_tokens, hq, hk, wpt,
                                       (long long)qs, (long long)ks, positions, pos_offset, inv);
                return hipGetLastError();
            }
        }
        if (d == 64 || d == 128) {
            const int mix = rope_mix<D>(hq ? q : nullptr, hk ? k : nullptr, CACHE != kNoCache ? kv.v : nullptr,
                                        (long long)qs, (long long)ks, kv.vs);
            return launch_planes_hd<D, CACHE>(d, pairing, q, k, n_tokens, hq, hk, (long long)qs,
                                              (long long)ks, positions, pos_offset, inv, kv, mix, stream);
        }
        return launch_fast_heads<D, CACHE, 64>(q, k, n_tokens, hq, hk, d, qs, ks, positions, pos_offset, inv,
                                               pairing, slots, gx, kv, stream);
    } else {
        if (pairing == QL_ROPE_INTERLEAVED)
            hipLaunchKernelGGL((rope_generic<D, QL_ROPE_INTERLEAVED, CACHE>), dim3(gx),
                               dim3(kBlock), 0, stream, q, k, n_tokens, hq, hk, d, (long long)qs,
                               (long long)ks, positions, pos_offset, theta, kv);
        else
            hipLaunchKernelGGL((rope_generic<D, QL_ROPE_HALF, CACHE>), dim3(gx), dim3(kBlock), 0,
                               stream, q, k, n_tokens, hq, hk, d, (long long)qs, (long long)ks,
                               positions, pos_offset, theta, kv);
    }
    return hipGetLastError();
}

template <typename D>
KvDst<D> no_cache() {
    KvDst<D> kv{};
    return kv;
}

}  // namespace

extern "C" hipError_t ql_rope_f32(float* q, float* k, int n_tokens, int n_heads,
                                  int n_kv_heads, int head_dim, int64_t q_row_stride,
                                  int64_t k_row_stride, const int32_t* positions,
                                  int pos_offset, float theta, int pairing,
                                  hipStream_t stream) {
    return rope_dispatch<float, kNoCache>(q, k, n_tokens, n_heads, n_kv_heads, head_dim,
                                          q_row_stride, k_row_stride, positions, pos_offset,
                                          theta, pairing, no_cache<float>(), stream);
}

extern "C" hipError_t ql_rope_f16(uint16_t* q, uint16_t* k, int n_tokens, int n_heads,
                                  int n_kv_heads, int head_dim, int64_t q_row_stride,
                                  int64_t k_row_stride, const int32_t* positions,
                                  int pos_offset, float theta, int pairing,
                                  hipStream_t stream) {
    return rope_dispatch<_Float16, kNoCache>(
        reinterpret_cast<_Float16*>(q), reinterpret_cast<_Float16*>(k), n_tokens, n_heads,
        n_kv_heads, head_dim, q_row_stride, k_row_stride, positions, pos_offset, theta, pairing,
        no_cache<_Float16>(), stream);
}

namespace {

hipError_t rope_paged_entry(uint16_t* q, uint16_t* k, const uint16_t* v, int n_tokens, int n_heads,
                            int n_kv_heads, int head_dim, int64_t q_row_stride, int64_t k_row_stride,
                            int64_t v_row_stride, const int32_t* positions, int pos_offset,
                            float theta, int pairing, uint16_t* const* k_blocks,
                            uint16_t* const* v_blocks, int n_blocks, const int32_t* slot_mapping,
                            int layer, int n_layers, bool skip_k_inplace, hipStream_t stream) {
    QL_CHECK_ARG(n_layers > 0 && layer >= 0 && layer < n_layers && n_blocks >= 0);
    QL_CHECK_ARG((long long)n_kv_heads * head_dim <= (1LL << 30));
    QL_CHECK_ARG(n_tokens <= 0 || (k_blocks && v_blocks && slot_mapping));
    KvDst<_Float16> kv{};
    kv.kb = reinterpret_cast<_Float16* const*>(k_blocks);
    kv.vb = reinterpret_cast<_Float16* const*>(v_blocks);
    kv.slots = slot_mapping;
    kv.n_blocks = n_blocks;
    kv.v = reinterpret_cast<const _Float16*>(v);
    kv.vs = v_row_stride;
    kv.layer = layer;
    kv.skip_k_inplace = skip_k_inplace ? 1 : 0;
    return rope_dispatch<_Float16, kPagedCache>(
        reinterpret_cast<_Float16*>(q), reinterpret_cast<_Float16*>(k), n_tokens, n_heads,
        n_kv_heads, head_dim, q_row_stride, k_row_stride, positions, pos_offset, theta, pairing,
        kv, stream);
}

}  // namespace

extern "C" hipError_t ql_rope_paged_kv_append_f16(
    uint16_t* q, uint16_t* k, const uint16_t* v, int n_tokens, int n_heads, int n_kv_heads,
    int head_dim, int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
    const int32_t* positions, int pos_offset, float theta, int pairing,
    uint16_t* const* k_blocks, uint16_t* const* v_blocks, int n_blocks,
    const int32_t* slot_mapping, int layer, int n_layers, hipStream_t stream) {
    return rope_paged_entry(q, k, v, n_tokens, n_heads, n_kv_heads, head_dim, q_row_stride,
                            k_row_stride, v_row_stride, positions, pos_offset, theta, pairing,
                            k_blocks, v_blocks, n_blocks, slot_mapping, layer, n_layers, false,
                            stream);
}

extern "C" hipError_t ql_rope_q_paged_kv_append_f16(
    uint16_t* q, const uint16_t* k, const uint16_t* v, int n_tokens, int n_heads, int n_kv_heads,
    int head_dim, int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
    const int32_t* positions, int pos_offset, float theta, int pairing,
    uint16_t* const* k_blocks, uint16_t* const* v_blocks, int n_blocks,
    const int32_t* slot_mapping, int layer, int n_layers, hipStream_t stream) {
    return rope_paged_entry(q, const_cast<uint16_t*>(k), v, n_tokens, n_heads, n_kv_heads, head_dim,
                            q_row_stride, k_row_stride, v_row_stride, positions, pos_offset, theta,
                            pairing, k_blocks, v_blocks, n_blocks, slot_mapping, layer, n_layers,
                            true, stream);
}

template <typename D>
hipError_t rope_contig_entry(D* q, D* k, const D* v, int n_tokens, int n_heads, int n_kv_heads,
                             int head_dim, int64_t qs, int64_t ks, int64_t vs,
                             const int32_t* positions, int pos_offset, float theta, int pairing,
                             D* k_cache, D* v_cache, int layer, int pos, int max_seq,
                             int n_layers, hipStream_t stream) {
    QL_CHECK_ARG(n_layers > 0 && layer >= 0 && layer < n_layers && max_seq > 0);
    QL_CHECK_ARG(n_tokens >= 0 && pos >= 0 && (long long)pos + n_tokens <= max_seq);
    QL_CHECK_ARG(n_tokens == 0 || (k_cache && v_cache));
    KvDst<D> kv{};
    kv.kc = k_cache;
    kv.vc = v_cache;
    kv.pos0 = pos;
    kv.max_seq = max_seq;
    kv.v = v;
    kv.vs = vs;
    kv.layer = layer;
    return rope_dispatch<D, kContigCache>(q, k, n_tokens, n_heads, n_kv_heads, head_dim, qs, ks,
                                          positions, pos_offset, theta, pairing, kv, stream);
}

extern "C" hipError_t ql_rope_kv_append_f16(
    uint16_t* q, uint16_t* k, const uint16_t* v, int n_tokens, int n_heads, int n_kv_heads,
    int head_dim, int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
    const int32_t* positions, int pos_offset, float theta, int pairing, uint16_t* k_cache,
    uint16_t* v_cache, int layer, int pos, int max_seq, int n_layers, hipStream_t stream) {
    return rope_contig_entry<_Float16>(
        reinterpret_cast<_Float16*>(q), reinterpret_cast<_Float16*>(k),
        reinterpret_cast<const _Float16*>(v), n_tokens, n_heads, n_kv_heads, head_dim,
        q_row_stride, k_row_stride, v_row_stride, positions, pos_offset, theta, pairing,
        reinterpret_cast<_Float16*>(k_cache), reinterpret_cast<_Float16*>(v_cache), layer, pos,
        max_seq, n_layers, stream);
}

extern "C" hipError_t ql_rope_kv_append_f32(
    float* q, float* k, const float* v, int n_tokens, int n_heads, int n_kv_heads, int head_dim,
    int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride, const int32_t* positions,
    int pos_offset, float theta, int pairing, float* k_cache, float* v_cache, int layer, int pos,
    int max_seq, int n_layers, hipStream_t stream) {
    return rope_contig_entry<float>(q, k, v, n_tokens, n_heads, n_kv_heads, head_dim,
                                    q_row_stride, k_row_stride, v_row_stride, positions,
                                    pos_offset, theta, pairing, k_cache, v_cache, layer, pos,
                                    max_seq, n_layers, stream);
}
