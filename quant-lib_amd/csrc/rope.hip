// rope.hip -- rotary position embedding on Q and K (GQA head counts) in one
// launch, in place, for gfx950.
//
// Arithmetic per pair i of a head at position pos (kernels/rope.cu:35-41,
// kernels/fp16_ops.cu:54-62), with the transcendental steps made accurate so a
// CPU restatement can reproduce them:
//   e   = (2i) / d                       fp32 division, as the reference
//   inv = 1 / (float)pow(theta, e)       pow in fp64, rounded to fp32
//   a   = (float)pos * inv               fp32
//   c   = (float)cos(a), s = (float)sin(a)   evaluated in fp64, rounded to fp32
//   y0  = fma(x0, c, -(x1*s)),  y1 = fma(x0, s, x1*c)
// Pairing: interleaved (2i, 2i+1) as the reference, or rotate-half (i, i+d/2).
//
// Fast path (d/2 <= 64 pairs, 16-byte aligned rows, head chunks that tile a
// wavefront): one wavefront per (token, group of heads).  Lane l evaluates the
// trig of pair l once per token in fp64 and the values are redistributed with
// cross-lane permutes, so the fp64 work is one sincos per pair per token,
// shared by all heads of the group.  Each lane then owns one 16-byte chunk
// position j of the head vector and walks the heads; every wavefront access is
// a contiguous, coalesced 16-byte-per-lane span.
#include "ql_common.hpp"
#include "quantlib_amd.h"

namespace {

using namespace ql;

__device__ __forceinline__ void rope_trig(int pos, int pair, int d, float theta, float& c,
                                          float& s) {
    const float e = (2.0f * (float)pair) / (float)d;
    const float p = (float)pow((double)theta, (double)e);
    const float inv = 1.0f / p;
    const float a = (float)pos * inv;
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

constexpr int kSlotsPerIter = 4;  // 16-byte chunks (pairs of chunks) in flight per lane

template <typename D, int PAIRING>
__global__ __launch_bounds__(kBlock) void rope_fast(D* q, D* k, int n_tokens, int hq, int hk,
                                                    int d, long long qs, long long ks,
                                                    const int32_t* __restrict__ positions,
                                                    int pos_offset, float theta,
                                                    int heads_per_wave) {
    constexpr int W = vec16<D>();
    constexpr int PPS = PAIRING == QL_ROPE_INTERLEAVED ? W / 2 : W;  // pairs per slot
    using V = Vec<D, W>;

    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * (kBlock / kWave) + (threadIdx.x / kWave);
    if (t >= n_tokens) return;  // wavefront-uniform; no barriers below
    const int npairs = d >> 1;
    const int pos = positions ? positions[t] : pos_offset + t;

    float c_own, s_own;
    rope_trig(pos, lane % npairs, d, theta, c_own, s_own);

    const int S = npairs / PPS;  // slots per head; divides 64
    const int j = lane % S;
    float c[PPS], s[PPS];
#pragma unroll
    for (int e = 0; e < PPS; ++e) {
        c[e] = __shfl(c_own, j * PPS + e, kWave);
        s[e] = __shfl(s_own, j * PPS + e, kWave);
    }

    const int h0 = blockIdx.y * heads_per_wave;
    const int h1 = min(hq + hk, h0 + heads_per_wave);
    const int nslots = (h1 - h0) * S;
    D* qt = q ? q + (long long)t * qs : nullptr;
    D* kt = k ? k + (long long)t * ks : nullptr;

    for (int base = lane; base < nslots; base += kWave * kSlotsPerIter) {
        V lo[kSlotsPerIter];
        V hi[PAIRING == QL_ROPE_HALF ? kSlotsPerIter : 1];
        V* plo[kSlotsPerIter];
#pragma unroll
        for (int u = 0; u < kSlotsPerIter; ++u) {
            const int sl = base + u * kWave;
            plo[u] = nullptr;
            if (sl < nslots) {
                const int h = h0 + sl / S;
                D* head = h < hq ? qt + (long long)h * d : kt + (long long)(h - hq) * d;
                plo[u] = reinterpret_cast<V*>(head) + j;
                lo[u] = *plo[u];
                if constexpr (PAIRING == QL_ROPE_HALF)
                    hi[u] = *reinterpret_cast<V*>(reinterpret_cast<D*>(plo[u]) + npairs);
            }
        }
#pragma unroll
        for (int u = 0; u < kSlotsPerIter; ++u) {
            if (!plo[u]) continue;
            if constexpr (PAIRING == QL_ROPE_INTERLEAVED) {
                V y;
#pragma unroll
                for (int e = 0; e < PPS; ++e) {
                    float y0, y1;
                    rotate(to_f32(lo[u].v[2 * e]), to_f32(lo[u].v[2 * e + 1]), c[e], s[e], y0,
                           y1);
                    y.v[2 * e] = from_f32<D>(y0);
                    y.v[2 * e + 1] = from_f32<D>(y1);
                }
                *plo[u] = y;
            } else {
                V ylo, yhi;
#pragma unroll
                for (int e = 0; e < PPS; ++e) {
                    float y0, y1;
                    rotate(to_f32(lo[u].v[e]), to_f32(hi[u].v[e]), c[e], s[e], y0, y1);
                    ylo.v[e] = from_f32<D>(y0);
                    yhi.v[e] = from_f32<D>(y1);
                }
                *plo[u] = ylo;
                *reinterpret_cast<V*>(reinterpret_cast<D*>(plo[u]) + npairs) = yhi;
            }
        }
    }
}

// Any even head_dim (<= 2048), any alignment: one wavefront per token, lane =
// pair index (strided), trig once per (token, pair), then every head.
template <typename D, int PAIRING>
__global__ __launch_bounds__(kBlock) void rope_generic(D* q, D* k, int n_tokens, int hq, int hk,
                                                       int d, long long qs, long long ks,
                                                       const int32_t* __restrict__ positions,
                                                       int pos_offset, float theta) {
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * (kBlock / kWave) + (threadIdx.x / kWave);
    if (t >= n_tokens) return;
    const int npairs = d >> 1;
    const int pos = positions ? positions[t] : pos_offset + t;
    for (int p = lane; p < npairs; p += kWave) {
        float c, s;
        rope_trig(pos, p, d, theta, c, s);
        const int i0 = PAIRING == QL_ROPE_INTERLEAVED ? 2 * p : p;
        const int i1 = PAIRING == QL_ROPE_INTERLEAVED ? 2 * p + 1 : p + npairs;
        for (int h = 0; h < hq + hk; ++h) {
            D* head = h < hq ? q + (long long)t * qs + (long long)h * d
                             : k + (long long)t * ks + (long long)(h - hq) * d;
            float y0, y1;
            rotate(to_f32(head[i0]), to_f32(head[i1]), c, s, y0, y1);
            head[i0] = from_f32<D>(y0);
            head[i1] = from_f32<D>(y1);
        }
    }
}

template <typename D>
hipError_t rope_dispatch(D* q, D* k, int n_tokens, int hq, int hk, int d, int64_t qs,
                         int64_t ks, const int32_t* positions, int pos_offset, float theta,
                         int pairing, hipStream_t stream) {
    QL_CHECK_ARG(n_tokens >= 0 && hq >= 0 && hk >= 0);
    QL_CHECK_ARG(pairing == QL_ROPE_INTERLEAVED || pairing == QL_ROPE_HALF);
    QL_CHECK_ARG(d > 0 && d % 2 == 0 && d <= 2048);
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
    const bool tile_ok = npairs <= 64 && slots > 0 && 64 % slots == 0;
    const bool align_ok = (!q || (qlh::aligned16(q) && (qs * (int64_t)sizeof(D)) % 16 == 0)) &&
                          (!k || (qlh::aligned16(k) && (ks * (int64_t)sizeof(D)) % 16 == 0)) &&
                          (d * (int)sizeof(D)) % 16 == 0;
    const int tok_per_block = kBlock / kWave;
    const unsigned gx = qlh::blocks_for(n_tokens, tok_per_block);
    if (tile_ok && align_ok) {
        // Split heads over more wavefronts when tokens alone do not give
        // ~8K wavefronts (32 per CU on 256 CUs).
        const int htot = hq + hk;
        int groups = (8192 + n_tokens - 1) / n_tokens;
        groups = groups < 1 ? 1 : (groups > htot ? htot : groups);
        const int hpw = (htot + groups - 1) / groups;
        groups = (htot + hpw - 1) / hpw;
        if (pairing == QL_ROPE_INTERLEAVED)
            hipLaunchKernelGGL((rope_fast<D, QL_ROPE_INTERLEAVED>), dim3(gx, groups),
                               dim3(kBlock), 0, stream, q, k, n_tokens, hq, hk, d,
                               (long long)qs, (long long)ks, positions, pos_offset, theta, hpw);
        else
            hipLaunchKernelGGL((rope_fast<D, QL_ROPE_HALF>), dim3(gx, groups), dim3(kBlock), 0,
                               stream, q, k, n_tokens, hq, hk, d, (long long)qs, (long long)ks,
                               positions, pos_offset, theta, hpw);
    } else {
        if (pairing == QL_ROPE_INTERLEAVED)
            hipLaunchKernelGGL((rope_generic<D, QL_ROPE_INTERLEAVED>), dim3(gx), dim3(kBlock), 0,
                               stream, q, k, n_tokens, hq, hk, d, (long long)qs, (long long)ks,
                               positions, pos_offset, theta);
        else
            hipLaunchKernelGGL((rope_generic<D, QL_ROPE_HALF>), dim3(gx), dim3(kBlock), 0,
                               stream, q, k, n_tokens, hq, hk, d, (long long)qs, (long long)ks,
                               positions, pos_offset, theta);
    }
    return hipGetLastError();
}

}  // namespace

extern "C" hipError_t ql_rope_f32(float* q, float* k, int n_tokens, int n_heads,
                                  int n_kv_heads, int head_dim, int64_t q_row_stride,
                                  int64_t k_row_stride, const int32_t* positions,
                                  int pos_offset, float theta, int pairing,
                                  hipStream_t stream) {
    return rope_dispatch<float>(q, k, n_tokens, n_heads, n_kv_heads, head_dim, q_row_stride,
                                k_row_stride, positions, pos_offset, theta, pairing, stream);
}

extern "C" hipError_t ql_rope_f16(uint16_t* q, uint16_t* k, int n_tokens, int n_heads,
                                  int n_kv_heads, int head_dim, int64_t q_row_stride,
                                  int64_t k_row_stride, const int32_t* positions,
                                  int pos_offset, float theta, int pairing,
                                  hipStream_t stream) {
    return rope_dispatch<_Float16>(reinterpret_cast<_Float16*>(q),
                                   reinterpret_cast<_Float16*>(k), n_tokens, n_heads,
                                   n_kv_heads, head_dim, q_row_stride, k_row_stride, positions,
                                   pos_offset, theta, pairing, stream);
}
