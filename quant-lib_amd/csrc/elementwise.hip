// elementwise.hip -- streaming kernels for gfx950: SwiGLU, residual add,
// binary16 <-> fp32 conversions, and the contiguous KV-cache append (a pair of
// copies).
//
// Every kernel moves each input once and each output once with 16-byte
// accesses.  A workgroup owns a contiguous chunk of 256*U vectors; thread t
// touches vectors t, t+256, ... so each wavefront instruction covers one
// contiguous 1 KiB span, and all U loads of a thread are issued before any
// arithmetic.  Elements past the last whole vector (n % W) are handled by
// workgroup 0.  Unaligned pointers take the same kernels with W = 1.
#include "ql_common.hpp"
#include "quantlib_amd.h"

namespace {

using namespace ql;

constexpr int kUnroll = 4;

// SwiGLU: out = (g / (1 + exp(-g))) * u  (kernels/feedforward.cu:4-6,24;
// kernels/fp16_ops.cu:74-77).  The quotient is g * rcp(1 + e) with v_rcp_f32
// (1 ulp); 1 + e >= 1 so it is well conditioned.  v_rcp_f32 flushes subnormal
// results, so for fp32 output a divisor above 2^126 is pre-scaled by 2^-64 and
// the product rescaled (the final multiply keeps subnormals); e = inf still
// gives the reference's signed zero.  binary16 output cannot represent that
// range, so its path skips the rescale.
struct SwigluOp {
    template <typename D>
    __device__ static float apply(float g, float u) {
        if constexpr (sizeof(D) == 4) {
            const float x = 1.0f + exp_f32(-g);
            const bool big = x > 0x1p126f;
            float q = g * __builtin_amdgcn_rcpf(big ? x * 0x1p-64f : x);
            q = big ? q * 0x1p-64f : q;
            return q * u;
        } else {
            return (g * __builtin_amdgcn_rcpf(1.0f + exp_f32_fast(-g))) * u;
        }
    }
};

// Residual add: x = round_D(x + d)  (src/forward.cu:128-130; kernels/fp16_ops.cu:92-100)
struct AddOp {
    template <typename D>
    __device__ static float apply(float x, float d) { return x + d; }
};

// out[i] = op(a[i], b[i]) over n elements; out may alias a (in-place add).
// BS threads per workgroup, U vectors per thread, NT = nontemporal loads and
// stores.  Measured on MI355X (buffers rotated past the MALL, clocks warm):
// one 16-byte vector per thread with nontemporal access streams fastest
// (unrolling further lowers occupancy without adding useful bytes in flight),
// and one-wavefront workgroups beat 128- and 256-thread ones at every size
// tried: C5 SwiGLU (705 MB) 0.6-3.7%, 8192 x 4096 fp16 3%, the 512 x 5632
// configs 6-7%, the residual add 1-3%.
// head > 0: the pointers were advanced past `head` (< BS) leading elements to a
// 16- or 128-byte boundary (all three share that offset); block 0 also computes those.
template <typename D, int W, int U, bool NT, typename Op, int BS = kBlock>
__global__ __launch_bounds__(BS) void binary_stream(const D* a, const D* b, D* out,
                                                    long long n, int head = 0) {
    using V = Vec<D, W>;
    const long long nvec = n / W;
    const long long base = (long long)blockIdx.x * (BS * U) + threadIdx.x;
    const V* av = reinterpret_cast<const V*>(a);
    const V* bv = reinterpret_cast<const V*>(b);
    V* ov = reinterpret_cast<V*>(out);
    // every thread loads (indices past the end re-read the last vector): a load
    // under a per-thread test makes the compiler wait for it before the next
    V ra[U], rb[U];
    if (nvec > 0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long i = min(base + (long long)u * BS, nvec - 1);
            ra[u] = load<NT>(av + i);
            rb[u] = load<NT>(bv + i);
        }
        __builtin_amdgcn_sched_barrier(0);   // every load issued before any arithmetic
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long i = base + (long long)u * BS;
        if (i < nvec) {
            V y;
#pragma unroll
            for (int e = 0; e < W; ++e)
                y.v[e] = from_f32<D>(Op::template apply<D>(to_f32(ra[u].v[e]), to_f32(rb[u].v[e])));
            store<NT>(ov + i, y);
        }
    }
    if (W > 1 && blockIdx.x == 0) {
        for (long long i = nvec * W + threadIdx.x; i < n; i += BS)
            out[i] = from_f32<D>(Op::template apply<D>(to_f32(a[i]), to_f32(b[i])));
        if ((int)threadIdx.x < head) {
            const long long i = (long long)threadIdx.x - head;
            out[i] = from_f32<D>(Op::template apply<D>(to_f32(a[i]), to_f32(b[i])));
        }
    }
}

constexpr int kStreamU = 1;
constexpr int kStreamBlock = 64;

template <typename D, typename Op>
hipError_t launch_binary(const D* a, const D* b, D* out, long long n, hipStream_t stream) {
    constexpr int W = vec16<D>();
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a);
    // a, b and out at one element-aligned offset mod 16: the leading elements up to
    // the next 128-byte boundary (16-byte when the offsets differ mod 128) go to
    // block 0, the rest streams as aligned vectors.  A stream whose wavefront spans
    // straddle 128-byte lines runs ~20% slower (C5 SwiGLU at a 2-byte offset:
    // 126.5 us against 103.4 aligned).
    const uintptr_t db = pa - reinterpret_cast<uintptr_t>(b), dout = pa - reinterpret_cast<uintptr_t>(out);
    const bool same = (pa & (sizeof(D) - 1)) == 0 && (db & 15) == 0 && (dout & 15) == 0;
    const uintptr_t line = ((db | dout) & 127) == 0 ? 128 : 16;
    const int head = same ? (int)(((line - (pa & (line - 1))) & (line - 1)) / sizeof(D)) : 0;
    if (same && n > head) {
        const long long nb = n - head;
        const long long nvec = nb / W;
        const unsigned grid =
            nvec > 0 ? qlh::blocks_for(nvec, (long long)kStreamBlock * kStreamU) : 1;
        hipLaunchKernelGGL((binary_stream<D, W, kStreamU, true, Op, kStreamBlock>), dim3(grid),
                           dim3(kStreamBlock), 0, stream, a + head, b + head, out + head, nb, head);
    } else {
        const unsigned grid = qlh::blocks_for(n, (long long)kBlock * kUnroll);
        hipLaunchKernelGGL((binary_stream<D, 1, kUnroll, false, Op>), dim3(grid), dim3(kBlock), 0,
                           stream, a, b, out, n);
    }
    return hipGetLastError();
}

// binary16 -> fp32 widening (kernels/fp16_ops.cu:103-110).  W = 4: 8-byte
// loads and 16-byte stores, so a wavefront's store covers one contiguous 1 KiB
// (16-byte loads and 32-byte stores per lane measured 4.6 TB/s against 6.2 on
// MI355X, 64 Mi elements).
// head > 0: src and dst were advanced past `head` (< kBlock) leading elements to
// aligned addresses; block 0 also converts those.
template <int W>
__global__ __launch_bounds__(kBlock) void widen_stream(const _Float16* __restrict__ src,
                                                       float* __restrict__ dst, long long n, int head = 0) {
    using VI = Vec<_Float16, W>;
    using VO = Vec<float, W>;
    const long long nvec = n / W;
    const long long base = (long long)blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
    VI r[kUnroll];   // every thread loads, as binary_stream
    if (nvec > 0) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
            r[u] = load<(W > 1)>(reinterpret_cast<const VI*>(src) + min(base + (long long)u * kBlock, nvec - 1));
        __builtin_amdgcn_sched_barrier(0);   // every load issued before any arithmetic
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long i = base + (long long)u * kBlock;
        if (i < nvec) {
            VO y;
#pragma unroll
            for (int e = 0; e < W; ++e) y.v[e] = (float)r[u].v[e];
            store<(W > 1)>(reinterpret_cast<VO*>(dst) + i, y);
        }
    }
    if (W > 1 && blockIdx.x == 0) {
        for (long long i = nvec * W + threadIdx.x; i < n; i += kBlock) dst[i] = (float)src[i];
        if ((int)threadIdx.x < head) dst[(int)threadIdx.x - head] = (float)src[(int)threadIdx.x - head];
    }
}

// fp32 -> binary16 narrowing, RNE (src/quant_forward.cu:18-21).  W = 4: 16-byte
// loads and 8-byte stores (a wavefront's load covers 1 KiB, its store 512 B);
// measured 6.34 TB/s on MI355X (64 Mi elements) against 6.06 for two 16-byte
// loads and one 16-byte store per lane; one-wavefront workgroups (BS = 64)
// a further 2.8%.
// head: as widen_stream (< BS)
template <int W, int BS = kBlock>
__global__ __launch_bounds__(BS) void narrow_stream(const float* __restrict__ src,
                                                        _Float16* __restrict__ dst, long long n, int head = 0) {
    using VI = Vec<float, W>;
    using VO = Vec<_Float16, W>;
    const long long nvec = n / W;
    const long long base = (long long)blockIdx.x * (BS * kUnroll) + threadIdx.x;
    VI r[kUnroll];   // every thread loads, as binary_stream
    if (nvec > 0) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
            r[u] = load<(W > 1)>(reinterpret_cast<const VI*>(src) + min(base + (long long)u * BS, nvec - 1));
        __builtin_amdgcn_sched_barrier(0);   // every load issued before any arithmetic
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long i = base + (long long)u * BS;
        if (i < nvec) {
            VO y;
#pragma unroll
            for (int e = 0; e < W; ++e) y.v[e] = from_f32<_Float16>(r[u].v[e]);
            store<(W > 1)>(reinterpret_cast<VO*>(dst) + i, y);
        }
    }
    if (W > 1 && blockIdx.x == 0) {
        for (long long i = nvec * W + threadIdx.x; i < n; i += BS) dst[i] = from_f32<_Float16>(src[i]);
        if ((int)threadIdx.x < head)
            dst[(int)threadIdx.x - head] = from_f32<_Float16>(src[(int)threadIdx.x - head]);
    }
}

// Two independent copies in one launch (blockIdx.y selects the pair): the K
// and V halves of a contiguous KV append.  16-byte units with nontemporal
// access (one unit per thread measured fastest for a pure copy; one-wavefront
// workgroups 8% faster than 256-thread ones at C5, 2 x 16 MiB) when all four
// pointers and the byte count allow it, else element-sized units.
template <int UNIT, int U, bool NT, int BS = kBlock>
__global__ __launch_bounds__(BS) void copy_pair(char* __restrict__ d0,
                                                    const char* __restrict__ s0,
                                                    char* __restrict__ d1,
                                                    const char* __restrict__ s1,
                                                    long long nbytes) {
    using V = Vec<char, UNIT>;
    char* dst = blockIdx.y == 0 ? d0 : d1;
    const char* src = blockIdx.y == 0 ? s0 : s1;
    const long long nvec = nbytes / UNIT;
    const long long base = (long long)blockIdx.x * (BS * U) + threadIdx.x;
    V r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long i = base + (long long)u * BS;
        if (i < nvec) r[u] = load<NT>(reinterpret_cast<const V*>(src) + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long i = base + (long long)u * BS;
        if (i < nvec) store<NT>(reinterpret_cast<V*>(dst) + i, r[u]);
    }
}

template <typename D>
hipError_t kv_append_dispatch(D* kc, D* vc, const D* kn, const D* vn, int layer, int pos,
                              int n_tokens, int hkv, int hd, int max_seq, int n_layers,
                              hipStream_t stream) {
    QL_CHECK_ARG(n_tokens >= 0 && hkv > 0 && hd > 0 && max_seq > 0 && n_layers > 0);
    QL_CHECK_ARG(layer >= 0 && layer < n_layers);
    QL_CHECK_ARG(pos >= 0 && (long long)pos + n_tokens <= max_seq);
    if (n_tokens == 0) return hipSuccess;
    QL_CHECK_ARG(kc && vc && kn && vn);
    const long long kv = (long long)hkv * hd;
    const long long off = ((long long)layer * max_seq + pos) * kv;
    const long long nbytes = (long long)n_tokens * kv * (long long)sizeof(D);
    char* d0 = reinterpret_cast<char*>(kc + off);
    char* d1 = reinterpret_cast<char*>(vc + off);
    const char* s0 = reinterpret_cast<const char*>(kn);
    const char* s1 = reinterpret_cast<const char*>(vn);
    const bool vec_ok = qlh::aligned16(d0) && qlh::aligned16(d1) && qlh::aligned16(s0) &&
                        qlh::aligned16(s1) && nbytes % 16 == 0;
    if (vec_ok) {
        hipLaunchKernelGGL((copy_pair<16, 1, true, kWave>), dim3(qlh::blocks_for(nbytes / 16, kWave), 2),
                           dim3(kWave), 0, stream, d0, s0, d1, s1, nbytes);
    } else {
        constexpr int U = (int)sizeof(D);
        hipLaunchKernelGGL((copy_pair<U, kUnroll, false>),
                           dim3(qlh::blocks_for(nbytes / U, kBlock * kUnroll), 2), dim3(kBlock), 0,
                           stream, d0, s0, d1, s1, nbytes);
    }
    return hipGetLastError();
}

}  // namespace

extern "C" hipError_t ql_swiglu_f32(const float* gate, const float* up, float* out, int rows,
                                    int ffn_dim, hipStream_t stream) {
    QL_CHECK_ARG(rows >= 0 && ffn_dim >= 0);
    const long long n = (long long)rows * ffn_dim;
    if (n == 0) return hipSuccess;
    QL_CHECK_ARG(gate && up && out);
    return launch_binary<float, SwigluOp>(gate, up, out, n, stream);
}

extern "C" hipError_t ql_swiglu_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out,
                                    int rows, int ffn_dim, hipStream_t stream) {
    QL_CHECK_ARG(rows >= 0 && ffn_dim >= 0);
    const long long n = (long long)rows * ffn_dim;
    if (n == 0) return hipSuccess;
    QL_CHECK_ARG(gate && up && out);
    return launch_binary<_Float16, SwigluOp>(reinterpret_cast<const _Float16*>(gate),
                                             reinterpret_cast<const _Float16*>(up),
                                             reinterpret_cast<_Float16*>(out), n, stream);
}

extern "C" hipError_t ql_add_f32(float* x, const float* d, int64_t n, hipStream_t stream) {
    QL_CHECK_ARG(n >= 0);
    if (n == 0) return hipSuccess;
    QL_CHECK_ARG(x && d);
    return launch_binary<float, AddOp>(x, d, x, n, stream);
}

extern "C" hipError_t ql_add_f16(uint16_t* x, const uint16_t* d, int64_t n, hipStream_t stream) {
    QL_CHECK_ARG(n >= 0);
    if (n == 0) return hipSuccess;
    QL_CHECK_ARG(x && d);
    _Float16* xh = reinterpret_cast<_Float16*>(x);
    return launch_binary<_Float16, AddOp>(xh, reinterpret_cast<const _Float16*>(d), xh, n,
                                          stream);
}

extern "C" hipError_t ql_f16_to_f32(const uint16_t* src, float* dst, int64_t n,
                                    hipStream_t stream) {
    QL_CHECK_ARG(n >= 0);
    if (n == 0) return hipSuccess;
    QL_CHECK_ARG(src && dst);
    const _Float16* s = reinterpret_cast<const _Float16*>(src);
    // src and dst at one element offset mod 32 elements (element-aligned): the leading
    // elements up to dst's next 128-byte boundary (src's 64-byte one) go to block 0
    const uintptr_t ps = (uintptr_t)src, pd = (uintptr_t)dst;
    const int head = (ps & 1) == 0 && (pd & 3) == 0 && (((ps >> 1) - (pd >> 2)) & 31) == 0
                         ? (int)(((128 - (pd & 127)) & 127) / 4) : -1;
    if (head >= 0 && n > head) {
        const long long nb = n - head, nvec = nb / 4;
        const unsigned grid = nvec > 0 ? qlh::blocks_for(nvec, (long long)kBlock * kUnroll) : 1;
        hipLaunchKernelGGL((widen_stream<4>), dim3(grid), dim3(kBlock), 0, stream, s + head, dst + head, nb, head);
    } else if ((ps & 7u) == 0 && qlh::aligned16(dst)) {
        const long long nvec = n / 4;
        const unsigned grid = nvec > 0 ? qlh::blocks_for(nvec, (long long)kBlock * kUnroll) : 1;
        hipLaunchKernelGGL((widen_stream<4>), dim3(grid), dim3(kBlock), 0, stream, s, dst,
                           (long long)n, 0);
    } else {
        hipLaunchKernelGGL((widen_stream<1>), dim3(qlh::blocks_for(n, (long long)kBlock * kUnroll)),
                           dim3(kBlock), 0, stream, s, dst, (long long)n);
    }
    return hipGetLastError();
}

extern "C" hipError_t ql_f32_to_f16(const float* src, uint16_t* dst, int64_t n,
                                    hipStream_t stream) {
    QL_CHECK_ARG(n >= 0);
    if (n == 0) return hipSuccess;
    QL_CHECK_ARG(src && dst);
    _Float16* d = reinterpret_cast<_Float16*>(dst);
    // as ql_f16_to_f32, src (fp32) advanced to its next 128-byte boundary
    const uintptr_t ps = (uintptr_t)src, pd = (uintptr_t)dst;
    const int head = (ps & 3) == 0 && (pd & 1) == 0 && (((ps >> 2) - (pd >> 1)) & 31) == 0
                         ? (int)(((128 - (ps & 127)) & 127) / 4) : -1;
    if (head >= 0 && n > head) {
        const long long nb = n - head, nvec = nb / 4;
        const unsigned grid = nvec > 0 ? qlh::blocks_for(nvec, (long long)kWave * kUnroll) : 1;
        hipLaunchKernelGGL((narrow_stream<4, kWave>), dim3(grid), dim3(kWave), 0, stream, src + head, d + head, nb,
                           head);
    } else if (qlh::aligned16(src) && (pd & 7u) == 0) {
        const long long nvec = n / 4;
        const unsigned grid = nvec > 0 ? qlh::blocks_for(nvec, (long long)kWave * kUnroll) : 1;
        hipLaunchKernelGGL((narrow_stream<4, kWave>), dim3(grid), dim3(kWave), 0, stream, src, d,
                           (long long)n, 0);
    } else {
        hipLaunchKernelGGL((narrow_stream<1>), dim3(qlh::blocks_for(n, (long long)kBlock * kUnroll)),
                           dim3(kBlock), 0, stream, src, d, (long long)n);
    }
    return hipGetLastError();
}

extern "C" hipError_t ql_kv_append_f32(float* k_cache, float* v_cache, const float* k_new,
                                       const float* v_new, int layer, int pos, int n_tokens,
                                       int n_kv_heads, int head_dim, int max_seq, int n_layers,
                                       hipStream_t stream) {
    return kv_append_dispatch<float>(k_cache, v_cache, k_new, v_new, layer, pos, n_tokens,
                                     n_kv_heads, head_dim, max_seq, n_layers, stream);
}

extern "C" hipError_t ql_kv_append_f16(uint16_t* k_cache, uint16_t* v_cache,
                                       const uint16_t* k_new, const uint16_t* v_new, int layer,
                                       int pos, int n_tokens, int n_kv_heads, int head_dim,
                                       int max_seq, int n_layers, hipStream_t stream) {
    return kv_append_dispatch<uint16_t>(k_cache, v_cache, k_new, v_new, layer, pos, n_tokens,
                                        n_kv_heads, head_dim, max_seq, n_layers, stream);
}
