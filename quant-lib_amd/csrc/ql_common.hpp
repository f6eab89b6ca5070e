// ql_common.hpp -- shared device helpers for the gfx950 kernels.
//
// Element types: kernels are written against the device element type D, either
// `float` or `_Float16` (IEEE binary16; the C ABI passes it as uint16_t bits).
// All arithmetic is fp32; binary16 values are widened exactly and narrowed with
// round-to-nearest-even (v_cvt_f16_f32 in the default rounding mode).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace ql {

constexpr int kWave = 64;      // CDNA wavefront width
constexpr int kBlock = 256;    // default workgroup: 4 wavefronts

// W contiguous elements moved as one access (16 bytes for the vector paths).
template <typename D, int W>
struct alignas(sizeof(D) * W) Vec {
    D v[W];
};

// 16-byte vector width in elements of D.
template <typename D>
constexpr int vec16() { return 16 / (int)sizeof(D); }

// Raw carriers for nontemporal (streaming) accesses of 2..32-byte values.
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int BYTES>
struct RawOf;
template <> struct RawOf<32> { using type = u32x8; };
template <> struct RawOf<16> { using type = u32x4; };
template <> struct RawOf<8> { using type = u32x2; };
template <> struct RawOf<4> { using type = uint32_t; };
template <> struct RawOf<2> { using type = uint16_t; };

// Load/store with the nontemporal hint when NT: data touched once is streamed
// past the caches instead of displacing lines other wavefronts still need.
template <bool NT, typename V>
__device__ __forceinline__ V load(const V* p) {
    if constexpr (NT) {
        using R = typename RawOf<sizeof(V)>::type;
        return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const R*>(p)));
    } else {
        return *p;
    }
}

template <bool NT, typename V>
__device__ __forceinline__ void store(V* p, const V& v) {
    if constexpr (NT) {
        using R = typename RawOf<sizeof(V)>::type;
        __builtin_nontemporal_store(__builtin_bit_cast(R, v), reinterpret_cast<R*>(p));
    } else {
        *p = v;
    }
}

// 16-byte store with the cache policy "sc1 nt" (device scope, nontemporal):
// the line is written through to memory rather than left dirty in L2.  Issued
// as a buffer store, whose instruction carries the policy bits: `base` must be
// the same for every lane of the wavefront (pass it through uniform() when the
// compiler cannot see that), `byte_off` is the lane's offset from it (below
// 4 GiB).  Measured on MI355X with buffers rotated past the MALL, against
// nontemporal stores: a plain 1-read/1-write stream 6.44 -> 6.55 TB/s, RoPE
// (which writes back the rows it just read) 2-11% faster; but the row kernels
// that write fresh buffers were no faster or slower (add+RMSNorm equal,
// SwiGLU -0.7%, fp16 softmax -5%, a 2048-row RMSNorm -35%), so only RoPE
// uses it.
constexpr int kStorePolicy = 16 | 2;   // sc1 | nt
template <typename V>
__device__ __forceinline__ void store_wt(const void* base, uint32_t byte_off, const V& v) {
    static_assert(sizeof(V) == 16, "16-byte stores");
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)byte_off, 0,
                                           kStorePolicy);
}

// Read of a table that no kernel of the launch writes (ids, slot maps, block
// pointers, positions) through the constant address space: at a
// wavefront-uniform index it is a scalar load, on the counter the vector row
// loads do not use, so waiting for it does not wait for them.
template <typename T>
__device__ __forceinline__ T ld_scalar(const T* p) {
    return *reinterpret_cast<const __attribute__((address_space(4))) T*>(reinterpret_cast<uintptr_t>(p));
}

// A zero held in a vector register that the compiler cannot see through.  A
// load whose address is uniform over the wavefront becomes a scalar load (or has
// its result moved to scalar registers right after it is issued); scalar loads
// share their wait counter with LDS accesses, so every wait for an LDS read would
// also wait for them.  Offset by this zero, the load stays a vector load on the
// vector memory counter.
__device__ __forceinline__ int divergent_zero() {
    int z;
    asm("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// A pointer that is the same in every lane of the wavefront, made scalar.
template <typename T>
__device__ __forceinline__ T* uniform(T* p) {
    const uint64_t a = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }

template <typename D>
__device__ __forceinline__ D from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
// The empty asm makes x an opaque, already-rounded fp32 value: without it the
// compiler may fold the fp32 operation that produced x and this narrowing into
// one mixed-precision FMA (v_fma_mix*), which rounds once instead of twice and
// so differs from "fp32 result, then RNE to binary16" in rare last-bit cases.
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float x) {
    asm("" : "+v"(x));
    return (_Float16)x;
}

// Round x to the precision of D and back (identity for float).
template <typename D>
__device__ __forceinline__ float round_to(float x) { return to_f32(from_f32<D>(x)); }

// Butterfly reductions over the 64 lanes of a wavefront.  Lane i combines
// with lane i^o at every step, so all lanes finish with bit-identical values
// (a+b == b+a and max is order-free).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// exp(y) in fp32 from the hardware base-2 exponential (v_exp_f32).
// y*log2(e) is formed as t + err with log2(e) split into hi/lo parts and an
// FMA residual (the classic compensated product), then
// exp(y) = 2^t * 2^err ~= 2^t * (1 + err*ln2); the correction keeps the
// argument error below one fp32 ulp for |y| <= 110.  Outside [-110, 110] the
// result is 0 or +inf in fp32 anyway, so y is clamped there (comparisons keep NaN).
__device__ __forceinline__ float exp_f32(float y) {
    const float kL2eHi = 1.44269502162933349609375f;  // fp32(log2 e)
    const float kL2eLo = 1.925963033500011e-08f;      // log2 e - kL2eHi
    const float kLn2 = 0.693147180559945309f;
    y = (y < -110.0f) ? -110.0f : y;
    y = (y > 110.0f) ? 110.0f : y;
    const float t = y * kL2eHi;
    const float err = fmaf(y, kL2eHi, -t) + y * kL2eLo;
    const float r = __builtin_amdgcn_exp2f(t);
    return r * (1.0f + err * kLn2);
}

// exp(y) without the residual correction: relative error ~|y|*2^-24 plus the
// v_exp_f32 error; used where the output is binary16 (2^-11 rounding).
__device__ __forceinline__ float exp_f32_fast(float y) {
    const float kL2e = 1.44269502162933349609375f;
    y = (y < -110.0f) ? -110.0f : y;
    y = (y > 110.0f) ? 110.0f : y;
    return __builtin_amdgcn_exp2f(y * kL2e);
}

// Elements S .. S + W - 1 of the concatenation a:b.
template <int S, typename V>
__device__ __forceinline__ V take(const V& a, const V& b) {
    constexpr int W = sizeof(V) / sizeof(a.v[0]);
    V r;
#pragma unroll
    for (int e = 0; e < W; ++e) r.v[e] = e + S < W ? a.v[e + S] : b.v[e + S - W];
    return r;
}

// take<s>(a, b) for a wavefront-uniform s in [0, W)
template <typename V>
__device__ __forceinline__ V take_at(int s, const V& a, const V& b) {
    constexpr int W = sizeof(V) / sizeof(a.v[0]);
    switch (s) {
    case 0: return a;
    case 1: return take<1>(a, b);
    case 2: return take<2>(a, b);
    case 3: return take<3>(a, b);
    default:
        if constexpr (W > 4) {
            switch (s) {
            case 4: return take<4>(a, b);
            case 5: return take<5>(a, b);
            case 6: return take<6>(a, b);
            default: return take<7>(a, b);
            }
        }
        return a;
    }
}

}  // namespace ql

// ---- host-side helpers --------------------------------------------------------
namespace qlh {

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline unsigned blocks_for(long long work, long long per_block) {
    return (unsigned)((work + per_block - 1) / per_block);
}

}  // namespace qlh

#define QL_CHECK_ARG(cond)                         \
    do {                                           \
        if (!(cond)) return hipErrorInvalidValue;  \
    } while (0)
