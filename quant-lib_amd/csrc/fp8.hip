// fp8.hip -- FP8 weight codec and the skinny FP8-weight GEMM (quantlib, gfx950).
//
// Codec (quantlib_src/kernels/fp8_convert.cu:15-173, quant_types.h:47-84):
//   scales  per group (per-tensor: the whole matrix; per-channel: a row; per-group:
//           runs of group_size elements of the row-major matrix):
//           scale = fmax / max|x| (max < 1e-8 -> 1), fmax = 448 (E4M3) / 57344 (E5M2)
//   quantize q = encode(x * scale)
//   dequant  x' = binary16(decode(q) / scale)
// QL_FP8_MODE_REFERENCE reproduces the reference's algorithm in IEEE arithmetic:
// its max reduction only sees the elements whose offset inside the group is < 32
// mod 128 (128 threads stride the group, only the first warp is reduced), and its
// encoder clamps, rebiases and TRUNCATES the mantissa with no subnormals.
// QL_FP8_MODE_OCP uses the whole group's max and the OCP E4M3FN / E5M2 encodings,
// converted by gfx950's v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 (round to nearest
// even, subnormals) after saturating to +-fmax; decode by v_cvt_f32_fp8/bf8.
//
// Codec kernels: groups of 8..512 elements (powers of two) and other multiples of 8
// below 256 quantize in one pass with several groups per wavefront; longer groups up
// to 16384 in one pass with one wavefront (or a workgroup of 2-4) per group held in
// registers; larger groups (per tensor) reduce workgroup maxima, then encode; lengths
// that are not a multiple of 8 take a scales pass and 8 elements per thread, each
// with its own group's scale.
//
// GEMM (quantlib_src/kernels/fp8_gemm.cu:34-139): C[M,N] = A[M,K] W'[N,K]^T with
// W' the dequantized weights in binary16 and fp32 accumulation.  For few rows the
// weights are streamed once and dequantized in registers: 1-2 rows as a stream of
// whole weight rows (v_dot2_f32_f16, no matrix cores), up to 8 rows by whole-row
// loads into v_mfma_f32_16x16x32_f16, up to 32 rows by the register kernel (each
// lane 16 codes of a row per chunk), 33-64 rows by whole 128-byte lines re-laid
// through LDS (C^T = W' A^T, K split over wavefronts and summed in LDS); the
// in-register dequant multiplies by 1/scale or scales the fp32 sums.  Larger M
// dequantizes into a workspace with the codec and runs the fp16 library GEMM.
#include "ql_common.hpp"
#include <type_traits>
#include "quantlib_amd.h"

#include <math.h>
#include <float.h>
#include <stdint.h>

#include <algorithm>

namespace {

using namespace ql;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));

__host__ __device__ constexpr float fp8_max(int fmt) { return fmt == QL_FP8_E4M3 ? 448.0f : 57344.0f; }

// ---- element codec -------------------------------------------------------------------
template <int FMT>
__device__ __forceinline__ uint32_t enc_ref(float v) {
    constexpr float fm = fp8_max(FMT);
    constexpr int MB = FMT == QL_FP8_E4M3 ? 3 : 2, BIAS = FMT == QL_FP8_E4M3 ? 7 : 15;
    constexpr int EMAX = FMT == QL_FP8_E4M3 ? 15 : 31;
    v = v > fm ? fm : (v < -fm ? -fm : v);
    const uint32_t bits = __float_as_uint(v);
    const uint32_t sign = (bits >> 31) & 1u;
    int e = (int)((bits >> 23) & 0xFFu) - 127 + BIAS;
    uint32_t m = (bits >> (23 - MB)) & ((1u << MB) - 1u);
    if (e <= 0) return sign << 7;
    if (e > EMAX) {
        e = EMAX;
        m = (1u << MB) - 1u;
    }
    return (sign << 7) | ((uint32_t)e << MB) | m;
}

template <int FMT>
__device__ __forceinline__ float dec_ref(uint32_t q) {
    constexpr int MB = FMT == QL_FP8_E4M3 ? 3 : 2, BIAS = FMT == QL_FP8_E4M3 ? 7 : 15;
    const uint32_t e = (q >> MB) & (FMT == QL_FP8_E4M3 ? 0xFu : 0x1Fu);
    const uint32_t m = q & ((1u << MB) - 1u);
    const uint32_t bits = ((q & 0x80u) << 24) | ((e + 127u - BIAS) << 23) | (m << (23 - MB));
    return (e == 0 && m == 0) ? 0.0f : __uint_as_float(bits);
}

// two values -> two OCP codes in the low 16 bits (NaN -> the canonical NaN code)
template <int FMT>
__device__ __forceinline__ uint32_t enc_ocp2(float a, float b) {
    constexpr float fm = fp8_max(FMT);
    constexpr uint32_t kNaN = FMT == QL_FP8_E4M3 ? 0x7Fu : 0x7Eu;
    const float ca = a > fm ? fm : (a < -fm ? -fm : a);
    const float cb = b > fm ? fm : (b < -fm ? -fm : b);
    uint32_t w;
    if constexpr (FMT == QL_FP8_E4M3)
        w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false);
    else
        w = (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(ca, cb, 0, false);
    const uint32_t lo = isnan(a) ? kNaN : (w & 0xFFu);
    const uint32_t hi = isnan(b) ? kNaN : ((w >> 8) & 0xFFu);
    return lo | (hi << 8);
}

// the two bytes of w's low (HI = false) or high 16-bit word
template <int FMT, bool HI = false>
__device__ __forceinline__ float2v dec_ocp2(uint32_t w) {
    if constexpr (FMT == QL_FP8_E4M3)
        return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, HI);
    else
        return __builtin_amdgcn_cvt_pk_f32_bf8((int)w, HI);
}

// two codes (the low or high half of w) -> two binary16, exact (every E4M3 / E5M2
// value is a binary16 value; the scale operand 1.0 leaves them as decoded)
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
template <int FMT, bool HI = false>
__device__ __forceinline__ half2v dec_ocp2_h(uint32_t w) {
    if constexpr (FMT == QL_FP8_E4M3)
        return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI);
    else
        return __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, 1.0f, HI);
}

// ---- scales ----------------------------------------------------------------------------
struct Geom {
    long long n;    // elements
    long long gs;   // group length
    int n_groups;
};

__device__ __forceinline__ bool seen(int mode, long long i_in_group) {
    return mode == QL_FP8_MODE_OCP || (i_in_group & 127) < 32;
}

// one wavefront per group (group_size <= 8192): group max of |x|
__global__ __launch_bounds__(kBlock) void absmax_wave(const _Float16* __restrict__ x, Geom g,
                                                      int mode, float* __restrict__ mx) {
    const int lane = threadIdx.x & (kWave - 1);
    const long long grp = (long long)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (grp >= g.n_groups) return;
    const long long base = grp * g.gs;
    const long long len = min(g.gs, g.n - base);
    float m = 0.0f;
    for (long long i = lane; i < len; i += kWave)
        if (seen(mode, i)) m = fmaxf(m, fabsf((float)x[base + i]));
    m = wave_max(m);
    if (lane == 0) mx[grp] = m;
}

// groups of GL*8 elements (GL = 1..64 lanes, a power of two), n % 8 == 0, 16-byte
// aligned: each lane reads 8 consecutive elements with one 16-byte load, the GL
// lanes of a group (a group starts at a lane multiple of GL, since every
// wavefront starts at a multiple of 64 vectors) reduce with shuffles, and each
// wavefront walks kAbsIters consecutive spans of 64 vectors.  In reference mode a
// lane whose 8 elements sit at offsets >= 32 mod 128 of their group loads nothing.
constexpr int kAbsIters = 8;

template <int GL>
__global__ __launch_bounds__(kBlock) void absmax_vec(const _Float16* __restrict__ x, Geom g, int mode,
                                                     float* __restrict__ mx) {
    const int lane = threadIdx.x & (kWave - 1);
    const long long n_vec = g.n / 8;
    const long long w0 = ((long long)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave) * kAbsIters * kWave;
#pragma unroll
    for (int it = 0; it < kAbsIters; ++it) {
        const long long v = w0 + (long long)it * kWave + lane;
        const long long off = (v * 8) % (8 * GL);                 // offset inside the group
        float m = 0.0f;
        if (v < n_vec && seen(mode, off)) {
            const Vec<_Float16, 8> h = load<true>(reinterpret_cast<const Vec<_Float16, 8>*>(x) + v);
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf((float)h.v[e]));
        }
#pragma unroll
        for (int o = 1; o < GL; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
        if ((lane & (GL - 1)) == 0 && v < n_vec) mx[v / GL] = m;
    }
}

// Groups of the block-strided kernels along grid y (at most 65535) and z.
constexpr unsigned kGroupsY = 65535;
inline dim3 group_grid(unsigned bx, int n_groups) {
    const unsigned gy = (unsigned)std::min<long long>(n_groups, kGroupsY);
    return dim3(bx, gy, (unsigned)(((long long)n_groups + kGroupsY - 1) / kGroupsY));
}

// large groups: blocks stride their group and combine with an atomic max on the
// bit pattern (non-negative floats order like their bits); mx pre-zeroed
__global__ __launch_bounds__(kBlock) void absmax_blocks(const _Float16* __restrict__ x, Geom g,
                                                        int mode, float* __restrict__ mx) {
    const long long grp = (long long)blockIdx.z * kGroupsY + blockIdx.y;   // grid y x z covers the groups
    if (grp >= g.n_groups) return;   // workgroup-uniform, before any barrier
    const long long base = grp * g.gs;
    const long long len = min(g.gs, g.n - base);
    float m = 0.0f;
    for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < len;
         i += (long long)gridDim.x * kBlock)
        if (seen(mode, i)) m = fmaxf(m, fabsf((float)x[base + i]));
    m = wave_max(m);
    __shared__ float part[kBlock / kWave];
    if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kBlock / kWave; ++w) m = fmaxf(m, part[w]);
        atomicMax(reinterpret_cast<unsigned int*>(mx) + grp, __float_as_uint(m));
    }
}

// absmax_blocks with 16-byte loads (n % 8 == 0, gs % 8 == 0, 16-byte aligned x): the
// workgroups of a group stride over batches of kBlock * kBlockIters of the vectors the
// mode sees, each thread issuing its kBlockIters loads of a batch before any max.  The
// reference mode sees elements at offsets below 32 mod 128, i.e. vectors 16j..16j+3:
// seen vector t is vector (t / 4) * 16 + t % 4, so only those are read.  The atomics
// of one group's workgroups hit one address and serialize (one per workgroup): at most
// kAbsBlocks workgroups in all (OCP quantize of one 14336 x 4096 tensor: 84 us with
// one workgroup per batch, 3584 of them; 57 us with 512; 59 us with 256).
constexpr int kBlockIters = 8;
constexpr long long kAbsBlocks = 512;

__host__ __device__ inline long long seen_vectors(int mode, long long nv) {
    return mode == QL_FP8_MODE_OCP ? nv : (nv / 16) * 4 + (nv % 16 < 4 ? nv % 16 : 4);
}

// PARTIAL: workgroup b of group g writes its max to mx[g * gridDim.x + b] instead
// (no atomics, nothing to clear first); reduce_partials then finishes the scales.
template <bool PARTIAL = false>
__global__ __launch_bounds__(kBlock) void absmax_blocks_vec(const _Float16* __restrict__ x, Geom g,
                                                            int mode, float* __restrict__ mx) {
    const long long grp = (long long)blockIdx.z * kGroupsY + blockIdx.y;   // grid y x z covers the groups
    if (grp >= g.n_groups) return;   // workgroup-uniform, before any barrier
    const long long base = grp * g.gs;
    const long long nt = seen_vectors(mode, min(g.gs, g.n - base) / 8);
    const Vec<_Float16, 8>* xv = reinterpret_cast<const Vec<_Float16, 8>*>(x + base);
    float m = 0.0f;
    for (long long b0 = (long long)blockIdx.x * kBlock * kBlockIters; b0 < nt;
         b0 += (long long)gridDim.x * kBlock * kBlockIters) {   // workgroup-uniform
        const long long t0 = b0 + threadIdx.x;
        Vec<_Float16, 8> h[kBlockIters];
#pragma unroll
        for (int it = 0; it < kBlockIters; ++it) {
            const long long t = min(t0 + (long long)it * kBlock, nt - 1);
            h[it] = load<true>(xv + (mode == QL_FP8_MODE_OCP ? t : (t >> 2) * 16 + (t & 3)));
        }
#pragma unroll
        for (int it = 0; it < kBlockIters; ++it)
            if (t0 + (long long)it * kBlock < nt) {
#pragma unroll
                for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf((float)h[it].v[e]));
            }
    }
    m = wave_max(m);
    __shared__ float part[kBlock / kWave];
    if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kBlock / kWave; ++w) m = fmaxf(m, part[w]);
        if constexpr (PARTIAL) mx[grp * gridDim.x + blockIdx.x] = m;
        else atomicMax(reinterpret_cast<unsigned int*>(mx) + grp, __float_as_uint(m));
    }
}

// one workgroup per group: the max of its nb partial maxima -> the group's scale
__global__ __launch_bounds__(kBlock) void reduce_partials(const float* __restrict__ part, int nb, float fmax,
                                                          float* __restrict__ scales) {
    const int grp = blockIdx.x;
    float m = 0.0f;
    for (int b = threadIdx.x; b < nb; b += kBlock) m = fmaxf(m, part[(size_t)grp * nb + b]);
    m = wave_max(m);
    __shared__ float red[kBlock / kWave];
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kBlock / kWave; ++w) m = fmaxf(m, red[w]);
        scales[grp] = m < 1e-8f ? 1.0f : fmax / m;
    }
}

// groups of at most 64 elements that are not a multiple of 8 (so groups start inside
// 16-byte vectors): one thread per group reads its elements, and writes the final
// scale (fmax / max, 1 below 1e-8) itself
__global__ __launch_bounds__(kBlock) void absmax_thread(const _Float16* __restrict__ x, Geom g, int mode,
                                                        float fmax, float* __restrict__ scales) {
    const long long grp = (long long)blockIdx.x * kBlock + threadIdx.x;
    if (grp >= g.n_groups) return;
    const long long base = grp * g.gs;
    const int len = (int)min(g.gs, g.n - base);
    float m = 0.0f;
    for (int i = 0; i < len; ++i)
        if (seen(mode, i)) m = fmaxf(m, fabsf((float)x[base + i]));
    scales[grp] = m < 1e-8f ? 1.0f : fmax / m;
}

__global__ void fill_zero(float* __restrict__ p, int n) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

__global__ void finalize_scales(float* __restrict__ s, int n, float fmax) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i < n) {
        const float m = s[i];
        s[i] = m < 1e-8f ? 1.0f : fmax / m;
    }
}

// ---- quantize / dequantize ------------------------------------------------------------
// 8 elements times their group's scale -> 8 codes (s: one float, or one per element)
template <int FMT, int MODE, typename S = float>
__device__ __forceinline__ u32x2 encode8(const Vec<_Float16, 8>& v, const S& s) {
    uint32_t w[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (std::is_same_v<S, float>) f[e] = (float)v.v[4 * h + e] * s;
            else f[e] = (float)v.v[4 * h + e] * s[4 * h + e];
        }
        if constexpr (MODE == QL_FP8_MODE_REFERENCE) {
            w[h] = enc_ref<FMT>(f[0]) | (enc_ref<FMT>(f[1]) << 8) | (enc_ref<FMT>(f[2]) << 16) |
                   (enc_ref<FMT>(f[3]) << 24);
        } else {
            w[h] = enc_ocp2<FMT>(f[0], f[1]) | (enc_ocp2<FMT>(f[2], f[3]) << 16);
        }
    }
    return u32x2{w[0], w[1]};
}

// The scales of the 8 elements from e0 (a multiple of 8): groups that are not a
// multiple of 8 long start inside vectors.  From g0 = e0 / gs and r0 = e0 - g0 * gs,
// element e is in group g0 + (r0 + e) / gs: g0 or g0 + 1 when gs >= 8 (two scale
// loads, the second clamped to the last group), up to 8 groups below 8.
__device__ __forceinline__ void scales8(const float* __restrict__ scales, const Geom& g, long long e0,
                                        float (&s)[8]) {
    const long long g0 = g.n_groups == 1 ? 0 : e0 / g.gs;   // per tensor: no 64-bit division
    const long long r0 = e0 - g0 * g.gs;                     // < gs
    if (g.gs >= 8) {
        const float s0 = scales[g0];
        const float s1 = scales[min(g0 + 1, (long long)g.n_groups - 1)];
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] = r0 + e < g.gs ? s0 : s1;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] = scales[g0 + (r0 + e) / g.gs];
    }
}

// VEC: 8 elements per thread (n % 8 == 0, 16-byte aligned x, 8-byte aligned q; groups
// of a multiple of 8 take one scale per thread, others scales8); else one element.
template <int FMT, int MODE, bool VEC>
__global__ __launch_bounds__(kBlock) void quantize_kernel(const _Float16* __restrict__ x, Geom g,
                                                          const float* __restrict__ scales,
                                                          uint8_t* __restrict__ q) {
    const long long t = (long long)blockIdx.x * kBlock + threadIdx.x;
    if constexpr (VEC) {
        if (t * 8 >= g.n) return;
        const Vec<_Float16, 8> v = load<true>(reinterpret_cast<const Vec<_Float16, 8>*>(x) + t);
        if (g.gs % 8 == 0) {   // uniform
            const long long gi = g.n_groups == 1 ? 0 : (t * 8) / g.gs;   // per tensor: no 64-bit division
            store<true>(reinterpret_cast<u32x2*>(q) + t, encode8<FMT, MODE>(v, scales[gi]));
        } else {
            float s8[8];
            scales8(scales, g, t * 8, s8);
            store<true>(reinterpret_cast<u32x2*>(q) + t, encode8<FMT, MODE>(v, s8));
        }
    } else {
        if (t >= g.n) return;
        const float f = (float)x[t] * scales[t / g.gs];
        q[t] = (uint8_t)(MODE == QL_FP8_MODE_REFERENCE ? enc_ref<FMT>(f) : (enc_ocp2<FMT>(f, 0.0f) & 0xFFu));
    }
}

// Scales and codes in one pass for groups of GL*8 elements (GL = 1..64 lanes, a
// power of two; n % 8 == 0, 16-byte aligned x, 8-byte aligned q): the layout of
// absmax_vec -- each lane loads its 8 elements with one 16-byte load, the GL
// lanes of a group reduce the group's max -- and then every lane computes the
// group's scale exactly as finalize_scales does (fmax / max, 1 below 1e-8) and
// encodes its 8 elements from the registers it loaded, so x is read once instead
// of twice.  One lane per group stores the scale.
constexpr int kQuantIters = 4;   // spans of 64 vectors per wavefront (2, 4, 8, 16 measured: 4 best)

template <int FMT, int MODE, int GL>
__global__ __launch_bounds__(kBlock) void quantize_groups(const _Float16* __restrict__ x, Geom g,
                                                          float* __restrict__ scales, uint8_t* __restrict__ q) {
    constexpr float kMax = fp8_max(FMT);
    const int lane = threadIdx.x & (kWave - 1);
    const long long n_vec = g.n / 8;
    const long long w0 = ((long long)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave) * kQuantIters * kWave;
    Vec<_Float16, 8> h[kQuantIters];
#pragma unroll
    for (int it = 0; it < kQuantIters; ++it) {   // every load first
        const long long v = w0 + (long long)it * kWave + lane;
        h[it] = load<true>(reinterpret_cast<const Vec<_Float16, 8>*>(x) + (v < n_vec ? v : 0));
    }
#pragma unroll
    for (int it = 0; it < kQuantIters; ++it) {
        const long long v = w0 + (long long)it * kWave + lane;
        const long long off = (v * 8) % (8 * GL);                 // offset inside the group
        float m = 0.0f;   // lanes past the end (their load repeated vector 0) add nothing
        if (v < n_vec && seen(MODE, off)) {
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf((float)h[it].v[e]));
        }
#pragma unroll
        for (int o = 1; o < GL; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
        const float sc = m < 1e-8f ? 1.0f : kMax / m;
        if (v < n_vec) {
            if ((lane & (GL - 1)) == 0) scales[v / GL] = sc;
            store<true>(reinterpret_cast<u32x2*>(q) + v, encode8<FMT, MODE>(h[it], sc));
        }
    }
}

// Scales and codes in one pass for short groups of V 16-byte vectors, V = 3..31 not a
// power of two (n % 8 == 0, 16-byte aligned x, 8-byte aligned q): a wavefront span is
// P = 64 / V whole groups in lanes [0, P*V) -- lane l holds vector l % V of group
// l / V -- so each load instruction reads P*V consecutive vectors.  A group's max is
// a segmented reduction (each step a lane takes the max of the lane o places up when
// that lane is in its group, o = 1, 2, 4, ...), which leaves it in the group's first
// lane, read back by the others.  kQuantIters spans per wavefront.  ENCODE false:
// scales only.
template <int FMT, int MODE, bool ENCODE>
__global__ __launch_bounds__(kBlock) void quantize_segments(const _Float16* __restrict__ x, Geom g, int V, int P,
                                                            float* __restrict__ scales, uint8_t* __restrict__ q) {
    constexpr float kMax = fp8_max(FMT);
    const int lane = threadIdx.x & (kWave - 1);
    const int seg = lane / V, first = seg * V, idx = lane - first;
    const bool in_span = seg < P;
    const long long n_vec = g.n / 8;
    const long long sp0 = ((long long)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave) * kQuantIters;
    Vec<_Float16, 8> h[kQuantIters];
#pragma unroll
    for (int it = 0; it < kQuantIters; ++it) {   // every load first
        const long long v = (sp0 + it) * P * V + lane;
        h[it] = load<true>(reinterpret_cast<const Vec<_Float16, 8>*>(x) + (in_span && v < n_vec ? v : 0));
    }
#pragma unroll
    for (int it = 0; it < kQuantIters; ++it) {
        const long long v = (sp0 + it) * P * V + lane;
        const bool ok = in_span && v < n_vec;
        float m = 0.0f;
        if (ok && seen(MODE, (long long)idx * 8)) {
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf((float)h[it].v[e]));
        }
        for (int o = 1; o < V; o <<= 1) {   // uniform trip count
            const float t = __shfl(m, min(lane + o, kWave - 1), kWave);
            if (idx + o < V) m = fmaxf(m, t);
        }
        m = __shfl(m, first, kWave);
        const float sc = m < 1e-8f ? 1.0f : kMax / m;
        if (ok) {
            if (idx == 0) scales[(sp0 + it) * P + seg] = sc;
            if constexpr (ENCODE) store<true>(reinterpret_cast<u32x2*>(q) + v, encode8<FMT, MODE>(h[it], sc));
        }
    }
}

// Scales and codes in one pass for any group length that is a multiple of 8, up to
// 16384 (per-channel rows, large or odd groups; n % 8 == 0, 16-byte aligned x, 8-byte
// aligned q): one wavefront per group holds the group in registers (NV 16-byte
// vectors per lane: 8, 16 or 32, the fewest that hold it), reduces its max, computes
// the scale as finalize_scales does and encodes from the registers: x is read once,
// with 16-byte loads.
constexpr int kWaveGroupVecs = 32;

// WPG > 1: one group per workgroup of WPG wavefronts (groups of more than 4096
// elements), wavefront w holding vectors j*64*WPG + 64*w + lane, the wavefronts'
// maxima combined through LDS: a row of 14336 per channel otherwise leaves one
// wavefront per row holding 32 vectors a lane, too few wavefronts to fill the chip
// for a 4096-row matrix.
template <int FMT, int MODE, int NV, bool ENCODE = true, int WPG = 1>
__global__ __launch_bounds__(WPG == 1 ? kBlock : kWave * WPG) void quantize_wave_groups(
    const _Float16* __restrict__ x, Geom g, float* __restrict__ scales, uint8_t* __restrict__ q) {
    constexpr float kMax = fp8_max(FMT);
    constexpr int kSpan = kWave * WPG;   // vectors per j
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = WPG == 1 ? 0 : (int)(threadIdx.x / kWave);
    const long long grp = WPG == 1 ? (long long)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave
                                   : (long long)blockIdx.x;
    if (grp >= g.n_groups) return;   // wavefront-uniform (workgroup-uniform for WPG > 1)
    const long long base = grp * g.gs;
    const int nv = (int)(min(g.gs, g.n - base) / 8);   // vectors of this group
    const Vec<_Float16, 8>* xv = reinterpret_cast<const Vec<_Float16, 8>*>(x + base);
    const int off = kWave * wv + lane;   // this lane's vector inside each span
    Vec<_Float16, 8> h[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j)
        if (j * kSpan < nv) h[j] = load<true>(xv + min(j * kSpan + off, nv - 1));   // uniform test
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = j * kSpan + off;
        if (i < nv && seen(MODE, (long long)i * 8)) {
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf((float)h[j].v[e]));
        }
    }
    m = wave_max(m);
    if constexpr (WPG > 1) {
        __shared__ float red[WPG];
        if (lane == 0) red[wv] = m;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < WPG; ++w) m = fmaxf(m, red[w]);
    }
    const float sc = m < 1e-8f ? 1.0f : kMax / m;
    if (lane == 0 && wv == 0) scales[grp] = sc;
    if constexpr (ENCODE) {
        u32x2* qv = reinterpret_cast<u32x2*>(q + base);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int i = j * kSpan + off;
            if (i < nv) store<true>(qv + i, encode8<FMT, MODE>(h[j], sc));
        }
    }
}

template <int FMT, int MODE>
__device__ __forceinline__ float decode1(uint32_t q) {
    if constexpr (MODE == QL_FP8_MODE_REFERENCE) return dec_ref<FMT>(q);
    else return dec_ocp2<FMT>(q)[0];
}

// d / s for a decoded code d: with r = RN(1/s) and s in [2^-90, 2^90] (every step
// normal: |d| lies in [2^-16, 2^17]), q0 = d * r plus one fma correction is RN(d / s)
// exactly (exhaustive over a binade of s and every FP8 mantissa on the CPU; every
// step scales exactly by powers of two).  Zeros, infinities and NaNs take q0
// (signed zeros keep their sign).  Callers outside that range of s divide.
__device__ __forceinline__ bool recip_ok(float s) { return s >= 0x1p-90f && s <= 0x1p90f; }
__device__ __forceinline__ float div_by_recip(float d, float s, float r) {
    const float q0 = d * r;
    const float q1 = fmaf(fmaf(-q0, s, d), r, q0);
    return d != 0.0f && __builtin_isfinite(d) ? q1 : q0;
}

// the four codes of w, decoded
template <int FMT, int MODE>
__device__ __forceinline__ void decode4(uint32_t w, float (&d)[4]) {
    if constexpr (MODE == QL_FP8_MODE_REFERENCE) {
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e] = dec_ref<FMT>((w >> (8 * e)) & 0xFFu);
    } else {
        const float2v lo = dec_ocp2<FMT>(w), hi = dec_ocp2<FMT, true>(w);
        d[0] = lo[0];
        d[1] = lo[1];
        d[2] = hi[0];
        d[3] = hi[1];
    }
}

// 16 codes per thread (n % 16 == 0, gs % 16 == 0, 16-byte aligned codes and output):
// one 16-byte load, the group's scale and its reciprocal once, two 16-byte stores.
template <int FMT, int MODE>
__global__ __launch_bounds__(kBlock) void dequantize16(const uint8_t* __restrict__ q, Geom g,
                                                       const float* __restrict__ scales,
                                                       _Float16* __restrict__ y) {
    const long long t = (long long)blockIdx.x * kBlock + threadIdx.x;
    if (t * 16 >= g.n) return;
    const u32x4 w = load<true>(reinterpret_cast<const u32x4*>(q) + t);
    const long long e0 = t * 16;
    const long long gi = g.n <= 0xFFFFFFFFLL ? (long long)((uint32_t)e0 / (uint32_t)g.gs) : e0 / g.gs;
    const float s = scales[gi];
    Vec<_Float16, 8> out[2];
    if (recip_ok(s)) {
        const float r = 1.0f / s;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float d[4];
            decode4<FMT, MODE>(w[j], d);
#pragma unroll
            for (int e = 0; e < 4; ++e) out[j >> 1].v[4 * (j & 1) + e] = from_f32<_Float16>(div_by_recip(d[e], s, r));
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float d[4];
            decode4<FMT, MODE>(w[j], d);
#pragma unroll
            for (int e = 0; e < 4; ++e) out[j >> 1].v[4 * (j & 1) + e] = from_f32<_Float16>(d[e] / s);
        }
    }
    store<true>(reinterpret_cast<Vec<_Float16, 8>*>(y) + 2 * t, out[0]);
    store<true>(reinterpret_cast<Vec<_Float16, 8>*>(y) + 2 * t + 1, out[1]);
}

template <int FMT, int MODE, bool VEC>
__global__ __launch_bounds__(kBlock) void dequantize_kernel(const uint8_t* __restrict__ q, Geom g,
                                                            const float* __restrict__ scales,
                                                            _Float16* __restrict__ y) {
    const long long t = (long long)blockIdx.x * kBlock + threadIdx.x;
    if constexpr (VEC) {
        if (t * 8 >= g.n) return;
        const u32x2 w = load<true>(reinterpret_cast<const u32x2*>(q) + t);
        Vec<_Float16, 8> out;
        if (g.gs % 8) {   // uniform: groups start inside vectors
            float s8[8];
            scales8(scales, g, t * 8, s8);
            bool ok = true;
#pragma unroll
            for (int e = 0; e < 8; ++e) ok = ok && recip_ok(s8[e]);
            if (ok) {   // both forms give RN(d / s); at most 2 distinct scales when gs >= 8
                float r8[8];
                if (g.gs >= 8) {   // s8 holds the scales of at most two groups, in order
                    const float ra = 1.0f / s8[0], rb = 1.0f / s8[7];
#pragma unroll
                    for (int e = 0; e < 8; ++e) r8[e] = s8[e] == s8[0] ? ra : rb;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) r8[e] = 1.0f / s8[e];
                }
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    out.v[e] = from_f32<_Float16>(
                        div_by_recip(decode1<FMT, MODE>((w[e >> 2] >> (8 * (e & 3))) & 0xFFu), s8[e], r8[e]));
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    out.v[e] = from_f32<_Float16>(decode1<FMT, MODE>((w[e >> 2] >> (8 * (e & 3))) & 0xFFu) / s8[e]);
            }
            store<true>(reinterpret_cast<Vec<_Float16, 8>*>(y) + t, out);
            return;
        }
        const float s = scales[(t * 8) / g.gs];
        if (recip_ok(s)) {
            const float r = 1.0f / s;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                out.v[e] = from_f32<_Float16>(div_by_recip(decode1<FMT, MODE>((w[e >> 2] >> (8 * (e & 3))) & 0xFFu), s, r));
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                out.v[e] = from_f32<_Float16>(decode1<FMT, MODE>((w[e >> 2] >> (8 * (e & 3))) & 0xFFu) / s);
        }
        store<true>(reinterpret_cast<Vec<_Float16, 8>*>(y) + t, out);
    } else {
        if (t >= g.n) return;
        y[t] = from_f32<_Float16>(decode1<FMT, MODE>(q[t]) / scales[t / g.gs]);
    }
}

// ---- skinny GEMM: C[M,N] = A[M,K] (dequant W[N,K])^T, M <= 64 --------------------------
// Computed as C^T = W' A^T with v_mfma_f32_16x16x32_f16: the weights are the A
// operand (16 rows x 32 k), the tokens the B operand (32 k x 16 tokens).
// Workgroup (4 wavefronts): R row tiles of 16 weight rows x all M tokens (MT tiles
// of 16) over one K-split's range of 64-k chunks; wavefront w takes chunks
// w, w+4, ... of that range, so the four read adjacent halves of each row's cache
// lines together.  Per chunk a lane loads 16 codes of row (tile base + lane%16) at
// k = 16*(lane/16) .. +15 and the same 16 k of token (16t + lane%16) -- the k order
// inside a chunk is permuted identically for both operands, so the products pair
// up -- and each token fragment serves all R row tiles.  Chunks stream through a
// ring of 3-4 register stages.  Token rows past M load row M-1 (in bounds): they
// only feed C^T columns that are never written.  The wavefronts' partial tiles are
// summed in LDS; with several K-splits the split's fp32 partial goes to
// part[split][M][N] and splitk_reduce sums the splits in order (deterministic).
constexpr int kGemmWaves = 4;

// scale lookup of the register path: one scale (tensor), one per weight row, per
// group with K % gs == 0 from the workgroup's LDS table of inverses -- applied to
// each 64-k chunk's sums when gs % 64 == 0 (GroupFold), else to each weight
// (GroupLds) -- or from global memory (Group), and groups that straddle rows (Any)
enum ScaleKind {
    kScaleTensor = 0, kScaleRow = 1, kScaleGroupFold = 2, kScaleGroupLds = 3, kScaleGroup = 4, kScaleAny = 5
};

// bytes of 4 reference-mode codes whose reference decode differs from the OCP
// decode (bit 7 of each byte of the result): E4M3 exponent 0 with a non-zero
// mantissa (the reference reads it as a normal number) and |code| 0x7F (the
// reference's 480, OCP's NaN); E5M2 exponent 0 with a non-zero mantissa and
// exponent 31 (finite in the reference).  With l = |code| (7 bits) per byte,
// l + 0x7F has bit 7 iff l >= 1, 0x87 - l (or 0x83 - l) iff l <= 7 (l <= 3), and
// l + 0x01 (l + 0x04) iff l == 0x7F (l >= 0x7C); none of these carries or borrows
// across bytes.  The caller masks the OR of several words with 0x80808080.
template <int FMT>
__device__ __forceinline__ uint32_t ref_special(uint32_t w) {
    const uint32_t l = w & 0x7F7F7F7Fu;
    const uint32_t ge1 = l + 0x7F7F7F7Fu;
    const uint32_t le_m = (FMT == QL_FP8_E4M3 ? 0x87878787u : 0x83838383u) - l;
    const uint32_t top = l + (FMT == QL_FP8_E4M3 ? 0x01010101u : 0x04040404u);
    return (ge1 & le_m) | top;
}

// 16 codes -> two fp16 fragments of binary16(decode(code) * inv).  The hardware
// decode is exact for every OCP code; in reference mode it is used when none of a
// lane's 16 codes is one of the codes whose reference value differs (the reference
// encoder only writes such a code for a NaN input) and the lane falls back to the
// bitwise reference decode otherwise.  SCALED = false leaves the scale out (the
// caller applies it to the accumulated products): every FP8 value is exact in
// binary16, so the fragments then hold the decoded codes themselves, converted
// two at a time straight to binary16 (callers keep reference-mode E5M2, whose
// exponent-31 codes exceed the binary16 range, on SCALED = true).
template <int FMT, int MODE, bool SCALED>
__device__ __forceinline__ void dequant16(uint4 codes, float inv, half8& lo, half8& hi) {
    const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
    if constexpr (!SCALED) {
        // straight to binary16: one conversion per two codes
        half2v h[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h[2 * j] = dec_ocp2_h<FMT>(w[j]);
            h[2 * j + 1] = dec_ocp2_h<FMT, true>(w[j]);
        }
        if constexpr (MODE == QL_FP8_MODE_REFERENCE) {
            const uint32_t special = (ref_special<FMT>(w[0]) | ref_special<FMT>(w[1]) | ref_special<FMT>(w[2]) |
                                      ref_special<FMT>(w[3])) & 0x80808080u;
            if (special) {
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    h[e >> 1][e & 1] = (_Float16)dec_ref<FMT>((w[e >> 2] >> (8 * (e & 3))) & 0xFFu);
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            lo[e] = h[e >> 1][e & 1];
            hi[e] = h[4 + (e >> 1)][e & 1];
        }
        return;
    }
    float f[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float2v a = dec_ocp2<FMT>(w[j]);
        const float2v b = dec_ocp2<FMT, true>(w[j]);
        f[4 * j] = a[0];
        f[4 * j + 1] = a[1];
        f[4 * j + 2] = b[0];
        f[4 * j + 3] = b[1];
    }
    if constexpr (MODE == QL_FP8_MODE_REFERENCE) {
        const uint32_t special = (ref_special<FMT>(w[0]) | ref_special<FMT>(w[1]) | ref_special<FMT>(w[2]) |
                                  ref_special<FMT>(w[3])) & 0x80808080u;
        if (special) {
#pragma unroll
            for (int e = 0; e < 16; ++e) f[e] = dec_ref<FMT>((w[e >> 2] >> (8 * (e & 3))) & 0xFFu);
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        lo[e] = (_Float16)(f[e] * inv);
        hi[e] = (_Float16)(f[8 + e] * inv);
    }
}

struct SkinnyArgs {
    const char* A;        // byte views: every offset below 2^32 (checked on the host)
                          // (packed_a: the fragment-major copy of the token rows)
    const char* W;
    const float* scales;
    _Float16* C;
    float* part;          // [splits][M][N] fp32 partials (splits > 1)
    int M, N, K;
    int chunks_per_split; // in the kernel's chunks (64 codes; 128 wide, 256 whole-row)
    long long gs;         // group length in elements
    int groups_per_row;   // K / gs (kScaleGroup)
    int g_step, r_step;   // 256 / gs, 256 % gs: a wavefront's next chunk starts 256 k on
    int packed_a;         // register path: A holds the token fragments fragment-major
};

// Fragment-major token layout of the register path (more than 32 tokens): the
// fragment of chunk c (64 k), token tile t and half h is 64 lanes x 16 bytes,
// lane l = 16*kq + j holding A[16t + j][64c + 16kq + 8h .. +7] (zeros past the
// last token), so each fragment load reads one contiguous 1 KiB (8 whole cache
// lines) instead of 16 half-used lines of the row-major rows.
constexpr uint32_t kPackFrag = 64u * 16u;   // bytes per fragment

__host__ __device__ constexpr size_t packed_a_bytes(int K, int mt) {
    return (size_t)(K / 64) * (size_t)mt * 2u * kPackFrag;
}

// One thread per 16-byte fragment slot (written in order, so the stores coalesce).
__global__ __launch_bounds__(kBlock) void pack_tokens(const _Float16* __restrict__ A, uint4* __restrict__ P,
                                                      int M, int K, int MT) {
    const long long i = (long long)blockIdx.x * kBlock + threadIdx.x;
    const long long total = (long long)(K / 64) * MT * 2 * kWave;
    if (i >= total) return;
    const int lane = (int)(i & (kWave - 1));
    const long long f = i / kWave;             // (c * MT + t) * 2 + h
    const int h = (int)(f & 1);
    const long long ct = f >> 1;
    const int t = (int)(ct % MT), c = (int)(ct / MT);
    const int j = lane & 15, kq = lane >> 4;
    const int row = 16 * t + j;
    uint4 v = {0u, 0u, 0u, 0u};
    if (row < M) v = *reinterpret_cast<const uint4*>(A + (size_t)row * K + 64 * c + 16 * kq + 8 * h);
    P[i] = v;
}

template <int MT, int R>
struct SkStage {
    uint4 w[R];
    half8 a[MT][2];
    float s[R];
    int gi;               // kScaleGroupFold: the chunk's group, relative to the table
};

// Per-tensor and per-row scales are applied once to the accumulated products
// instead of to every weight, except for reference-mode E5M2, whose exponent-31
// codes decode beyond the binary16 range before scaling.
template <int FMT, int MODE, int SK>
constexpr bool fold_scale() {
    return SK <= kScaleRow && !(MODE == QL_FP8_MODE_REFERENCE && FMT == QL_FP8_E5M2);
}

template <int SK>
__device__ __forceinline__ float scale_at(const SkinnyArgs& p, int row, int k) {
    if constexpr (SK == kScaleTensor) return p.scales[0];
    else if constexpr (SK == kScaleRow) return p.scales[row];
    else if constexpr (SK == kScaleAny) return p.scales[((long long)row * p.K + k) / p.gs];
    else return p.scales[row * p.groups_per_row + (int)((unsigned)k / (unsigned)p.gs)];
}

// kScaleGroup*: the group of a lane's next chunk, advanced by 256 k per load (the
// loads of a wavefront run through its chunks in order, 4 apart) and clamped to
// the group of its last chunk (the loads past the end repeat that chunk).  For
// kScaleGroupFold the whole chunk lies in one group, so the cursor is uniform.
struct GroupCursor {
    int g, rem, g_last;
    const float* lds;     // inverse scales of groups g0 .. g0+ng-1: [NR][ng] (GroupLds),
    int ng, g0;           // [ng][NR] (GroupFold)
};

template <int MT, int R, int SK>
__device__ __forceinline__ void sk_load(SkStage<MT, R>& st, const SkinnyArgs& p, const uint32_t (&woff)[R],
                                        const int (&row)[R], const uint32_t (&aoff)[MT], int c, int kq,
                                        GroupCursor& gc) {
    const uint32_t k = (uint32_t)c * 64u;
#pragma unroll
    for (int r = 0; r < R; ++r) st.w[r] = *reinterpret_cast<const uint4*>(p.W + (woff[r] + k));
    // row-major rows: the chunk is 128 bytes on, the second half 16; fragment-major:
    // MT * 2 fragments on, the second half one fragment
    const uint32_t a_c = p.packed_a ? (uint32_t)c * (uint32_t)(MT * 2) * kPackFrag : 2u * k;
    const uint32_t a_h = p.packed_a ? kPackFrag : 16u;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        st.a[t][0] = *reinterpret_cast<const half8*>(p.A + (aoff[t] + a_c));
        st.a[t][1] = *reinterpret_cast<const half8*>(p.A + (aoff[t] + a_c + a_h));
    }
    if constexpr (SK == kScaleGroupFold || SK == kScaleGroupLds || SK == kScaleGroup) {
        const int g = min(gc.g, gc.g_last);
        const int lane16 = threadIdx.x & 15;
        if constexpr (SK == kScaleGroupFold) st.gi = g - gc.g0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (SK == kScaleGroupLds) st.s[r] = gc.lds[(16 * r + lane16) * gc.ng + g - gc.g0];
            else if constexpr (SK == kScaleGroup) st.s[r] = p.scales[row[r] * p.groups_per_row + g];
        }
        gc.g += p.g_step;
        gc.rem += p.r_step;
        if (gc.rem >= (int)p.gs) {
            gc.rem -= (int)p.gs;
            ++gc.g;
        }
    } else if constexpr (SK == kScaleAny) {
#pragma unroll
        for (int r = 0; r < R; ++r) st.s[r] = scale_at<SK>(p, row[r], (int)k + 16 * kq);
    }
}

template <int FMT, int MODE, int MT, int R, int SK>
__device__ __forceinline__ void sk_compute(const SkStage<MT, R>& st, const float (&inv_fixed)[R],
                                           const float* table, int kq, floatx4 (&acc)[R][MT]) {
    constexpr bool kFold = fold_scale<FMT, MODE, SK>();
    if constexpr (SK == kScaleGroupFold) {
        // the chunk's products of decoded codes, then one multiply-add per output
        // by the inverse scale of its weight row (lane rows 16r + 4*kq + i)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            half8 wlo, whi;
            dequant16<FMT, MODE, false>(st.w[r], 1.0f, wlo, whi);
            const float4 inv = *reinterpret_cast<const float4*>(table + st.gi * (16 * R) + 16 * r + 4 * kq);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                floatx4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(wlo, st.a[t][0], floatx4{}, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi, st.a[t][1], c, 0, 0, 0);
                acc[r][t][0] = fmaf(c[0], inv.x, acc[r][t][0]);
                acc[r][t][1] = fmaf(c[1], inv.y, acc[r][t][1]);
                acc[r][t][2] = fmaf(c[2], inv.z, acc[r][t][2]);
                acc[r][t][3] = fmaf(c[3], inv.w, acc[r][t][3]);
            }
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        // v_rcp_f32 (1 ulp): the weight is rounded to binary16 right after
        const float inv = SK <= kScaleRow ? inv_fixed[r]
                                          : (SK == kScaleGroupLds ? st.s[r] : __builtin_amdgcn_rcpf(st.s[r]));
        half8 wlo, whi;
        dequant16<FMT, MODE, !kFold>(st.w[r], inv, wlo, whi);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            acc[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wlo, st.a[t][0], acc[r][t], 0, 0, 0);
            acc[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi, st.a[t][1], acc[r][t], 0, 0, 0);
        }
    }
}

// floats of the skinny kernel's LDS: the four wavefronts' partial tiles, and at
// least 16 KB for the inverse-scale table
__host__ __device__ constexpr int skinny_smem_floats(int nr, int mc, int sk) {
    return (sk == kScaleGroupLds || sk == kScaleGroupFold) && kGemmWaves * nr * (mc + 1) < 4096
               ? 4096
               : kGemmWaves * nr * (mc + 1);
}

template <int FMT, int MODE, int MT, int R, int SK>
__global__ __launch_bounds__(kGemmWaves * kWave) void fp8_gemm_skinny(SkinnyArgs p) {
    constexpr int NR = 16 * R, MC = 16 * MT;
    constexpr bool kFold = fold_scale<FMT, MODE, SK>();
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * NR;
    const int kq = lane >> 4;
    const int n_chunks = p.K / 64;
    const int c_begin = blockIdx.y * p.chunks_per_split;
    const int c_end = min(n_chunks, c_begin + p.chunks_per_split);
    uint32_t woff[R];
    int row[R];
    float inv_fixed[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        row[r] = n0 + 16 * r + (lane & 15);
        woff[r] = (uint32_t)row[r] * (uint32_t)p.K + 16u * kq;
        inv_fixed[r] = 1.0f;
        if constexpr (SK <= kScaleRow && !kFold) inv_fixed[r] = 1.0f / scale_at<SK>(p, row[r], 0);
    }
    uint32_t aoff[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t)
        aoff[t] = p.packed_a ? (uint32_t)(2 * t) * kPackFrag + 16u * (uint32_t)lane
                             : 2u * ((uint32_t)min(16 * t + (lane & 15), p.M - 1) * (uint32_t)p.K + 16u * kq);
    floatx4 acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[r][t] = floatx4{};

    // LDS: the inverse-scale table during the loop (kScaleGroupLds; the host checks
    // that NR * ng fits), then the partial tiles
    constexpr int kSmemFloats = skinny_smem_floats(NR, MC, SK);
    __shared__ float smem[kSmemFloats];
    GroupCursor gc{0, 0, 0, nullptr, 0, 0};
    if constexpr (SK == kScaleGroupLds || SK == kScaleGroupFold) {
        const int gs = (int)p.gs;
        gc.g0 = c_begin * 64 / gs;
        gc.ng = (c_end * 64 - 1) / gs + 1 - gc.g0;
        for (int i = threadIdx.x; i < NR * gc.ng; i += kGemmWaves * kWave) {
            int rr, gg;
            if constexpr (SK == kScaleGroupFold) {   // group-major: a lane's 4 rows are adjacent
                gg = i / NR;
                rr = i - gg * NR;
            } else {
                rr = i / gc.ng;
                gg = i - rr * gc.ng;
            }
            smem[i] = 1.0f / p.scales[(n0 + rr) * p.groups_per_row + gc.g0 + gg];
        }
        gc.lds = smem;
        __syncthreads();
    }

    // ring of NS register stages: stage s holds chunk first + 4*(s + NS*j); while one
    // is dequantized and multiplied the loads of the other NS - 1 are in flight.
    // Loads past the wavefront's last chunk repeat that chunk (in bounds, never
    // used), so every round issues the same loads and the waits count them exactly.
    constexpr int NS = MT == 4 ? 3 : 4;
    const int first = c_begin + wave;              // wave-uniform
    if (first < c_end) {
        const int last = first + kGemmWaves * ((c_end - 1 - first) / kGemmWaves);
        if constexpr (SK == kScaleGroupFold || SK == kScaleGroupLds || SK == kScaleGroup) {
            const int kl = SK == kScaleGroupFold ? 0 : 16 * kq;
            const int k0 = first * 64 + kl;
            gc.g = k0 / (int)p.gs;
            gc.rem = k0 - gc.g * (int)p.gs;
            gc.g_last = (last * 64 + kl) / (int)p.gs;
        }
        SkStage<MT, R> st[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s)
            sk_load<MT, R, SK>(st[s], p, woff, row, aoff, min(first + kGemmWaves * s, last), kq, gc);
        for (int c0 = first; c0 <= last; c0 += kGemmWaves * NS) {
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const int cs = c0 + kGemmWaves * s;
                if (cs <= last) sk_compute<FMT, MODE, MT, R, SK>(st[s], inv_fixed, gc.lds, kq, acc);
                sk_load<MT, R, SK>(st[s], p, woff, row, aoff, min(cs + kGemmWaves * NS, last), kq, gc);
            }
        }
    }
    if constexpr (SK == kScaleGroupLds || SK == kScaleGroupFold)
        __syncthreads();   // the table's space is reused below
    // lane holds C^T[16r + 4*(lane/16) + i][16t + lane%16]; sum the four wavefronts
    // (the folded scale is per weight row, i.e. per i)
    float (*part)[NR][MC + 1] = reinterpret_cast<float (*)[NR][MC + 1]>(smem);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float rs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (kFold) {
#pragma unroll
            for (int i = 0; i < 4; ++i) rs[i] = 1.0f / scale_at<SK>(p, n0 + 16 * r + 4 * kq + i, 0);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                part[wave][16 * r + 4 * kq + i][16 * t + (lane & 15)] = kFold ? acc[r][t][i] * rs[i] : acc[r][t][i];
    }
    __syncthreads();
    const int m_end = min(p.M, MC);
    for (int e = threadIdx.x; e < NR * m_end; e += kGemmWaves * kWave) {
        const int m = e / NR, nn = e % NR;
        float s = part[0][nn][m];
#pragma unroll
        for (int w = 1; w < kGemmWaves; ++w) s += part[w][nn][m];
        const size_t o = (size_t)m * p.N + n0 + nn;
        if (gridDim.y == 1) p.C[o] = from_f32<_Float16>(s);
        else p.part[(size_t)blockIdx.y * p.M * p.N + o] = s;
    }
}

// ---- four token tiles (33-64 tokens): whole-line loads ---------------------------------
// Workgroup (4 wavefronts) = 64 weight rows x 64 tokens over one K-split's range of
// 128-k chunks; wavefront w takes chunks w, w+4, ...  Per chunk each weight load
// instruction covers 8 complete 128-byte row lines (lane l: row 8i + l/8, bytes
// 16*(l%8)), so a load touches 8 lines instead of 16 half-used ones; the chunk is
// re-laid through a wavefront-private 8 KB LDS tile (16-byte slots XOR-swizzled by
// row, conflict-free for both the writes and the fragment reads; one wavefront's
// LDS operations complete in order, so no barrier) into the register path's
// fragments: for row tile r and 64-k half s, lane (j = l%16, kq = l/16) takes slot
// 4s + kq of row 16r + j, i.e. codes 64s + 16kq .. +15 of the chunk, matching the
// token fragments of 64-k chunk 2c + s.  Tokens (TS, fixed per scale kind by
// wide_token_stages from measurements): TS = 0 loads the fragments from the
// fragment-major copy; TS = 1, 2 read the token rows themselves, 4 rows x 256
// bytes per instruction, re-laid through a second wavefront tile (16 KB, column
// XORed with row % 16) with 1 or 2 chunks of them in registers.  Scales: per
// tensor / per row applied to the sums (for reference-mode E5M2, per row to the
// weights); per group from the workgroup's LDS table of inverses -- for groups of
// a multiple of 64 codes one multiply-add per output per group-chunk on the sums
// of decoded codes (not reference-mode E5M2), else per weight.  The fp32 summation
// order differs from the register kernel's (another split of K over the
// wavefronts), not the bound; TS does not change it.
constexpr int kWideChunk = 128;
constexpr int kWideStages = 2;
constexpr int kWideTileU4 = 64 * 8;    // 16-byte slots per wavefront weight tile
constexpr int kWideTokU4 = 64 * 16;    // 16-byte slots per wavefront token tile
constexpr int kWideTableFloats = 4096;

// token staging per (decode mode, scale kind): measured on MI355X at 48 and 64
// tokens x 14336 x 4096 and 4096 x 14336 (us per call, copy / 1 / 2 stages):
// per channel 25.2 / 24.7 / 23.8 and 27.5 / 26.3 / 24.9; groups of 128, OCP decode
// 26.2 / 25.5 / 26.6 and 29.0 / 28.0 / 28.2; reference decode 28.2 / 30.5 / 37.2
// and 30.1 / 32.0 / 36.5 (the two direct forms need more registers than that
// instance has without spilling)
__host__ __device__ constexpr int wide_token_stages(int mode, int sk) {
    return sk <= kScaleRow ? 2 : (sk == kScaleGroupFold && mode == QL_FP8_MODE_OCP ? 1 : 0);
}

template <int TS>
struct WideStage {
    u32x4 w[8];
    // TS 0: fragments [64-k half s][token tile t][half h]; TS 2: raw row segments
    // (instruction i: rows 4i .. 4i+3); TS 1 keeps one set outside the ring
    std::conditional_t<TS == 0, half8[2][4][2], std::conditional_t<TS == 2, u32x4[16], u32x4[1]>> a;
};

// slot of (row, 16-byte column) in a wavefront tile: rows of 128 bytes, the column
// XORed with (row ^ row/8) % 8 -- distinct over any 8 consecutive rows and over
// the even and the odd rows of any 16
__device__ __forceinline__ int wide_slot(int row, int col) {
    return row * 8 + (col ^ ((row ^ (row >> 3)) & 7));
}

template <int TS>
__device__ __forceinline__ void wide_load_w(WideStage<TS>& st, const SkinnyArgs& p, const uint32_t (&woff)[8], int c) {
    const uint32_t kb = (uint32_t)c * kWideChunk;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.w[i] = *reinterpret_cast<const u32x4*>(p.W + (woff[i] + kb));
}

// copy: chunk c is 64-k chunks 2c and 2c + 1, 16 KB of fragments from byte c * 16 KB
__device__ __forceinline__ void wide_load_frags(half8 (&a)[2][4][2], const SkinnyArgs& p, uint32_t lane16, int c) {
    const uint32_t base = (uint32_t)c * (2u * 4u * 2u * kPackFrag) + lane16;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                a[s][t][h] = *reinterpret_cast<const half8*>(p.A + base + (uint32_t)((s * 4 + t) * 2 + h) * kPackFrag);
}

// token rows: the chunk's 256 bytes of each row, lane l of instruction i reading
// row 4i + l/16 (rows past M repeat row M - 1: in bounds, and their products only
// reach outputs that are never written), bytes 16*(l%16) of the chunk
__device__ __forceinline__ void wide_load_rows(u32x4 (&a)[16], const SkinnyArgs& p, const uint32_t (&aoff)[16], int c) {
    const uint32_t kb = (uint32_t)c * (2u * kWideChunk);
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = *reinterpret_cast<const u32x4*>(p.A + (aoff[i] + kb));
}

template <int FMT, int MODE, int SK>
__global__ __launch_bounds__(kGemmWaves * kWave) void fp8_gemm_wide(SkinnyArgs p) {
    constexpr int NR = 64, MC = 64;
    constexpr int TS = wide_token_stages(MODE, SK);
    constexpr bool kFold = fold_scale<FMT, MODE, SK>();
    static_assert(SK == kScaleTensor || SK == kScaleRow || SK == kScaleGroupFold || SK == kScaleGroupLds,
                  "wide kernel scale kinds");
    const int lane = threadIdx.x & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int j = lane & 15, kq = lane >> 4;
    const int n0 = blockIdx.x * NR;
    const int n_chunks = p.K / kWideChunk;
    const int c_begin = blockIdx.y * p.chunks_per_split;
    const int c_end = min(n_chunks, c_begin + p.chunks_per_split);
    uint32_t woff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) woff[i] = (uint32_t)(n0 + 8 * i + (lane >> 3)) * (uint32_t)p.K + 16u * (lane & 7);
    uint32_t aoff[16];   // TS > 0: token row segments
#pragma unroll
    for (int i = 0; i < 16; ++i)
        aoff[i] = 2u * (uint32_t)min(4 * i + (lane >> 4), p.M - 1) * (uint32_t)p.K + 16u * (lane & 15);
    float inv_fixed[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        inv_fixed[r] = 1.0f;
        if constexpr (SK <= kScaleRow && !kFold) inv_fixed[r] = 1.0f / scale_at<SK>(p, n0 + 16 * r + j, 0);
    }
    floatx4 acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[r][t] = floatx4{};

    // LDS: the wavefront tiles and the inverse-scale table ([NR][ng], GroupLds; the
    // host checks NR * ng <= kWideTableFloats) during the loop, then the partial tiles
    constexpr int kTileFloats = kGemmWaves * (kWideTileU4 + (TS > 0 ? kWideTokU4 : 0)) * 4;
    constexpr int kLoopFloats = kTileFloats + (SK >= kScaleGroupFold ? kWideTableFloats : 0);
    constexpr int kPartFloats = kGemmWaves * NR * (MC + 1);
    __shared__ __align__(16) float smem[kLoopFloats > kPartFloats ? kLoopFloats : kPartFloats];
    u32x4* tile = reinterpret_cast<u32x4*>(smem) + wave * kWideTileU4;
    u32x4* ttile = reinterpret_cast<u32x4*>(smem) + kGemmWaves * kWideTileU4 + wave * kWideTokU4;   // TS > 0
    const float* table = smem + kTileFloats;
    int g0 = 0, ng = 0;
    if constexpr (SK == kScaleGroupLds || SK == kScaleGroupFold) {
        const int gs = (int)p.gs;
        g0 = c_begin * kWideChunk / gs;
        ng = (c_end * kWideChunk - 1) / gs + 1 - g0;
        for (int i = threadIdx.x; i < NR * ng; i += kGemmWaves * kWave) {
            int rr, gg;
            if constexpr (SK == kScaleGroupFold) {   // group-major: a lane's 4 rows are adjacent
                gg = i / NR;
                rr = i - gg * NR;
            } else {
                rr = i / ng;
                gg = i - rr * ng;
            }
            smem[kTileFloats + i] = 1.0f / p.scales[(n0 + rr) * p.groups_per_row + g0 + gg];
        }
        __syncthreads();
    }
    int wslot[8], rslot[4][2];
#pragma unroll
    for (int i = 0; i < 8; ++i) wslot[i] = wide_slot(8 * i + (lane >> 3), lane & 7);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int s = 0; s < 2; ++s) rslot[r][s] = wide_slot(16 * r + j, 4 * s + kq);
    const uint32_t lane16 = 16u * (uint32_t)lane;
    // token tile: row 4i + l/16 of instruction i, 16-byte column l%16 XORed with row % 16
    int twslot[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) twslot[i] = (4 * i + (lane >> 4)) * 16 + ((lane & 15) ^ ((4 * i + (lane >> 4)) & 15));
    u32x4 tk[16];   // TS = 1: the next chunk's token rows

    // one chunk from stage st; with LOAD, the stage is refilled with chunk c_next
    // (weights and token rows as soon as they are in LDS, fragments after the
    // products); TS = 1 refills tk with chunk c_tok
    auto step = [&](WideStage<TS>& st, int c, int c_next, int c_tok, auto load) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) tile[wslot[i]] = st.w[i];
        if constexpr (decltype(load)::value) wide_load_w(st, p, woff, c_next);
        if constexpr (TS == 1) {
#pragma unroll
            for (int i = 0; i < 16; ++i) ttile[twslot[i]] = tk[i];
            wide_load_rows(tk, p, aoff, c_tok);
        } else if constexpr (TS == 2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) ttile[twslot[i]] = st.a[i];
            if constexpr (decltype(load)::value) wide_load_rows(st.a, p, aoff, c_next);
        }
        // orders the compiler only: one wavefront's LDS operations execute in order
        __builtin_amdgcn_wave_barrier();
        u32x4 codes[4][2];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int s = 0; s < 2; ++s) codes[r][s] = tile[rslot[r][s]];
        // token fragment (s, t, h): lane (j, kq) holds k = 64s + 16kq + 8h .. +7 of
        // token 16t + j, i.e. column 8s + 2kq + h of its row in the tile
        half8 frag[2][4][2];
        if constexpr (TS > 0) {
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        frag[s][t][h] = __builtin_bit_cast(half8, ttile[(16 * t + j) * 16 + ((8 * s + 2 * kq + h) ^ j)]);
        }
        __builtin_amdgcn_wave_barrier();
        auto fr = [&](int s_, int t_, int h_) __attribute__((always_inline)) -> const half8& {
            if constexpr (TS == 0) return st.a[s_][t_][h_];
            else return frag[s_][t_][h_];
        };
        if constexpr (SK == kScaleGroupFold) {
            // the products of decoded codes per group (the chunk, or each 64-k half
            // for groups of 64), then one multiply-add per output by the inverse
            // scale of its weight row (lane rows 16r + 4*kq + i)
            const bool halves = (int)p.gs % kWideChunk != 0;   // uniform
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                floatx4 part[4];
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    half8 wlo, whi;
                    const u32x4 cv = codes[r][s];
                    dequant16<FMT, MODE, false>(uint4{cv[0], cv[1], cv[2], cv[3]}, 1.0f, wlo, whi);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        part[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wlo, fr(s, t, 0), s == 0 ? floatx4{} : part[t], 0, 0, 0);
                        part[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi, fr(s, t, 1), part[t], 0, 0, 0);
                    }
                    if (s == 1 || halves) {
                        const int g = (c * kWideChunk + 64 * s) / (int)p.gs - g0;
                        const float4 inv = *reinterpret_cast<const float4*>(table + g * NR + 16 * r + 4 * kq);
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            acc[r][t][0] = fmaf(part[t][0], inv.x, acc[r][t][0]);
                            acc[r][t][1] = fmaf(part[t][1], inv.y, acc[r][t][1]);
                            acc[r][t][2] = fmaf(part[t][2], inv.z, acc[r][t][2]);
                            acc[r][t][3] = fmaf(part[t][3], inv.w, acc[r][t][3]);
                            part[t] = floatx4{};
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    // per-weight scale: the lane's row 16r + j, group of its 16 codes
                    float inv = inv_fixed[r];
                    if constexpr (SK == kScaleGroupLds)
                        inv = table[(16 * r + j) * ng + (c * kWideChunk + 64 * s + 16 * kq) / (int)p.gs - g0];
                    half8 wlo, whi;
                    const u32x4 cv = codes[r][s];
                    dequant16<FMT, MODE, !kFold>(uint4{cv[0], cv[1], cv[2], cv[3]}, inv, wlo, whi);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        acc[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wlo, fr(s, t, 0), acc[r][t], 0, 0, 0);
                        acc[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi, fr(s, t, 1), acc[r][t], 0, 0, 0);
                    }
                }
        }
        if constexpr (TS == 0) {
            if constexpr (decltype(load)::value) wide_load_frags(st.a, p, lane16, c_next);
        }
    };
    // ring of NS stages: stage s holds the wavefront's chunks s, s + NS, ... (4 apart
    // in K).  Whole rounds refill every stage (loads past the last chunk repeat it:
    // in bounds, never used, and the waits count every round's loads exactly); the
    // remaining chunks are computed without refills, except TS = 1's token rows,
    // loaded one chunk ahead in every step (the last step's repeat the last chunk).
    constexpr int NS = kWideStages, CS = kGemmWaves;
    const int first = c_begin + wave;   // wave-uniform
    if (first < c_end) {
        const int n_mine = (c_end - 1 - first) / CS + 1;
        const int last = first + CS * (n_mine - 1);
        WideStage<TS> st[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            wide_load_w(st[s], p, woff, min(first + CS * s, last));
            if constexpr (TS == 0) wide_load_frags(st[s].a, p, lane16, min(first + CS * s, last));
            if constexpr (TS == 2) wide_load_rows(st[s].a, p, aoff, min(first + CS * s, last));
            if constexpr (TS == 1)
                if (s == 0) wide_load_rows(tk, p, aoff, first);
        }
        const int rounds = n_mine / NS;
        int c = first;
        for (int rd = 0; rd < rounds; ++rd) {
#pragma unroll
            for (int s = 0; s < NS; ++s, c += CS)
                step(st[s], c, min(c + CS * NS, last), min(c + CS, last), std::true_type{});
        }
#pragma unroll
        for (int s = 0; s < NS - 1; ++s, c += CS)
            if (s < n_mine - rounds * NS) step(st[s], c, 0, min(c + CS, last), std::false_type{});
    }
    __syncthreads();   // the tiles' and the table's space is reused below
    // lane holds C^T[16r + 4*(lane/16) + i][16t + lane%16]; sum the four wavefronts
    float (*part)[NR][MC + 1] = reinterpret_cast<float (*)[NR][MC + 1]>(smem);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float rs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (kFold) {
#pragma unroll
            for (int i = 0; i < 4; ++i) rs[i] = 1.0f / scale_at<SK>(p, n0 + 16 * r + 4 * kq + i, 0);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                part[wave][16 * r + 4 * kq + i][16 * t + j] = kFold ? acc[r][t][i] * rs[i] : acc[r][t][i];
    }
    __syncthreads();
    const int m_end = min(p.M, MC);
    for (int e = threadIdx.x; e < NR * m_end; e += kGemmWaves * kWave) {
        const int m = e / NR, nn = e % NR;
        float s = part[0][nn][m];
#pragma unroll
        for (int w = 1; w < kGemmWaves; ++w) s += part[w][nn][m];
        const size_t o = (size_t)m * p.N + n0 + nn;
        if (gridDim.y == 1) p.C[o] = from_f32<_Float16>(s);
        else p.part[(size_t)blockIdx.y * p.M * p.N + o] = s;
    }
}

// C = binary16(sum over splits of part[s]), 4 outputs per thread (M*N % 4 == 0)
__global__ __launch_bounds__(kBlock) void splitk_reduce(const float* __restrict__ part,
                                                        _Float16* __restrict__ C, int splits,
                                                        long long mn) {
    const long long i = ((long long)blockIdx.x * kBlock + threadIdx.x) * 4;
    if (i >= mn) return;
    float4 s = *reinterpret_cast<const float4*>(part + i);
    for (int k = 1; k < splits; ++k) {
        const float4 v = *reinterpret_cast<const float4*>(part + (size_t)k * mn + i);
        s.x += v.x;
        s.y += v.y;
        s.z += v.z;
        s.w += v.w;
    }
    Vec<_Float16, 4> o;
    o.v[0] = from_f32<_Float16>(s.x);
    o.v[1] = from_f32<_Float16>(s.y);
    o.v[2] = from_f32<_Float16>(s.z);
    o.v[3] = from_f32<_Float16>(s.w);
    store<true>(reinterpret_cast<Vec<_Float16, 4>*>(C + i), o);
}

// ---- one token tile (M <= 16): whole-row weight loads -----------------------------------
// Workgroup = RW x KW wavefronts over 16*RW weight rows and one K-split: wavefront
// w owns row tile w % RW and every KW-th chunk of 256 codes from w / RW on.  One
// load instruction covers 4 complete 256-byte row segments (16 lanes per row): that
// shape streams the matrix markedly faster than 16 rows x 64 bytes.  Each chunk is
// re-laid through a wavefront-private LDS tile (16-byte slots XOR-swizzled by row,
// conflict-free both ways; LDS operations of one wavefront complete in order, so
// no barrier) into MFMA fragments: lane (row l%16, q = l/16) takes piece p = 0..3
// from slot 4p + q, i.e. codes 64p + 16q .. +15 of the chunk, and the token
// fragments use the same k order, so MFMA pair p covers k = 64p .. 64p + 63 of the
// chunk -- inside one scale group when the group length is a multiple of 64.
// Token rows come through a buffer resource that ends at row M: lanes of tokens
// past M read zeros without touching memory.  Scales: per tensor / per row applied
// once to the sums; per group (length a multiple of 64, dividing K) one multiply-add
// per output per piece with the inverse from the workgroup's LDS table.  The KW
// partial tiles of a row tile are summed in LDS in wavefront order.
constexpr int kRowsChunk = 256;
constexpr int kRowsStages = 2;        // register ring depth (chunks in flight)
constexpr int kRowsMaxTokens = 8;     // more tokens: the register path is faster
constexpr int kRowsOcpWaves = 1024;   // wavefront budgets of the launch shape
constexpr int kRowsRefWaves = 2048;
constexpr int kRowsTableFloats = 4096;
constexpr uint32_t kBufferWord3 = 0x00020000u;          // raw buffer, 32-bit dwords (gfx9)

struct RowsStage {
    u32x4 w[4];        // instruction i: row 4i + lane/16, bytes 16*(lane%16) .. of the chunk
    half8 a[4][2];     // piece p: token k = 64p + 16q .. +7 and +8 .. +15 of the chunk
};

__device__ __forceinline__ void rows_load_w(RowsStage& st, const SkinnyArgs& p, const uint32_t (&woff)[4], int c) {
    const uint32_t kb = (uint32_t)c * kRowsChunk;
#pragma unroll
    for (int i = 0; i < 4; ++i) st.w[i] = *reinterpret_cast<const u32x4*>(p.W + (woff[i] + kb));
}

__device__ __forceinline__ void rows_load_a(RowsStage& st, __amdgpu_buffer_rsrc_t ra, uint32_t aoff, int c) {
    const uint32_t kb = 2u * (uint32_t)c * kRowsChunk;
#pragma unroll
    for (int pc = 0; pc < 4; ++pc) {
        const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(ra, aoff + kb + 128u * pc, 0, 0);
        const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(ra, aoff + kb + 128u * pc + 16u, 0, 0);
        st.a[pc][0] = __builtin_bit_cast(half8, lo);
        st.a[pc][1] = __builtin_bit_cast(half8, hi);
    }
}

template <int FMT, int MODE, int SK, int RW, int KW>
__global__ __launch_bounds__(RW * KW * kWave) void fp8_gemm_rows(SkinnyArgs p) {
    constexpr int NW = RW * KW, NR = 16 * RW;
    // the wavefront index in a scalar register: the chunk loop's branches are uniform
    const int lane = threadIdx.x & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int rt = wave % RW, kp = wave / RW;
    const int q = lane >> 4, r16 = lane & 15;
    const int n0 = blockIdx.x * NR;
    const int rbase = n0 + 16 * rt;
    const int n_chunks = p.K / kRowsChunk;
    const int c_begin = blockIdx.y * p.chunks_per_split;
    const int c_end = min(n_chunks, c_begin + p.chunks_per_split);
    uint32_t woff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) woff[i] = (uint32_t)(rbase + 4 * i + q) * (uint32_t)p.K + 16u * r16;
    // byte offsets into the token rows; rows past M start at the resource's end
    // (the host checks (M + 1) * K * 2 < 2^32)
    const uint32_t a_bytes = 2u * (uint32_t)p.M * (uint32_t)p.K;
    const uint32_t aoff = (r16 < p.M ? 2u * (uint32_t)r16 * (uint32_t)p.K : a_bytes) + 32u * q;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p.A), (short)0, (int)a_bytes, (int)kBufferWord3);

    __shared__ u32x4 tile[NW][16][16];
    __shared__ float table[SK == kScaleGroupFold ? kRowsTableFloats : 1];   // [group - g0][NR rows]
    __shared__ floatx4 red[KW > 1 ? NW : 1][kWave];
    int g0 = 0;
    if constexpr (SK == kScaleGroupFold) {
        const int gs = (int)p.gs;
        g0 = c_begin * kRowsChunk / gs;
        const int ng = (c_end * kRowsChunk - 1) / gs + 1 - g0;   // the host checks NR * ng fits
        for (int i = threadIdx.x; i < NR * ng; i += NW * kWave) {
            const int gg = i / NR, rr = i - NR * gg;
            table[i] = 1.0f / p.scales[(n0 + rr) * p.groups_per_row + g0 + gg];
        }
        __syncthreads();
    }

    floatx4 acc = floatx4{};
    // one chunk from stage st: re-lay, decode, multiply; with LOAD, the stage is
    // refilled with chunk c_next (weights as soon as they are in LDS, tokens after
    // the products)
    auto step = [&](RowsStage& st, int c, int c_next, auto load) {
        // re-lay the chunk: row 4i + q, slot r16 -> position r16 ^ row
#pragma unroll
        for (int i = 0; i < 4; ++i) tile[wave][4 * i + q][r16 ^ (4 * i + q)] = st.w[i];
        if constexpr (decltype(load)::value) rows_load_w(st, p, woff, c_next);
        // orders the compiler only: one wavefront's LDS operations execute in order
        __builtin_amdgcn_wave_barrier();
        const u32x4 codes4[4] = {tile[wave][r16][q ^ r16], tile[wave][r16][(4 + q) ^ r16],
                                 tile[wave][r16][(8 + q) ^ r16], tile[wave][r16][(12 + q) ^ r16]};
        __builtin_amdgcn_wave_barrier();
        // pieces of one scale group (groups of 64 codes: every piece; 128: pairs;
        // 256 and longer: the whole chunk) share one partial and one multiply-add
        const int gp = SK == kScaleGroupFold ? min(4, (int)p.gs / 64) : 4;   // 1, 2 or 4 (gs % 64 == 0)
        floatx4 part = floatx4{};
#pragma unroll
        for (int pc = 0; pc < 4; ++pc) {
            const u32x4 cv = codes4[pc];
            half8 wlo, whi;
            dequant16<FMT, MODE, false>(uint4{cv[0], cv[1], cv[2], cv[3]}, 1.0f, wlo, whi);
            if constexpr (SK == kScaleGroupFold) {
                part = __builtin_amdgcn_mfma_f32_16x16x32_f16(wlo, st.a[pc][0], part, 0, 0, 0);
                part = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi, st.a[pc][1], part, 0, 0, 0);
                if ((pc + 1) % gp == 0) {   // wave-uniform
                    const int g = (c * kRowsChunk + 64 * pc) / (int)p.gs - g0;
                    const float4 inv = *reinterpret_cast<const float4*>(table + g * NR + 16 * rt + 4 * q);
                    acc[0] = fmaf(part[0], inv.x, acc[0]);
                    acc[1] = fmaf(part[1], inv.y, acc[1]);
                    acc[2] = fmaf(part[2], inv.z, acc[2]);
                    acc[3] = fmaf(part[3], inv.w, acc[3]);
                    part = floatx4{};
                }
            } else {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wlo, st.a[pc][0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi, st.a[pc][1], acc, 0, 0, 0);
            }
        }
        if constexpr (decltype(load)::value) rows_load_a(st, ra, aoff, c_next);
    };
    // ring of NS stages: stage s holds the wavefront's chunks s, s + NS, ...  Whole
    // rounds refill every stage (loads past the last chunk repeat it: in bounds,
    // never used, and the waits count every round's loads exactly); the remaining
    // chunks are computed without refills.
    constexpr int NS = kRowsStages;
    // wavefront kp of a row tile takes the kp-th contiguous run of the split's chunks
    constexpr int CS = 1;
    const int per_w = (c_end - c_begin + KW - 1) / KW;
    const int first = c_begin + kp * per_w;   // wave-uniform
    const int w_end = min(c_end, first + per_w);
    if (first < w_end) {
        const int n_mine = (w_end - 1 - first) / CS + 1;
        const int last = first + CS * (n_mine - 1);
        RowsStage st[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            rows_load_w(st[s], p, woff, min(first + CS * s, last));
            rows_load_a(st[s], ra, aoff, min(first + CS * s, last));
        }
        const int rounds = n_mine / NS;
        int c = first;
        for (int r = 0; r < rounds; ++r) {
#pragma unroll
            for (int s = 0; s < NS; ++s, c += CS) step(st[s], c, min(c + CS * NS, last), std::true_type{});
        }
#pragma unroll
        for (int s = 0; s < NS - 1; ++s, c += CS)
            if (s < n_mine - rounds * NS) step(st[s], c, 0, std::false_type{});
    }
    // lane holds C^T[rbase + 4q + i][token r16]; the KW wavefronts of a row tile
    // are summed in order by the first
    if constexpr (KW > 1) {
        red[wave][lane] = acc;
        __syncthreads();
        if (kp != 0) return;
#pragma unroll
        for (int j = 1; j < KW; ++j) {
            const floatx4 o = red[rt + RW * j][lane];
            acc[0] += o[0];
            acc[1] += o[1];
            acc[2] += o[2];
            acc[3] += o[3];
        }
    }
    if constexpr (SK == kScaleTensor || SK == kScaleRow) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= 1.0f / scale_at<SK>(p, rbase + 4 * q + i, 0);
    }
    if (r16 < p.M) {
        const size_t o = (size_t)r16 * p.N + rbase + 4 * q;
        if (gridDim.y == 1) {
            Vec<_Float16, 4> h;
#pragma unroll
            for (int i = 0; i < 4; ++i) h.v[i] = from_f32<_Float16>(acc[i]);
            *reinterpret_cast<Vec<_Float16, 4>*>(p.C + o) = h;
        } else {
            *reinterpret_cast<float4*>(p.part + (size_t)blockIdx.y * p.M * p.N + o) =
                float4{acc[0], acc[1], acc[2], acc[3]};
        }
    }
}

// ---- one or two tokens: contiguous row streams -----------------------------------------
// At most kVecMaxTokens tokens the GEMM is a stream of the weight matrix, and the
// shape of that stream decides its speed: measured on MI355X, a wavefront
// reading its own contiguous region 1 KiB per instruction moves a 58.7 MB matrix
// in 10-11 us (5.3-6.0 TB/s), while row tiles read as 256-byte pieces of 16 rows
// 4 KiB apart (the whole-row kernel's shape, every row of the matrix in flight
// at once) take 15-18 us even with no arithmetic.  So wavefront w of W takes rows
// [w*N/W, (w+1)*N/W) -- one contiguous region -- row by row: instruction j of a
// row reads its bytes 1024j .. 1024j+1023, lane l the 16 codes at k = 1024j + 16l
// (lanes past K load the row's first 16 bytes, to stay in bounds, and drop their
// sums: an inf code there times a padding zero would be NaN).  Loads run
// kVecStages instructions ahead through a register ring, unconditionally (past
// the end they repeat the last one), each with the lane's scale.  The token rows
// sit in LDS (zero-padded to whole instructions); each lane decodes its 16 codes
// to binary16 pairs and multiplies them with v_dot2_f32_f16 (exact products,
// fp32 sums), and at each row's end the 64 lane sums are added by a butterfly.
// Scales: per tensor / per row applied to the row's sum, per group (the lane's
// 16 codes lie in one group) to each lane's 16-code sum; reference-mode E5M2
// scales each weight (its exponent-31 codes exceed the binary16 range).
constexpr int kVecMaxTokens = 2;
constexpr int kVecStages = 4;
constexpr int kVecThreads = 512;      // 8 wavefronts per workgroup share the token rows
constexpr int kVecTargetWaves = 2048;
constexpr int kVecMaxTokBytes = 64 * 1024;

// Sum over the wavefront: DPP adds within each row of 16 lanes (xor 1, xor 2, then
// the mirrored quads and halves), then the four row sums read as scalars.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));  // quad_perm 1,0,3,2
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));  // quad_perm 2,3,0,1
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true)); // row_half_mirror
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true)); // row_mirror
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

template <int FMT, int MODE, int SK, int M>
__global__ __launch_bounds__(kVecThreads) void fp8_gemv(SkinnyArgs p, int W, int J) {
    constexpr bool kScaled = !fold_scale<FMT, MODE, SK == kScaleGroupFold ? kScaleRow : SK>();
    extern __shared__ __align__(16) _Float16 tok[];   // [M][J * 1024]
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * (kVecThreads / kWave) + threadIdx.x / kWave));
    const int KP = J * 1024;   // padded row length of the token tile
    // rows split evenly over the W wavefronts (W <= N); the grid's last workgroup
    // may hold wavefronts past W, which get none
    const int r0 = (int)min((long long)p.N, (long long)wave * p.N / W);
    const int r1 = (int)min((long long)p.N, (long long)(wave + 1) * p.N / W);
    const int S = (r1 - r0) * J;
    // instruction (row, j): bytes 1024 j + 16 lane of the row; the fetch cursor runs
    // kVecStages instructions ahead of the compute cursor and stops at the last one
    // (wavefronts past the last row load row N-1's first instruction, unused)
    int f_row = min(r0, p.N - 1), f_j = 0, f_left = S;   // next instruction to load
    auto fetch = [&](u32x4& v, float& sc) __attribute__((always_inline)) {
        const int k = 1024 * f_j + 16 * lane;
        v = *reinterpret_cast<const u32x4*>(p.W + (size_t)f_row * p.K + (k < p.K ? k : 0));
        // vector loads (divergent_zero): as scalar loads, the wait for each
        // instruction's LDS token reads would wait for them too
        if constexpr (SK == kScaleTensor) sc = p.scales[divergent_zero()];
        else if constexpr (SK == kScaleRow) sc = p.scales[f_row + divergent_zero()];
        else sc = p.scales[(size_t)f_row * (size_t)p.groups_per_row + (unsigned)min(k, p.K - 1) / (unsigned)p.gs];
        if (f_left > 1) {   // uniform
            --f_left;
            if (++f_j == J) {
                f_j = 0;
                ++f_row;
            }
        }
    };
    // token rows: loads issued first, then the wavefront's first weight loads (they
    // do not depend on the tokens), then the LDS stores; the barrier waits for the
    // LDS stores only, so the weight loads stay in flight across it
    constexpr int kTokIters = kVecMaxTokBytes / (kVecThreads * 16);
    half8 tv[kTokIters];
#pragma unroll
    for (int it = 0; it < kTokIters; ++it) {
        const int i = (it * kVecThreads + (int)threadIdx.x) * 8;
        const int m = i / KP, k = i - m * KP;
        const bool ok = i < M * KP && k < p.K;
        tv[it] = *reinterpret_cast<const half8*>(reinterpret_cast<const _Float16*>(p.A) +
                                                 (ok ? (size_t)m * p.K + k : 0));
        tv[it] = ok ? tv[it] : half8{};
    }
    u32x4 v[kVecStages];
    float sc[kVecStages];
#pragma unroll
    for (int u = 0; u < kVecStages; ++u) fetch(v[u], sc[u]);
#pragma unroll
    for (int it = 0; it < kTokIters; ++it) {
        const int i = (it * kVecThreads + (int)threadIdx.x) * 8;
        if (i < M * KP) *reinterpret_cast<half8*>(tok + i) = tv[it];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (r0 >= r1) return;   // wavefront-uniform, after the only barrier
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    int c_row = r0, c_j = 0;
    for (int s0 = 0; s0 < S; s0 += kVecStages) {
#pragma unroll
        for (int u = 0; u < kVecStages; ++u) {
            if (s0 + u < S) {   // uniform
                const int k = 1024 * c_j + 16 * lane;
                // v_rcp_f32 (1 ulp) for the per-instruction inverses
                const float inv = kScaled || SK == kScaleGroupFold ? __builtin_amdgcn_rcpf(sc[u]) : 1.0f;
                half8 lo, hi;
                dequant16<FMT, MODE, kScaled>(uint4{v[u][0], v[u][1], v[u][2], v[u][3]}, inv, lo, hi);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const half8 a0 = *reinterpret_cast<const half8*>(tok + m * KP + k);
                    const half8 a1 = *reinterpret_cast<const half8*>(tok + m * KP + k + 8);
                    float part = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        part = __builtin_amdgcn_fdot2(half2v{lo[e], lo[e + 1]}, half2v{a0[e], a0[e + 1]}, part, false);
                        part = __builtin_amdgcn_fdot2(half2v{hi[e], hi[e + 1]}, half2v{a1[e], a1[e + 1]}, part, false);
                    }
                    part = k < p.K ? part : 0.0f;   // past K: padding zeros times codes not of this row's tail
                    if constexpr (SK == kScaleGroupFold && !kScaled) acc[m] = fmaf(part, inv, acc[m]);
                    else acc[m] += part;
                }
                if (++c_j == J) {   // the row's last instruction (uniform)
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        float t = wave_sum_dpp(acc[m]);
                        if constexpr (!kScaled && SK != kScaleGroupFold) t *= 1.0f / sc[u];
                        if (lane == 0) p.C[(size_t)m * p.N + c_row] = from_f32<_Float16>(t);
                        acc[m] = 0.0f;
                    }
                    c_j = 0;
                    ++c_row;
                }
            }
            // refill with the next instruction (the last one repeated past the end)
            fetch(v[u], sc[u]);
        }
    }
}

// ---- host helpers ----------------------------------------------------------------------
bool geom_for(int rows, int cols, int gran, int group_size, Geom& g) {
    if (rows < 0 || cols < 0) return false;
    g.n = (long long)rows * cols;
    if (gran == QL_QUANT_PER_TENSOR) g.gs = g.n > 0 ? g.n : 1;
    else if (gran == QL_QUANT_PER_CHANNEL) g.gs = cols > 0 ? cols : 1;
    else if (gran == QL_QUANT_PER_GROUP && group_size > 0) g.gs = group_size;
    else return false;
    const long long ng = g.n > 0 ? (gran == QL_QUANT_PER_CHANNEL ? rows : (g.n + g.gs - 1) / g.gs) : 0;
    if (ng > 0x7fffffffLL) return false;
    g.n_groups = (int)ng;
    return true;
}

template <int FMT, int MODE>
void launch_quantize_groups(const _Float16* x, const Geom& g, float* s, uint8_t* q, hipStream_t st) {
    const dim3 grid(qlh::blocks_for(g.n / 8, (long long)kQuantIters * kBlock)), block(kBlock);
    switch (g.gs) {
    case 8: hipLaunchKernelGGL((quantize_groups<FMT, MODE, 1>), grid, block, 0, st, x, g, s, q); break;
    case 16: hipLaunchKernelGGL((quantize_groups<FMT, MODE, 2>), grid, block, 0, st, x, g, s, q); break;
    case 32: hipLaunchKernelGGL((quantize_groups<FMT, MODE, 4>), grid, block, 0, st, x, g, s, q); break;
    case 64: hipLaunchKernelGGL((quantize_groups<FMT, MODE, 8>), grid, block, 0, st, x, g, s, q); break;
    case 128: hipLaunchKernelGGL((quantize_groups<FMT, MODE, 16>), grid, block, 0, st, x, g, s, q); break;
    case 256: hipLaunchKernelGGL((quantize_groups<FMT, MODE, 32>), grid, block, 0, st, x, g, s, q); break;
    default: hipLaunchKernelGGL((quantize_groups<FMT, MODE, 64>), grid, block, 0, st, x, g, s, q); break;
    }
}

// q == nullptr: scales only (ql_fp8_scales).  Groups up to 4096 elements: one
// wavefront each; longer ones 2 or 4 wavefronts of 8 vectors a lane.
template <int FMT, int MODE>
void launch_quantize_wave_groups(const _Float16* x, const Geom& g, float* s, uint8_t* q, hipStream_t st) {
    const dim3 grid(qlh::blocks_for(g.n_groups, kBlock / kWave)), block(kBlock);
    const dim3 grid1((unsigned)g.n_groups);
    if (!q) {
        if (g.gs <= 8 * kWave * 8)
            hipLaunchKernelGGL((quantize_wave_groups<FMT, MODE, 8, false>), grid, block, 0, st, x, g, s, q);
        else if (g.gs <= 8 * kWave * 16)
            hipLaunchKernelGGL((quantize_wave_groups<FMT, MODE, 8, false, 2>), grid1, dim3(2 * kWave), 0, st, x, g,
                               s, q);
        else
            hipLaunchKernelGGL((quantize_wave_groups<FMT, MODE, 8, false, 4>), grid1, dim3(4 * kWave), 0, st, x, g,
                               s, q);
    } else if (g.gs <= 8 * kWave * 8) {
        hipLaunchKernelGGL((quantize_wave_groups<FMT, MODE, 8>), grid, block, 0, st, x, g, s, q);
    } else if (g.gs <= 8 * kWave * 16) {
        hipLaunchKernelGGL((quantize_wave_groups<FMT, MODE, 8, true, 2>), grid1, dim3(2 * kWave), 0, st, x, g, s, q);
    } else {
        hipLaunchKernelGGL((quantize_wave_groups<FMT, MODE, 8, true, 4>), grid1, dim3(4 * kWave), 0, st, x, g, s, q);
    }
}

// q == nullptr: scales only (ql_fp8_scales)
template <int FMT, int MODE>
void launch_quantize_segments(const _Float16* x, const Geom& g, float* s, uint8_t* q, hipStream_t st) {
    const int V = (int)(g.gs / 8), P = kWave / V;
    const long long spans = (g.n_groups + P - 1) / P;
    const dim3 grid(qlh::blocks_for(spans, (long long)kQuantIters * (kBlock / kWave))), block(kBlock);
    if (q) hipLaunchKernelGGL((quantize_segments<FMT, MODE, true>), grid, block, 0, st, x, g, V, P, s, q);
    else hipLaunchKernelGGL((quantize_segments<FMT, MODE, false>), grid, block, 0, st, x, g, V, P, s, q);
}

template <int FMT, int MODE>
void launch_quantize(const _Float16* x, const Geom& g, const float* s, uint8_t* q, bool vec,
                     hipStream_t st) {
    if (vec)
        hipLaunchKernelGGL((quantize_kernel<FMT, MODE, true>), dim3(qlh::blocks_for(g.n / 8, kBlock)),
                           dim3(kBlock), 0, st, x, g, s, q);
    else
        hipLaunchKernelGGL((quantize_kernel<FMT, MODE, false>), dim3(qlh::blocks_for(g.n, kBlock)),
                           dim3(kBlock), 0, st, x, g, s, q);
}

template <int FMT, int MODE>
void launch_dequantize(const uint8_t* q, const Geom& g, const float* s, _Float16* y, bool vec,
                       hipStream_t st) {
    if (vec && g.n % 16 == 0 && g.gs % 16 == 0 && qlh::aligned16(q))
        hipLaunchKernelGGL((dequantize16<FMT, MODE>), dim3(qlh::blocks_for(g.n / 16, kBlock)), dim3(kBlock), 0,
                           st, q, g, s, y);
    else if (vec)
        hipLaunchKernelGGL((dequantize_kernel<FMT, MODE, true>), dim3(qlh::blocks_for(g.n / 8, kBlock)),
                           dim3(kBlock), 0, st, q, g, s, y);
    else
        hipLaunchKernelGGL((dequantize_kernel<FMT, MODE, false>), dim3(qlh::blocks_for(g.n, kBlock)),
                           dim3(kBlock), 0, st, q, g, s, y);
}

// Skinny GEMM launch shape: MT token tiles, R = 4 row tiles per workgroup (64
// weight rows: each wavefront streams 64 contiguous rows' 64-byte chunks, and the
// token fragments serve four row tiles) when N allows, and K-splits only while
// there are fewer row blocks than CUs: floor(256 / row blocks), at least two chunks
// per wavefront, and splits*M*N*4 bytes of workspace for the fp32 partials.
// (Measured on MI355X with weights streamed from HBM: one split at 224 row blocks,
// two at 96, four at 64.)
constexpr int kSkinnyTargetWgs = 256;

inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

struct SkinnyPlan {
    int mt, r, splits, chunks_per_split;
    int rw = 0, kw = 0;   // whole-row path: row tiles per workgroup, wavefronts per row tile
};

SkinnyPlan skinny_plan(int M, int N, int K, size_t ws_bytes) {
    SkinnyPlan s;
    s.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
    s.r = 4;
    while (s.r > 1 && (N / 16) % s.r) s.r /= 2;
    const int row_blocks = N / (16 * s.r);
    const int n_chunks = K / 64;
    int splits = row_blocks >= kSkinnyTargetWgs ? 1 : kSkinnyTargetWgs / row_blocks;
    splits = std::min(splits, std::max(1, n_chunks / (2 * kGemmWaves)));
    while (splits > 1 && (size_t)splits * (size_t)M * (size_t)N * sizeof(float) > ws_bytes) --splits;
    s.chunks_per_split = (n_chunks + splits - 1) / splits;
    s.splits = (n_chunks + s.chunks_per_split - 1) / s.chunks_per_split;
    return s;
}

int scale_kind(const Geom& g, int K, const SkinnyPlan& pl, int format, int mode) {
    if (g.n_groups == 1) return kScaleTensor;
    if (g.gs == K) return kScaleRow;
    if (K % g.gs) return kScaleAny;
    // chunk sums need every decoded code in binary16 range (not reference-mode E5M2);
    // with 4 token tiles the 16 multiply-adds per row tile cost more than scaling
    // the 16 weights
    const bool fold = g.gs % 64 == 0 && pl.mt <= 2 && !(format == QL_FP8_E5M2 && mode == QL_FP8_MODE_REFERENCE);
    // the largest group range of a K-split must fit the LDS table
    const int n_chunks = K / 64;
    int ng_max = 0;
    for (int s = 0; s < pl.splits; ++s) {
        const int cb = s * pl.chunks_per_split, ce = std::min(n_chunks, cb + pl.chunks_per_split);
        ng_max = std::max(ng_max, (int)((ce * 64LL - 1) / g.gs + 1 - cb * 64LL / g.gs));
    }
    const int nr = 16 * pl.r, mc = 16 * pl.mt;
    if ((long long)nr * ng_max > skinny_smem_floats(nr, mc, kScaleGroupLds)) return kScaleGroup;
    return fold ? kScaleGroupFold : kScaleGroupLds;
}

template <int FMT, int MODE, int MT, int R>
void launch_skinny_rs(const SkinnyArgs& a, int kind, dim3 grid, hipStream_t st) {
    const dim3 block(kGemmWaves * kWave);
    switch (kind) {
    case kScaleTensor: hipLaunchKernelGGL((fp8_gemm_skinny<FMT, MODE, MT, R, kScaleTensor>), grid, block, 0, st, a); break;
    case kScaleRow: hipLaunchKernelGGL((fp8_gemm_skinny<FMT, MODE, MT, R, kScaleRow>), grid, block, 0, st, a); break;
    case kScaleGroupFold:
        // scale_kind() folds only for up to 2 token tiles and not for reference-mode
        // E5M2; elsewhere the LDS-table kernel, which covers every folded case, runs
        if constexpr (MT <= 2 && !(FMT == QL_FP8_E5M2 && MODE == QL_FP8_MODE_REFERENCE))
            hipLaunchKernelGGL((fp8_gemm_skinny<FMT, MODE, MT, R, kScaleGroupFold>), grid, block, 0, st, a);
        else
            hipLaunchKernelGGL((fp8_gemm_skinny<FMT, MODE, MT, R, kScaleGroupLds>), grid, block, 0, st, a);
        break;
    case kScaleGroupLds: hipLaunchKernelGGL((fp8_gemm_skinny<FMT, MODE, MT, R, kScaleGroupLds>), grid, block, 0, st, a); break;
    case kScaleGroup: hipLaunchKernelGGL((fp8_gemm_skinny<FMT, MODE, MT, R, kScaleGroup>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((fp8_gemm_skinny<FMT, MODE, MT, R, kScaleAny>), grid, block, 0, st, a); break;
    }
}

template <int FMT, int MODE, int MT>
void launch_skinny_mt(const SkinnyArgs& a, const SkinnyPlan& pl, int kind, dim3 grid, hipStream_t st) {
    if (pl.r == 4) launch_skinny_rs<FMT, MODE, MT, 4>(a, kind, grid, st);
    else if (pl.r == 2) launch_skinny_rs<FMT, MODE, MT, 2>(a, kind, grid, st);
    else launch_skinny_rs<FMT, MODE, MT, 1>(a, kind, grid, st);
}

template <int FMT, int MODE>
void launch_skinny(const SkinnyArgs& a, const SkinnyPlan& pl, int kind, hipStream_t st) {
    const dim3 grid((unsigned)(a.N / (16 * pl.r)), (unsigned)pl.splits);
    if (pl.mt == 1) launch_skinny_mt<FMT, MODE, 1>(a, pl, kind, grid, st);
    else if (pl.mt == 2) launch_skinny_mt<FMT, MODE, 2>(a, pl, kind, grid, st);
    else launch_skinny_mt<FMT, MODE, 4>(a, pl, kind, grid, st);
}

// The wide kernel's K-splits: the register plan's split count over 128-k chunks
// (never more splits, so the workspace covers the partials); scale kinds per
// tensor, per row and per group from the LDS table when every split's groups fit.
// Returns the scale kind, or -1 for the register kernel.
int wide_kind(const Geom& g, int K, const SkinnyPlan& pl, int kind, bool fold_ok, int& cps, int& splits) {
    if (pl.mt != 4 || pl.r != 4 || K % kWideChunk) return -1;
    if (kind != kScaleTensor && kind != kScaleRow && kind != kScaleGroupLds) return -1;
    // groups of a multiple of 64 codes: chunk sums of decoded codes, scaled per group
    // (not reference-mode E5M2, whose codes can decode beyond the binary16 range)
    if (kind == kScaleGroupLds && g.gs % 64 == 0 && fold_ok) kind = kScaleGroupFold;
    const int n = K / kWideChunk;
    cps = (n + pl.splits - 1) / pl.splits;
    splits = (n + cps - 1) / cps;
    if (kind >= kScaleGroupFold)
        for (int s = 0; s < splits; ++s) {
            const int cb = s * cps, ce = std::min(n, cb + cps);
            const long long ngs = (ce * (long long)kWideChunk - 1) / g.gs + 1 - cb * (long long)kWideChunk / g.gs;
            if (64 * ngs > kWideTableFloats) return -1;
        }
    return kind;
}

template <int FMT, int MODE>
void launch_wide(const SkinnyArgs& a, int kind, int splits, hipStream_t st) {
    const dim3 grid((unsigned)(a.N / 64), (unsigned)splits), block(kGemmWaves * kWave);
    if (kind == kScaleTensor) hipLaunchKernelGGL((fp8_gemm_wide<FMT, MODE, kScaleTensor>), grid, block, 0, st, a);
    else if (kind == kScaleRow) hipLaunchKernelGGL((fp8_gemm_wide<FMT, MODE, kScaleRow>), grid, block, 0, st, a);
    else if (kind == kScaleGroupLds) hipLaunchKernelGGL((fp8_gemm_wide<FMT, MODE, kScaleGroupLds>), grid, block, 0, st, a);
    else if constexpr (!(FMT == QL_FP8_E5M2 && MODE == QL_FP8_MODE_REFERENCE))
        hipLaunchKernelGGL((fp8_gemm_wide<FMT, MODE, kScaleGroupFold>), grid, block, 0, st, a);
}

// The contiguous-stream kernel's scale kind (kScaleGroupFold: groups folded per
// lane, kScaleGroupLds: reference-mode E5M2 groups, scaled per weight), or -1.
int gemv_kind(const Geom& g, int M, int K, int format, int mode, int& J) {
    J = (K + 1023) / 1024;
    if (M < 1 || M > kVecMaxTokens || K % 16 || (size_t)M * (size_t)J * 1024u * 2u > (size_t)kVecMaxTokBytes)
        return -1;
    if (g.n_groups == 1) return kScaleTensor;
    if (g.gs == K) return kScaleRow;
    if (K % g.gs || g.gs % 16) return -1;
    return format == QL_FP8_E5M2 && mode == QL_FP8_MODE_REFERENCE ? kScaleGroupLds : kScaleGroupFold;
}

template <int FMT, int MODE, int SK>
void launch_gemv_sk(const SkinnyArgs& a, int J, hipStream_t st) {
    const int waves = std::min(a.N, kVecTargetWaves);
    const dim3 grid((unsigned)((waves + kVecThreads / kWave - 1) / (kVecThreads / kWave))), block(kVecThreads);
    const size_t lds = (size_t)a.M * (size_t)J * 1024u * sizeof(_Float16);
    if (a.M == 1) hipLaunchKernelGGL((fp8_gemv<FMT, MODE, SK, 1>), grid, block, lds, st, a, waves, J);
    else hipLaunchKernelGGL((fp8_gemv<FMT, MODE, SK, 2>), grid, block, lds, st, a, waves, J);
}

// (gemv_kind gives groups kScaleGroupLds exactly for reference-mode E5M2, so each
// format/mode pair instantiates one group kind)
template <int FMT, int MODE>
void launch_gemv(const SkinnyArgs& a, int kind, int J, hipStream_t st) {
    if (kind == kScaleTensor) launch_gemv_sk<FMT, MODE, kScaleTensor>(a, J, st);
    else if (kind == kScaleRow) launch_gemv_sk<FMT, MODE, kScaleRow>(a, J, st);
    else if constexpr (FMT == QL_FP8_E5M2 && MODE == QL_FP8_MODE_REFERENCE)
        launch_gemv_sk<FMT, MODE, kScaleGroupLds>(a, J, st);
    else
        launch_gemv_sk<FMT, MODE, kScaleGroupFold>(a, J, st);
}

// Whole-row path for one token tile: chunks of 256 codes, scales per tensor, per
// row or per group of a multiple of 64 codes dividing K (the group table of a split
// must fit LDS).  It multiplies decoded codes and scales the sums, so
// reference-mode E5M2 (whose exponent-31 codes decode beyond the binary16 range)
// stays on the register path.
int rows_kind(const Geom& g, int M, int N, int K, int format, int mode) {
    if (M > kRowsMaxTokens || N % 16 || K % kRowsChunk || (format == QL_FP8_E5M2 && mode == QL_FP8_MODE_REFERENCE) ||
        (uint64_t)(M + 1) * (uint64_t)K * 2u >= (1ull << 32))
        return -1;
    if (g.n_groups == 1) return kScaleTensor;
    if (g.gs == K) return kScaleRow;
    if (K % g.gs || g.gs % 64) return -1;
    return kScaleGroupFold;
}

// Shape of the whole-row launch: KW (wavefronts sharing a row tile, splitting its
// chunks) is the largest of 1, 2, 4, 8 that keeps N/16 * KW wavefronts within
// max_waves and gives every wavefront at least a ring of chunks; RW = 4 / KW row
// tiles per workgroup (1 for KW >= 4), lowered until N divides.  K-splits over
// launches (fp32 partials + splitk_reduce) only when KW = 8 leaves the chip
// short of wavefronts.  Measured on MI355X with weights streamed from HBM:
// about 1024 wavefronts suit the OCP decode, about 2048 the reference-mode decode
// (its check of every code needs more wavefronts to hide).
SkinnyPlan rows_plan(int M, int N, int K, int mode, size_t ws_bytes) {
    const int max_waves = mode == QL_FP8_MODE_REFERENCE ? kRowsRefWaves : kRowsOcpWaves;
    SkinnyPlan s;
    const int tiles = N / 16;
    const int n_chunks = K / kRowsChunk;
    s.kw = 1;
    while (s.kw < 8 && tiles * 2 * s.kw <= max_waves && n_chunks / (2 * s.kw) >= kRowsStages) s.kw *= 2;
    s.rw = s.kw >= 4 ? 1 : 4 / s.kw;
    while (tiles % s.rw) s.rw /= 2;
    s.mt = 1;
    s.r = s.rw;
    int splits = 1;
    if (s.kw == 8 && tiles * 16 <= max_waves)
        splits = std::min(max_waves / (tiles * 8), std::max(1, n_chunks / (8 * kRowsStages)));
    while (splits > 1 && (size_t)splits * (size_t)M * (size_t)N * sizeof(float) > ws_bytes) --splits;
    s.chunks_per_split = (n_chunks + splits - 1) / splits;
    s.splits = (n_chunks + s.chunks_per_split - 1) / s.chunks_per_split;
    return s;
}

// largest number of scale groups one K-split of the plan touches
int rows_groups_per_split(const SkinnyPlan& pl, int K, long long gs) {
    const int n_chunks = K / kRowsChunk;
    int ng_max = 0;
    for (int s = 0; s < pl.splits; ++s) {
        const int cb = s * pl.chunks_per_split, ce = std::min(n_chunks, cb + pl.chunks_per_split);
        ng_max = std::max(ng_max, (int)((ce * (long long)kRowsChunk - 1) / gs + 1 - cb * (long long)kRowsChunk / gs));
    }
    return ng_max;
}

template <int FMT, int MODE, int RW, int KW>
void launch_rows_shape(const SkinnyArgs& a, const SkinnyPlan& pl, int kind, hipStream_t st) {
    const dim3 grid((unsigned)(a.N / (16 * RW)), (unsigned)pl.splits), block(RW * KW * kWave);
    if (kind == kScaleTensor) hipLaunchKernelGGL((fp8_gemm_rows<FMT, MODE, kScaleTensor, RW, KW>), grid, block, 0, st, a);
    else if (kind == kScaleRow) hipLaunchKernelGGL((fp8_gemm_rows<FMT, MODE, kScaleRow, RW, KW>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((fp8_gemm_rows<FMT, MODE, kScaleGroupFold, RW, KW>), grid, block, 0, st, a);
}

template <int FMT, int MODE>
void launch_rows(const SkinnyArgs& a, const SkinnyPlan& pl, int kind, hipStream_t st) {
    if (pl.kw == 8) launch_rows_shape<FMT, MODE, 1, 8>(a, pl, kind, st);
    else if (pl.kw == 4) launch_rows_shape<FMT, MODE, 1, 4>(a, pl, kind, st);
    else if (pl.kw == 2 && pl.rw == 2) launch_rows_shape<FMT, MODE, 2, 2>(a, pl, kind, st);
    else if (pl.kw == 2) launch_rows_shape<FMT, MODE, 1, 2>(a, pl, kind, st);
    else if (pl.rw == 4) launch_rows_shape<FMT, MODE, 4, 1>(a, pl, kind, st);
    else if (pl.rw == 2) launch_rows_shape<FMT, MODE, 2, 1>(a, pl, kind, st);
    else launch_rows_shape<FMT, MODE, 1, 1>(a, pl, kind, st);
}

// the register path addresses W and A with 32-bit byte offsets
bool skinny_ok(int M, int N, int K, const Geom& g) {
    return M <= 64 && N % 16 == 0 && K % 64 == 0 && g.gs % 16 == 0 && (uint64_t)N * (uint64_t)K < (1ull << 32) &&
           (uint64_t)M * (uint64_t)K * 2u < (1ull << 32);
}

#define QL_FP8_DISPATCH(fmt, mode, FN, ...)                                                   \
    do {                                                                                      \
        if (fmt == QL_FP8_E4M3 && mode == QL_FP8_MODE_REFERENCE)                              \
            FN<QL_FP8_E4M3, QL_FP8_MODE_REFERENCE>(__VA_ARGS__);                              \
        else if (fmt == QL_FP8_E4M3)                                                          \
            FN<QL_FP8_E4M3, QL_FP8_MODE_OCP>(__VA_ARGS__);                                    \
        else if (mode == QL_FP8_MODE_REFERENCE)                                               \
            FN<QL_FP8_E5M2, QL_FP8_MODE_REFERENCE>(__VA_ARGS__);                              \
        else                                                                                  \
            FN<QL_FP8_E5M2, QL_FP8_MODE_OCP>(__VA_ARGS__);                                    \
    } while (0)

bool fmt_mode_ok(int fmt, int mode) {
    return (fmt == QL_FP8_E4M3 || fmt == QL_FP8_E5M2) &&
           (mode == QL_FP8_MODE_REFERENCE || mode == QL_FP8_MODE_OCP);
}

// decoding entries also take QL_FP8_MODE_REFERENCE_CLEAN: codes without any of the
// codes whose reference decode differs decode to the same values with the OCP
// decode (up to the sign of zero for 0x80, which no product or sum sees)
bool decode_mode_ok(int fmt, int mode) {
    return fmt_mode_ok(fmt, mode) || ((fmt == QL_FP8_E4M3 || fmt == QL_FP8_E5M2) && mode == QL_FP8_MODE_REFERENCE_CLEAN);
}
int decode_mode(int mode) { return mode == QL_FP8_MODE_REFERENCE_CLEAN ? QL_FP8_MODE_OCP : mode; }

// number of codes (16 per thread per step) whose reference decode differs from the
// OCP decode; one 64-bit atomic add per wavefront
template <int FMT>
__global__ __launch_bounds__(kBlock) void count_ref_special(const uint8_t* __restrict__ q, size_t n,
                                                           unsigned long long* __restrict__ count) {
    const size_t n16 = n / 16;
    const size_t stride = (size_t)gridDim.x * kBlock;
    unsigned c = 0;
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n16; i += stride) {
        const uint4 v = reinterpret_cast<const uint4*>(q)[i];
        c += __popc(ref_special<FMT>(v.x) & 0x80808080u) + __popc(ref_special<FMT>(v.y) & 0x80808080u) +
             __popc(ref_special<FMT>(v.z) & 0x80808080u) + __popc(ref_special<FMT>(v.w) & 0x80808080u);
    }
    if (blockIdx.x == 0 && threadIdx.x < n - 16 * n16)   // the last n % 16 codes
        c += __popc(ref_special<FMT>(q[16 * n16 + threadIdx.x]) & 0x80u);
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) c += __shfl_xor(c, o, kWave);
    if ((threadIdx.x & (kWave - 1)) == 0 && c) atomicAdd(count, (unsigned long long)c);
}

__global__ void clear_u64(unsigned long long* p) { *p = 0; }

}  // namespace

extern "C" hipError_t ql_fp8_num_scales(int rows, int cols, int granularity, int group_size,
                                        int* n_scales) {
    Geom g;
    QL_CHECK_ARG(n_scales && geom_for(rows, cols, granularity, group_size, g));
    *n_scales = g.n_groups;
    return hipSuccess;
}

extern "C" hipError_t ql_fp8_scales(const uint16_t* src, int rows, int cols, int format,
                                    int granularity, int group_size, int mode, float* scales,
                                    hipStream_t stream) {
    Geom g;
    QL_CHECK_ARG(fmt_mode_ok(format, mode) && geom_for(rows, cols, granularity, group_size, g));
    if (g.n == 0) return hipSuccess;
    QL_CHECK_ARG(src && scales);
    const _Float16* x = reinterpret_cast<const _Float16*>(src);
    const unsigned sblocks = qlh::blocks_for(g.n_groups, kBlock);
    const bool vec = g.n % 8 == 0 && qlh::aligned16(src);
    if (vec && (g.gs == 8 || g.gs == 16 || g.gs == 32 || g.gs == 64 || g.gs == 128 || g.gs == 256 || g.gs == 512)) {
        const unsigned blocks = qlh::blocks_for(g.n / 8, (long long)kAbsIters * kBlock);
        switch (g.gs) {
        case 8: hipLaunchKernelGGL(absmax_vec<1>, dim3(blocks), dim3(kBlock), 0, stream, x, g, mode, scales); break;
        case 16: hipLaunchKernelGGL(absmax_vec<2>, dim3(blocks), dim3(kBlock), 0, stream, x, g, mode, scales); break;
        case 32: hipLaunchKernelGGL(absmax_vec<4>, dim3(blocks), dim3(kBlock), 0, stream, x, g, mode, scales); break;
        case 64: hipLaunchKernelGGL(absmax_vec<8>, dim3(blocks), dim3(kBlock), 0, stream, x, g, mode, scales); break;
        case 128: hipLaunchKernelGGL(absmax_vec<16>, dim3(blocks), dim3(kBlock), 0, stream, x, g, mode, scales); break;
        case 256: hipLaunchKernelGGL(absmax_vec<32>, dim3(blocks), dim3(kBlock), 0, stream, x, g, mode, scales); break;
        default: hipLaunchKernelGGL(absmax_vec<64>, dim3(blocks), dim3(kBlock), 0, stream, x, g, mode, scales); break;
        }
    } else if (vec && g.gs % 8 == 0 && g.gs < 8 * 32) {
        // several short groups per wavefront; it writes the final scales itself
        QL_FP8_DISPATCH(format, mode, launch_quantize_segments, x, g, scales, nullptr, stream);
        return hipGetLastError();
    } else if (vec && g.gs % 8 == 0 && g.gs <= 8LL * kWave * kWaveGroupVecs) {
        // one wavefront per group in registers; it writes the final scales itself
        QL_FP8_DISPATCH(format, mode, launch_quantize_wave_groups, x, g, scales, nullptr, stream);
        return hipGetLastError();
    } else if (g.gs <= 64 && g.gs % 8) {
        hipLaunchKernelGGL(absmax_thread, dim3(sblocks), dim3(kBlock), 0, stream, x, g, mode, fp8_max(format),
                           scales);
        return hipGetLastError();
    } else if (g.gs <= 8192) {
        hipLaunchKernelGGL(absmax_wave, dim3(qlh::blocks_for(g.n_groups, kBlock / kWave)), dim3(kBlock),
                           0, stream, x, g, mode, scales);
    } else {
        hipLaunchKernelGGL(fill_zero, dim3(sblocks), dim3(kBlock), 0, stream, scales, g.n_groups);
        if (vec && g.gs % 8 == 0) {
            // workgroups of one group end in atomics on one address, which serialize:
            // at most kAbsBlocks workgroups in all, each looping over its share
            const long long want = qlh::blocks_for(seen_vectors(mode, g.gs / 8), (long long)kBlock * kBlockIters);
            const unsigned bx = (unsigned)std::max(1LL, std::min(want, kAbsBlocks / g.n_groups));
            hipLaunchKernelGGL(absmax_blocks_vec<false>, group_grid(bx, g.n_groups), dim3(kBlock), 0, stream, x,
                               g, mode, scales);
        } else {
            const long long per = 16LL * kBlock;
            unsigned bx = (unsigned)((g.gs + per - 1) / per);
            if (bx > 1024) bx = 1024;
            hipLaunchKernelGGL(absmax_blocks, group_grid(bx, g.n_groups), dim3(kBlock), 0, stream, x, g,
                               mode, scales);
        }
    }
    hipLaunchKernelGGL(finalize_scales, dim3(sblocks), dim3(kBlock), 0, stream, scales, g.n_groups,
                       fp8_max(format));
    return hipGetLastError();
}

extern "C" hipError_t ql_fp8_quantize(const uint16_t* src, int rows, int cols, int format,
                                      int granularity, int group_size, int mode, uint8_t* dst,
                                      float* scales, hipStream_t stream) {
    Geom g;
    QL_CHECK_ARG(fmt_mode_ok(format, mode) && geom_for(rows, cols, granularity, group_size, g));
    if (g.n == 0) return hipSuccess;
    QL_CHECK_ARG(dst);
    if (src && scales && g.n % 8 == 0 && qlh::aligned16(src) && ((uintptr_t)dst & 7) == 0 && g.gs >= 8 &&
        g.gs <= 512 && (g.gs & (g.gs - 1)) == 0) {   // one pass: scales and codes together
        QL_FP8_DISPATCH(format, mode, launch_quantize_groups, reinterpret_cast<const _Float16*>(src), g, scales,
                        dst, stream);
        return hipGetLastError();
    }
    if (src && scales && g.n % 8 == 0 && g.gs % 8 == 0 && g.gs < 8 * 32 && qlh::aligned16(src) &&
        ((uintptr_t)dst & 7) == 0) {   // several short groups per wavefront, one pass
        QL_FP8_DISPATCH(format, mode, launch_quantize_segments, reinterpret_cast<const _Float16*>(src), g, scales,
                        dst, stream);
        return hipGetLastError();
    }
    if (src && scales && g.n % 8 == 0 && g.gs % 8 == 0 && g.gs <= 8LL * kWave * kWaveGroupVecs &&
        qlh::aligned16(src) && ((uintptr_t)dst & 7) == 0) {   // one wavefront per group, one pass
        QL_FP8_DISPATCH(format, mode, launch_quantize_wave_groups, reinterpret_cast<const _Float16*>(src), g,
                        scales, dst, stream);
        return hipGetLastError();
    }
    if (src && scales && g.n % 8 == 0 && g.gs % 8 == 0 && g.gs > 8LL * kWave * kWaveGroupVecs &&
        qlh::aligned16(src) && ((uintptr_t)dst & 7) == 0) {
        // groups too large for one wavefront (per tensor): the workgroups' maxima go to
        // the front of dst (at most kAbsBlocks floats, or one per group; n > 16384
        // bytes), one workgroup per group reduces them into the scale, then the codes
        // overwrite them
        const long long want =
            qlh::blocks_for(seen_vectors(mode, g.gs / 8), (long long)kBlock * kBlockIters);
        const unsigned bx = (unsigned)std::max(1LL, std::min(want, kAbsBlocks / g.n_groups));
        float* part = reinterpret_cast<float*>(dst);
        hipLaunchKernelGGL(absmax_blocks_vec<true>, group_grid(bx, g.n_groups), dim3(kBlock), 0, stream,
                           reinterpret_cast<const _Float16*>(src), g, mode, part);
        hipLaunchKernelGGL(reduce_partials, dim3((unsigned)g.n_groups), dim3(kBlock), 0, stream, part, (int)bx,
                           fp8_max(format), scales);
        QL_FP8_DISPATCH(format, mode, launch_quantize, reinterpret_cast<const _Float16*>(src), g, scales, dst,
                        true, stream);
        return hipGetLastError();
    }
    const hipError_t e = ql_fp8_scales(src, rows, cols, format, granularity, group_size, mode, scales, stream);
    if (e != hipSuccess) return e;
    const bool vec = g.n % 8 == 0 && qlh::aligned16(src) && ((uintptr_t)dst & 7) == 0;
    QL_FP8_DISPATCH(format, mode, launch_quantize, reinterpret_cast<const _Float16*>(src), g, scales,
                    dst, vec, stream);
    return hipGetLastError();
}

extern "C" hipError_t ql_fp8_dequantize(const uint8_t* src, const float* scales, int rows, int cols,
                                        int format, int granularity, int group_size, int mode,
                                        uint16_t* dst, hipStream_t stream) {
    Geom g;
    QL_CHECK_ARG(decode_mode_ok(format, mode) && geom_for(rows, cols, granularity, group_size, g));
    if (g.n == 0) return hipSuccess;
    QL_CHECK_ARG(src && scales && dst);
    // the reference's decoder throughout (its +0 for code 0x80 included): cheap here
    if (mode == QL_FP8_MODE_REFERENCE_CLEAN) mode = QL_FP8_MODE_REFERENCE;
    const bool vec = g.n % 8 == 0 && qlh::aligned16(dst) && ((uintptr_t)src & 7) == 0;
    QL_FP8_DISPATCH(format, mode, launch_dequantize, src, g, scales, reinterpret_cast<_Float16*>(dst),
                    vec, stream);
    return hipGetLastError();
}

extern "C" hipError_t ql_fp8_gemm_workspace_size(int M, int N, int K, int granularity, int group_size,
                                                 size_t* bytes) {
    Geom g;
    QL_CHECK_ARG(bytes && M >= 0 && N >= 0 && K >= 0 && geom_for(N, K, granularity, group_size, g));
    *bytes = 0;
    if (M == 0 || N == 0 || K == 0) return hipSuccess;
    if (skinny_ok(M, N, K, g)) {
        // the format and mode only narrow the whole-row path's group case; the
        // reservation covers either path
        const SkinnyPlan pl = skinny_plan(M, N, K, SIZE_MAX);
        size_t splits = (size_t)pl.splits;
        if (rows_kind(g, M, N, K, QL_FP8_E4M3, QL_FP8_MODE_OCP) >= 0)
            for (int mode : {QL_FP8_MODE_REFERENCE, QL_FP8_MODE_OCP})
                splits = std::max(splits, (size_t)rows_plan(M, N, K, mode, SIZE_MAX).splits);
        *bytes = splits > 1 ? splits * (size_t)M * (size_t)N * sizeof(float) : 0;
        if (pl.mt == 4) *bytes = align256(*bytes) + packed_a_bytes(K, pl.mt);   // fragment-major tokens
    } else {
        *bytes = (size_t)N * (size_t)K * sizeof(uint16_t);
    }
    return hipSuccess;
}

extern "C" hipError_t ql_fp8_gemm_f16(const uint16_t* A, const uint8_t* W, const float* scales,
                                      int M, int N, int K, int format, int granularity,
                                      int group_size, int mode, uint16_t* C, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream) {
    Geom g;
    QL_CHECK_ARG(decode_mode_ok(format, mode) && M >= 0 && N >= 0 && K >= 0);
    QL_CHECK_ARG(geom_for(N, K, granularity, group_size, g));
    if (M == 0 || N == 0) return hipSuccess;
    QL_CHECK_ARG(A && W && scales && C && K > 0);
    mode = decode_mode(mode);
    int gemv_j = 0;
    const int gkind = gemv_kind(g, M, K, format, mode, gemv_j);
    if (gkind >= 0 && qlh::aligned16(A) && qlh::aligned16(W)) {
        SkinnyArgs a{};
        a.A = reinterpret_cast<const char*>(A);
        a.W = reinterpret_cast<const char*>(W);
        a.scales = scales;
        a.C = reinterpret_cast<_Float16*>(C);
        a.M = M;
        a.N = N;
        a.K = K;
        a.gs = g.gs;
        a.groups_per_row = K % g.gs == 0 ? (int)(K / g.gs) : 0;
        QL_FP8_DISPATCH(format, mode, launch_gemv, a, gkind, gemv_j, stream);
        return hipGetLastError();
    }
    if (skinny_ok(M, N, K, g) && qlh::aligned16(A) && qlh::aligned16(W)) {
        const bool ws_ok = workspace && qlh::aligned16(workspace) && ((uintptr_t)C & 7) == 0;
        const size_t ws = ws_ok ? workspace_bytes : 0;
        int rkind = rows_kind(g, M, N, K, format, mode);
        SkinnyPlan pl = rkind >= 0 ? rows_plan(M, N, K, mode, ws) : skinny_plan(M, N, K, ws);
        if (rkind == kScaleGroupFold && 16LL * pl.rw * rows_groups_per_split(pl, K, g.gs) > kRowsTableFloats) {
            rkind = -1;
            pl = skinny_plan(M, N, K, ws);
        }
        // more than 32 tokens (four token tiles) on the register path: the token
        // rows are copied fragment-major after the split partials, when the
        // workspace holds both, and the whole-line kernel reads them where it
        // applies.  Measured on MI355X, weights streamed from HBM, 64 rows x
        // gate/up (14336 x 4096) / down (4096 x 14336), us per call: register
        // kernel on row-major tokens 35.2 / 34.9 (E4M3 groups of 128, codes
        // checked clean) and 32.8 / 32.6 (per channel, OCP); with the copy
        // 31.3 / 32.9 and 28.1 / 31.5; whole-line kernel 26.1 / 28.9 and
        // 24.9 / 28.5 (the fp16 library GEMM: 26.5 / 29.7).  At 32 rows the
        // copy's launch cost more than it saved (+3-4%).
        const size_t part_bytes = pl.splits > 1 ? (size_t)pl.splits * (size_t)M * (size_t)N * sizeof(float) : 0;
        const bool pack_fits = rkind < 0 && pl.mt == 4 && ws_ok &&
                               align256(part_bytes) + packed_a_bytes(K, pl.mt) <= workspace_bytes;
        // the whole-line kernel where it applies, reading the token rows itself or
        // (wide_token_stages 0) the copy; else the register kernel, on the copy when
        // the workspace holds it
        int kind = -1, wk = -1, cps = 0, wsplits = 0;
        if (rkind < 0) {
            kind = scale_kind(g, K, pl, format, mode);
            const bool fold_ok = !(format == QL_FP8_E5M2 && mode == QL_FP8_MODE_REFERENCE);
            wk = wide_kind(g, K, pl, kind, fold_ok, cps, wsplits);
            if (wk >= 0 && wide_token_stages(mode, wk) == 0 && !pack_fits) wk = -1;
        }
        const bool pack = pack_fits && (wk < 0 || wide_token_stages(mode, wk) == 0);
        SkinnyArgs a;
        a.A = reinterpret_cast<const char*>(A);
        a.packed_a = 0;
        if (pack) {
            char* pa = static_cast<char*>(workspace) + align256(part_bytes);
            const long long slots = (long long)(K / 64) * pl.mt * 2 * kWave;
            hipLaunchKernelGGL(pack_tokens, dim3(qlh::blocks_for(slots, kBlock)), dim3(kBlock), 0, stream,
                               reinterpret_cast<const _Float16*>(A), reinterpret_cast<uint4*>(pa), M, K, pl.mt);
            a.A = pa;
            a.packed_a = 1;
        }
        a.W = reinterpret_cast<const char*>(W);
        a.scales = scales;
        a.C = reinterpret_cast<_Float16*>(C);
        a.part = static_cast<float*>(workspace);
        a.M = M;
        a.N = N;
        a.K = K;
        a.chunks_per_split = pl.chunks_per_split;
        a.gs = g.gs;
        a.groups_per_row = K % g.gs == 0 ? (int)(K / g.gs) : 0;
        a.g_step = (int)(256 / g.gs);
        a.r_step = (int)(256 % g.gs);
        if (rkind >= 0) {
            // rows_kind() keeps reference-mode E5M2 on the register path
            if (format == QL_FP8_E4M3 && mode == QL_FP8_MODE_REFERENCE)
                launch_rows<QL_FP8_E4M3, QL_FP8_MODE_REFERENCE>(a, pl, rkind, stream);
            else if (format == QL_FP8_E4M3)
                launch_rows<QL_FP8_E4M3, QL_FP8_MODE_OCP>(a, pl, rkind, stream);
            else if (mode == QL_FP8_MODE_OCP)
                launch_rows<QL_FP8_E5M2, QL_FP8_MODE_OCP>(a, pl, rkind, stream);
            else
                return hipErrorInvalidValue;
        } else {
            if (wk >= 0) {
                a.chunks_per_split = cps;
                pl.splits = wsplits;
                QL_FP8_DISPATCH(format, mode, launch_wide, a, wk, wsplits, stream);
            } else
                QL_FP8_DISPATCH(format, mode, launch_skinny, a, pl, kind, stream);
        }
        if (pl.splits > 1) {
            const long long mn = (long long)M * N;
            hipLaunchKernelGGL(splitk_reduce, dim3(qlh::blocks_for(mn / 4, kBlock)), dim3(kBlock), 0, stream,
                               a.part, a.C, pl.splits, mn);
        }
        return hipGetLastError();
    }
    // dequantize into the workspace, then the fp16 library GEMM
    const size_t need = (size_t)N * (size_t)K * sizeof(uint16_t);
    QL_CHECK_ARG(workspace && workspace_bytes >= need && qlh::aligned16(workspace));
    uint16_t* wf = static_cast<uint16_t*>(workspace);
    const hipError_t e = ql_fp8_dequantize(W, scales, N, K, format, granularity, group_size, mode, wf, stream);
    if (e != hipSuccess) return e;
    return ql_gemm_f16(A, wf, C, M, N, K, stream);
}

extern "C" hipError_t ql_fp8_count_ref_special(const uint8_t* codes, size_t n, int format,
                                               unsigned long long* count, hipStream_t stream) {
    QL_CHECK_ARG((format == QL_FP8_E4M3 || format == QL_FP8_E5M2) && count);
    QL_CHECK_ARG(n == 0 || (codes && qlh::aligned16(codes)));
    hipLaunchKernelGGL(clear_u64, dim3(1), dim3(1), 0, stream, count);
    if (n == 0) return hipGetLastError();
    const unsigned blocks = (unsigned)std::max<size_t>(1, std::min<size_t>(2048, (n / 16 + kBlock - 1) / kBlock));
    if (format == QL_FP8_E4M3)
        hipLaunchKernelGGL(count_ref_special<QL_FP8_E4M3>, dim3(blocks), dim3(kBlock), 0, stream, codes, n, count);
    else
        hipLaunchKernelGGL(count_ref_special<QL_FP8_E5M2>, dim3(blocks), dim3(kBlock), 0, stream, codes, n, count);
    return hipGetLastError();
}
