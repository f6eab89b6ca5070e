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
// GEMM (quantlib_src/kernels/fp8_gemm.cu:34-139): C[M,N] = A[M,K] W'[N,K]^T with
// W' the dequantized weights in binary16 and fp32 accumulation.  For few rows
// (decode, M <= 64) the weights are streamed once, dequantized in registers and
// fed to v_mfma_f32_16x16x32_f16 (C^T = W' A^T: 16 weight rows x up to 64 tokens
// per workgroup, K split over its 4 wavefronts and summed in LDS); the in-register
// dequant multiplies by 1/scale.  Larger M dequantizes into a workspace with the
// codec and runs the fp16 library GEMM.
#include "ql_common.hpp"
#include "quantlib_amd.h"

#include <math.h>
#include <float.h>

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

template <int FMT>
__device__ __forceinline__ float2v dec_ocp2(uint32_t w) {   // the two low bytes of w
    if constexpr (FMT == QL_FP8_E4M3)
        return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    else
        return __builtin_amdgcn_cvt_pk_f32_bf8((int)w, false);
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

// large groups: blocks stride their group and combine with an atomic max on the
// bit pattern (non-negative floats order like their bits); mx pre-zeroed
__global__ __launch_bounds__(kBlock) void absmax_blocks(const _Float16* __restrict__ x, Geom g,
                                                        int mode, float* __restrict__ mx) {
    const long long grp = blockIdx.y;
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
// VEC: 8 elements per thread (n % 8 == 0, gs % 8 == 0, aligned); else one element.
template <int FMT, int MODE, bool VEC>
__global__ __launch_bounds__(kBlock) void quantize_kernel(const _Float16* __restrict__ x, Geom g,
                                                          const float* __restrict__ scales,
                                                          uint8_t* __restrict__ q) {
    const long long t = (long long)blockIdx.x * kBlock + threadIdx.x;
    if constexpr (VEC) {
        if (t * 8 >= g.n) return;
        const Vec<_Float16, 8> v = load<true>(reinterpret_cast<const Vec<_Float16, 8>*>(x) + t);
        const float s = scales[(t * 8) / g.gs];
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float f[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = (float)v.v[4 * h + e] * s;
            if constexpr (MODE == QL_FP8_MODE_REFERENCE) {
                w[h] = enc_ref<FMT>(f[0]) | (enc_ref<FMT>(f[1]) << 8) | (enc_ref<FMT>(f[2]) << 16) |
                       (enc_ref<FMT>(f[3]) << 24);
            } else {
                w[h] = enc_ocp2<FMT>(f[0], f[1]) | (enc_ocp2<FMT>(f[2], f[3]) << 16);
            }
        }
        store<true>(reinterpret_cast<u32x2*>(q) + t, u32x2{w[0], w[1]});
    } else {
        if (t >= g.n) return;
        const float f = (float)x[t] * scales[t / g.gs];
        q[t] = (uint8_t)(MODE == QL_FP8_MODE_REFERENCE ? enc_ref<FMT>(f) : (enc_ocp2<FMT>(f, 0.0f) & 0xFFu));
    }
}

template <int FMT, int MODE>
__device__ __forceinline__ float decode1(uint32_t q) {
    if constexpr (MODE == QL_FP8_MODE_REFERENCE) return dec_ref<FMT>(q);
    else return dec_ocp2<FMT>(q)[0];
}

template <int FMT, int MODE, bool VEC>
__global__ __launch_bounds__(kBlock) void dequantize_kernel(const uint8_t* __restrict__ q, Geom g,
                                                            const float* __restrict__ scales,
                                                            _Float16* __restrict__ y) {
    const long long t = (long long)blockIdx.x * kBlock + threadIdx.x;
    if constexpr (VEC) {
        if (t * 8 >= g.n) return;
        const u32x2 w = load<true>(reinterpret_cast<const u32x2*>(q) + t);
        const float s = scales[(t * 8) / g.gs];
        Vec<_Float16, 8> out;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t code = (w[e >> 2] >> (8 * (e & 3))) & 0xFFu;
            out.v[e] = from_f32<_Float16>(decode1<FMT, MODE>(code) / s);
        }
        store<true>(reinterpret_cast<Vec<_Float16, 8>*>(y) + t, out);
    } else {
        if (t >= g.n) return;
        y[t] = from_f32<_Float16>(decode1<FMT, MODE>(q[t]) / scales[t / g.gs]);
    }
}

// ---- skinny GEMM: C[M,N] = A[M,K] (dequant W[N,K])^T, M <= 64 --------------------------
// Workgroup: 16 weight rows (n), all M tokens; wavefront w sums K-range w of 4.
// Per 64-k chunk a lane holds 16 codes of row n0 + lane%16 at k = 16*(lane/16) ..,
// used as the A operand of two 16x16x32 steps (k order permuted identically in
// the B operand: token rows A[m][same k]).
constexpr int kGemmWaves = 4;

template <int FMT, int MODE>
__device__ __forceinline__ void dequant16(uint4 codes, float inv, half8& lo, half8& hi) {
    const uint32_t w[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float f[4];
        if constexpr (MODE == QL_FP8_MODE_REFERENCE) {
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = dec_ref<FMT>((w[j] >> (8 * e)) & 0xFFu);
        } else {
            const float2v a = dec_ocp2<FMT>(w[j]);
            const float2v b = dec_ocp2<FMT>(w[j] >> 16);
            f[0] = a[0];
            f[1] = a[1];
            f[2] = b[0];
            f[3] = b[1];
        }
        half8& dst = j < 2 ? lo : hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[4 * (j & 1) + e] = from_f32<_Float16>(f[e] * inv);
    }
}

template <int FMT, int MODE, int MT>
__global__ __launch_bounds__(kGemmWaves * kWave) void fp8_gemm_skinny(
    const _Float16* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ scales,
    _Float16* __restrict__ C, int M, int N, int K, long long gs) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * 16;
    const int row = n0 + (lane & 15);             // weight row this lane loads
    const int kq = lane >> 4;                     // which 16-k slice of a 64-k chunk
    const int n_chunks = K / 64;
    const int per = (n_chunks + kGemmWaves - 1) / kGemmWaves;
    const int c_begin = wave * per, c_end = min(n_chunks, c_begin + per);
    floatx4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = floatx4{};
    const uint8_t* wrow = W + (size_t)row * K;
    const long long wbase = (long long)row * K;
    for (int c = c_begin; c < c_end; ++c) {
        const int k = c * 64 + 16 * kq;
        const uint4 codes = *reinterpret_cast<const uint4*>(wrow + k);
        const float inv = 1.0f / scales[(wbase + k) / gs];
        half8 wlo, whi;
        dequant16<FMT, MODE>(codes, inv, wlo, whi);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int m = 16 * t + (lane & 15);
            const _Float16* arow = A + (size_t)(m < M ? m : 0) * K + k;
            half8 alo = *reinterpret_cast<const half8*>(arow);
            half8 ahi = *reinterpret_cast<const half8*>(arow + 8);
            if (m >= M) {
                alo = half8{};
                ahi = half8{};
            }
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wlo, alo, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(whi, ahi, acc[t], 0, 0, 0);
        }
    }
    // sum the wavefronts' partial C^T tiles: lane holds C^T[n0 + 4*(lane/16) + i][16t + lane%16]
    __shared__ float part[kGemmWaves][MT * 16][17];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave][16 * t + (lane & 15)][4 * (lane >> 4) + i] = acc[t][i];
    __syncthreads();
    for (int e = threadIdx.x; e < MT * 16 * 16; e += kGemmWaves * kWave) {
        const int m = e / 16, nn = e % 16;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kGemmWaves; ++w) s += part[w][m][nn];
        if (m < M && n0 + nn < N) C[(size_t)m * N + n0 + nn] = from_f32<_Float16>(s);
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
    if (vec)
        hipLaunchKernelGGL((dequantize_kernel<FMT, MODE, true>), dim3(qlh::blocks_for(g.n / 8, kBlock)),
                           dim3(kBlock), 0, st, q, g, s, y);
    else
        hipLaunchKernelGGL((dequantize_kernel<FMT, MODE, false>), dim3(qlh::blocks_for(g.n, kBlock)),
                           dim3(kBlock), 0, st, q, g, s, y);
}

template <int FMT, int MODE, int MT>
void launch_skinny(const _Float16* A, const uint8_t* W, const float* s, _Float16* C, int M, int N,
                   int K, long long gs, hipStream_t st) {
    hipLaunchKernelGGL((fp8_gemm_skinny<FMT, MODE, MT>), dim3((unsigned)(N / 16)),
                       dim3(kGemmWaves * kWave), 0, st, A, W, s, C, M, N, K, gs);
}

template <int FMT, int MODE>
void launch_skinny_mt(const _Float16* A, const uint8_t* W, const float* s, _Float16* C, int M, int N,
                      int K, long long gs, hipStream_t st) {
    if (M <= 16) launch_skinny<FMT, MODE, 1>(A, W, s, C, M, N, K, gs, st);
    else if (M <= 32) launch_skinny<FMT, MODE, 2>(A, W, s, C, M, N, K, gs, st);
    else launch_skinny<FMT, MODE, 4>(A, W, s, C, M, N, K, gs, st);
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
    if (g.gs <= 8192) {
        hipLaunchKernelGGL(absmax_wave, dim3(qlh::blocks_for(g.n_groups, kBlock / kWave)), dim3(kBlock),
                           0, stream, x, g, mode, scales);
    } else {
        QL_CHECK_ARG(g.n_groups <= 65535);
        hipLaunchKernelGGL(fill_zero, dim3(sblocks), dim3(kBlock), 0, stream, scales, g.n_groups);
        const long long per = 16LL * kBlock;
        unsigned bx = (unsigned)((g.gs + per - 1) / per);
        if (bx > 1024) bx = 1024;
        hipLaunchKernelGGL(absmax_blocks, dim3(bx, (unsigned)g.n_groups), dim3(kBlock), 0, stream, x, g,
                           mode, scales);
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
    const hipError_t e = ql_fp8_scales(src, rows, cols, format, granularity, group_size, mode, scales, stream);
    if (e != hipSuccess) return e;
    const bool vec = g.n % 8 == 0 && g.gs % 8 == 0 && qlh::aligned16(src) && ((uintptr_t)dst & 7) == 0;
    QL_FP8_DISPATCH(format, mode, launch_quantize, reinterpret_cast<const _Float16*>(src), g, scales,
                    dst, vec, stream);
    return hipGetLastError();
}

extern "C" hipError_t ql_fp8_dequantize(const uint8_t* src, const float* scales, int rows, int cols,
                                        int format, int granularity, int group_size, int mode,
                                        uint16_t* dst, hipStream_t stream) {
    Geom g;
    QL_CHECK_ARG(fmt_mode_ok(format, mode) && geom_for(rows, cols, granularity, group_size, g));
    if (g.n == 0) return hipSuccess;
    QL_CHECK_ARG(src && scales && dst);
    const bool vec = g.n % 8 == 0 && g.gs % 8 == 0 && qlh::aligned16(dst) && ((uintptr_t)src & 7) == 0;
    QL_FP8_DISPATCH(format, mode, launch_dequantize, src, g, scales, reinterpret_cast<_Float16*>(dst),
                    vec, stream);
    return hipGetLastError();
}

extern "C" hipError_t ql_fp8_gemm_f16(const uint16_t* A, const uint8_t* W, const float* scales,
                                      int M, int N, int K, int format, int granularity,
                                      int group_size, int mode, uint16_t* C, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream) {
    Geom g;
    QL_CHECK_ARG(fmt_mode_ok(format, mode) && M >= 0 && N >= 0 && K >= 0);
    QL_CHECK_ARG(geom_for(N, K, granularity, group_size, g));
    if (M == 0 || N == 0) return hipSuccess;
    QL_CHECK_ARG(A && W && scales && C && K > 0);
    const bool skinny = M <= 64 && N % 16 == 0 && K % 64 == 0 && g.gs % 16 == 0 &&
                        qlh::aligned16(A) && qlh::aligned16(W) && N / 16 <= 0x7fffffff;
    if (skinny) {
        QL_FP8_DISPATCH(format, mode, launch_skinny_mt, reinterpret_cast<const _Float16*>(A), W, scales,
                        reinterpret_cast<_Float16*>(C), M, N, K, g.gs, stream);
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
