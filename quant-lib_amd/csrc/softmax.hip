// softmax.hip -- numerically stable row softmax for gfx950.
//
// Arithmetic (kernels/softmax.cu:44-85):
//   m   = max(-FLT_MAX, max_c x_c)
//   e_c = exp(x_c - m)             (-inf inputs give exactly 0)
//   out = e_c * (1 / sum_c e_c)    (one correctly rounded division per row)
// The reference makes three passes over the row (max; exp + write e; rescale),
// i.e. three reads and two writes.  Here the row lives in registers: one read
// and one write per element, with nontemporal hints.  WPR wavefronts share a
// row; each lane holds NV 16-byte vectors, lanes past the row end hold -inf
// (no effect on max or sum).  Every lane loads -- an index past the row
// re-reads the row's last vector, masked afterwards -- so all NV loads issue
// back to back; rows that are exactly NV*64*WPR vectors (FULL) skip the masks;
// rows past the end re-read the last row and store nothing.
// The fp16 variant (no reference kernel) is the same fp32 arithmetic with
// binary16 input and RNE binary16 output.
#include <float.h>

#include "ql_common.hpp"
#include "quantlib_amd.h"

namespace {

using namespace ql;

template <typename D>
__device__ __forceinline__ float softmax_exp(float y) {
    // fp32 output keeps the residual-corrected exponential (1e-5 relative
    // budget); binary16 output cannot see the difference.
    if constexpr (sizeof(D) == 4) return exp_f32(y);
    else return exp_f32_fast(y);
}

// ANY: rows of any length, whose starts need not be 16-byte aligned (in and out at
// the same offset modulo 16): a row's vectors are the aligned 16-byte vectors that
// cover it, the first starting p elements before the row; elements outside the row
// count as -inf, and the first and last vectors, shared with the neighbouring rows,
// are stored element by element.  (An aligned 16-byte vector never crosses a page,
// so the covering loads stay within mapped memory.)
template <typename D, int NV, int WPR, bool FULL, bool ANY = false>
__global__ __launch_bounds__(WPR <= 4 ? kBlock : kWave * WPR) void softmax_rows(
    const D* __restrict__ in, D* __restrict__ out, int rows, int cols) {
    constexpr int W = vec16<D>();
    constexpr int TPR = kWave * WPR;
    constexpr int BLOCK = WPR <= 4 ? kBlock : kWave * WPR;
    constexpr int RPB = BLOCK / TPR;
    using V = Vec<D, W>;

    const int tid = threadIdx.x;
    const int row = blockIdx.x * RPB + tid / TPR;
    const int rl = tid % TPR;
    const bool row_ok = row < rows;
    const size_t roff = (size_t)(row_ok ? row : rows - 1) * (size_t)cols;
    const int p = ANY ? (int)((reinterpret_cast<uintptr_t>(in + roff) & 15) / sizeof(D)) : 0;
    const int nvec = ANY ? (p + cols + W - 1) / W : cols / W;
    const V* src = reinterpret_cast<const V*>(in + roff - p);

    // every lane loads (an index past the row re-reads its last vector, masked
    // below): a load under a per-lane test makes the compiler wait for it before
    // issuing the next one
    V raw[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) raw[k] = load<true>(src + (FULL ? rl + k * TPR : min(rl + k * TPR, nvec - 1)));

    float v[NV][W];
    float m = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int vi = rl + k * TPR;
        const bool ok = FULL || vi < nvec;
#pragma unroll
        for (int e = 0; e < W; ++e) v[k][e] = ok ? to_f32(raw[k].v[e]) : -INFINITY;
        if (ANY && ok && (vi * W < p || vi * W + W - p > cols)) {   // the row's first or last vector
#pragma unroll
            for (int e = 0; e < W; ++e)
                if (vi * W + e - p < 0 || vi * W + e - p >= cols) v[k][e] = -INFINITY;
        }
#pragma unroll
        for (int e = 0; e < W; ++e) m = fmaxf(m, v[k][e]);
    }
    m = wave_max(m);
    if constexpr (WPR > 1) {
        __shared__ float redm[BLOCK / kWave];
        if ((tid & (kWave - 1)) == 0) redm[tid / kWave] = m;
        __syncthreads();
        const int w0 = (tid / TPR) * WPR;
        m = -FLT_MAX;
#pragma unroll
        for (int i = 0; i < WPR; ++i) m = fmaxf(m, redm[w0 + i]);
    }

    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
#pragma unroll
        for (int e = 0; e < W; ++e) {
            v[k][e] = softmax_exp<D>(v[k][e] - m);
            s += v[k][e];
        }
    }
    s = wave_sum(s);
    if constexpr (WPR > 1) {
        __shared__ float reds[BLOCK / kWave];
        if ((tid & (kWave - 1)) == 0) reds[tid / kWave] = s;
        __syncthreads();
        const int w0 = (tid / TPR) * WPR;
        s = 0.0f;
#pragma unroll
        for (int i = 0; i < WPR; ++i) s += reds[w0 + i];
    }
    const float inv = 1.0f / s;

    if (!row_ok) return;
    V* dst = reinterpret_cast<V*>(out + roff - p);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int vi = rl + k * TPR;
        if (FULL || vi < nvec) {
            V y;
#pragma unroll
            for (int e = 0; e < W; ++e) y.v[e] = from_f32<D>(v[k][e] * inv);
            if (!ANY || (vi * W >= p && vi * W + W - p <= cols)) {
                store<true>(dst + vi, y);
            } else {   // a vector shared with a neighbouring row: this row's elements only
                D* d = out + roff - p + (size_t)vi * W;
#pragma unroll
                for (int e = 0; e < W; ++e)
                    if (vi * W + e - p >= 0 && vi * W + e - p < cols) d[e] = y.v[e];
            }
        }
    }
}

// Block-per-row three-pass loop for any width / alignment (exp recomputed in
// pass 3, bit-identical to pass 2).
template <typename D>
__global__ __launch_bounds__(kBlock) void softmax_rows_generic(const D* __restrict__ in,
                                                              D* __restrict__ out, int rows,
                                                              int cols) {
    const int row = blockIdx.x;  // grid.x == rows
    (void)rows;
    const int tid = threadIdx.x;
    const size_t roff = (size_t)row * (size_t)cols;
    __shared__ float red[kBlock / kWave];

    float m = -FLT_MAX;
    for (int c = tid; c < cols; c += kBlock) m = fmaxf(m, to_f32(in[roff + c]));
    m = wave_max(m);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = m;
    __syncthreads();
    m = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < kBlock / kWave; ++i) m = fmaxf(m, red[i]);
    __syncthreads();

    float s = 0.0f;
    for (int c = tid; c < cols; c += kBlock) s += softmax_exp<D>(to_f32(in[roff + c]) - m);
    s = wave_sum(s);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = s;
    __syncthreads();
    s = 0.0f;
#pragma unroll
    for (int i = 0; i < kBlock / kWave; ++i) s += red[i];
    const float inv = 1.0f / s;

    for (int c = tid; c < cols; c += kBlock)
        out[roff + c] = from_f32<D>(softmax_exp<D>(to_f32(in[roff + c]) - m) * inv);
}

template <typename D, int NV, int WPR, bool ANY = false>
hipError_t launch_fast(const D* in, D* out, int rows, int cols, hipStream_t stream) {
    constexpr int BLOCK = WPR <= 4 ? kBlock : kWave * WPR;
    constexpr int RPB = BLOCK / (kWave * WPR);
    const dim3 grid(qlh::blocks_for(rows, RPB));
    if constexpr (ANY)
        hipLaunchKernelGGL((softmax_rows<D, NV, WPR, false, true>), grid, dim3(BLOCK), 0, stream, in,
                           out, rows, cols);
    else if (cols / vec16<D>() == NV * kWave * WPR)
        hipLaunchKernelGGL((softmax_rows<D, NV, WPR, true>), grid, dim3(BLOCK), 0, stream, in,
                           out, rows, cols);
    else
        hipLaunchKernelGGL((softmax_rows<D, NV, WPR, false>), grid, dim3(BLOCK), 0, stream, in,
                           out, rows, cols);
    return hipGetLastError();
}

template <typename D>
hipError_t softmax_dispatch(const D* in, D* out, int rows, int cols, hipStream_t stream) {
    QL_CHECK_ARG(rows >= 0 && cols >= 0);
    if (rows == 0) return hipSuccess;
    QL_CHECK_ARG(cols > 0);
    QL_CHECK_ARG(in && out);
    constexpr int W = vec16<D>();
    const bool vec_ok = cols % W == 0 && qlh::aligned16(in) && qlh::aligned16(out);
    // other lengths or element-aligned pointers: the covering aligned vectors of each
    // row, when in and out share their offset mod 16
    const bool any = !vec_ok && (reinterpret_cast<uintptr_t>(in) & (sizeof(D) - 1)) == 0 &&
                     ((reinterpret_cast<uintptr_t>(in) - reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (any) {   // at most (cols + 2W - 2) / W covering vectors
        const int nv = (cols + 2 * W - 2) / W;
        if (nv <= 64) return launch_fast<D, 1, 1, true>(in, out, rows, cols, stream);
        if (nv <= 128) return launch_fast<D, 2, 1, true>(in, out, rows, cols, stream);
        if constexpr (sizeof(D) == 2) {
            if (nv <= 256) return launch_fast<D, 4, 1, true>(in, out, rows, cols, stream);
            if (nv <= 512) return launch_fast<D, 8, 1, true>(in, out, rows, cols, stream);
            if (nv <= 576) return launch_fast<D, 9, 1, true>(in, out, rows, cols, stream);
        } else {
            if (nv <= 256) return launch_fast<D, 2, 2, true>(in, out, rows, cols, stream);
            if (nv <= 512) return launch_fast<D, 2, 4, true>(in, out, rows, cols, stream);
        }
        if (nv <= 1024) return launch_fast<D, 2, 8, true>(in, out, rows, cols, stream);
        if (nv <= 1536) return launch_fast<D, 3, 8, true>(in, out, rows, cols, stream);
        if (nv <= 2048) return launch_fast<D, 2, 16, true>(in, out, rows, cols, stream);
        if (nv <= 3072) return launch_fast<D, 3, 16, true>(in, out, rows, cols, stream);
        if (nv <= 4096) return launch_fast<D, 4, 16, true>(in, out, rows, cols, stream);
        if (nv <= 6144) return launch_fast<D, 6, 16, true>(in, out, rows, cols, stream);
        if (nv <= 8192) return launch_fast<D, 8, 16, true>(in, out, rows, cols, stream);
        if (nv <= 12288) return launch_fast<D, 12, 16, true>(in, out, rows, cols, stream);
        if (nv <= 16384) return launch_fast<D, 16, 16, true>(in, out, rows, cols, stream);
    }
    const int nvec = cols / W;
    if (vec_ok) {
        if (nvec <= 64) return launch_fast<D, 1, 1>(in, out, rows, cols, stream);
        if (nvec <= 128) return launch_fast<D, 2, 1>(in, out, rows, cols, stream);
        if constexpr (sizeof(D) == 2) {
            // binary16 rows up to 4096 wide: one wavefront per row, up to eight
            // 16-byte vectors per lane, four rows per workgroup (C4 fp16: 11.6
            // us against 14.2 us for four wavefronts of two vectors per row).
            if (nvec <= 256) return launch_fast<D, 4, 1>(in, out, rows, cols, stream);
            if (nvec <= 512) return launch_fast<D, 8, 1>(in, out, rows, cols, stream);
        } else {
            // Two 16-byte vectors per lane, as many wavefronts per row as that
            // needs: measured fastest at C4 fp32.
            if (nvec <= 256) return launch_fast<D, 2, 2>(in, out, rows, cols, stream);
            if (nvec <= 512) return launch_fast<D, 2, 4>(in, out, rows, cols, stream);
        }
        // wider rows, both: 8-16 wavefronts per row, 2-16 vectors per lane
        if (nvec <= 1024) return launch_fast<D, 2, 8>(in, out, rows, cols, stream);
        if (nvec <= 2048) return launch_fast<D, 2, 16>(in, out, rows, cols, stream);
        if (nvec <= 4096) return launch_fast<D, 4, 16>(in, out, rows, cols, stream);
        if (nvec <= 8192) return launch_fast<D, 8, 16>(in, out, rows, cols, stream);
        if (nvec <= 16384) return launch_fast<D, 16, 16>(in, out, rows, cols, stream);
    }
    hipLaunchKernelGGL((softmax_rows_generic<D>), dim3((unsigned)rows), dim3(kBlock), 0,
                       stream, in, out, rows, cols);
    return hipGetLastError();
}

}  // namespace

extern "C" hipError_t ql_softmax_f32(const float* in, float* out, int rows, int cols,
                                     hipStream_t stream) {
    return softmax_dispatch<float>(in, out, rows, cols, stream);
}

extern "C" hipError_t ql_softmax_f16(const uint16_t* in, uint16_t* out, int rows, int cols,
                                     hipStream_t stream) {
    return softmax_dispatch<_Float16>(reinterpret_cast<const _Float16*>(in),
                                      reinterpret_cast<_Float16*>(out), rows, cols, stream);
}
