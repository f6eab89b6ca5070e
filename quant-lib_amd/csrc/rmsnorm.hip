// rmsnorm.hip -- RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Arithmetic (kernels/rmsnorm.cu:27-48, kernels/fp16_ops.cu:18-41):
//   ss  = sum_i x_i^2                       (fp32)
//   inv = 1 / sqrt(ss / dim + eps)          (correctly rounded div and sqrt)
//   y_i = (x_i * inv) * w_i                 (fp32, then RNE to binary16 for fp16)
// Fused add (src/fp16_forward.cu:213-216 chain): x_i <- round_D(x_i + d_i) is
// stored and the norm is taken of that rounded value.
//
// Layout: rows of `dim` contiguous elements.  Fast path: the row is held in
// registers; WPR wavefronts share a row, each lane owns NV 16-byte vectors
// (vector index lane + k*64*WPR, so every load instruction of a wavefront is
// one contiguous 1 KiB span).  x (and d) are read once and y (and x') written
// once: 2 (4 fused) row transfers per row, the HBM minimum, with nontemporal
// hints on the streamed rows and ordinary (cached) loads of the shared weight.
// Other lengths and offsets hold the row's covering aligned vectors in registers;
// rows too wide for registers, or x, d and out at different offsets modulo 16,
// take a block-per-row loop that re-reads x.
#include "ql_common.hpp"
#include "quantlib_amd.h"

namespace {

using namespace ql;

// A row-group of WPR wavefronts handles RPT consecutive rows: all their loads
// are issued first, the RPT partial sums are reduced together (one LDS
// exchange and one barrier per group), then the rows are written.
template <typename D, int NV, int WPR, int RPT, bool ADD, bool NT = true>
__global__ __launch_bounds__(WPR <= 4 ? kBlock : kWave * WPR) void rmsnorm_rows(
    D* x, const D* __restrict__ d, const D* __restrict__ w, D* __restrict__ out,
    int rows, int dim, float eps) {
    constexpr int W = vec16<D>();
    constexpr int TPR = kWave * WPR;                       // threads per row-group
    constexpr int BLOCK = WPR <= 4 ? kBlock : kWave * WPR;
    constexpr int GPB = BLOCK / TPR;                       // row-groups per block
    using V = Vec<D, W>;

    const int tid = threadIdx.x;
    const int row0 = (blockIdx.x * GPB + tid / TPR) * RPT;
    const int rl = tid % TPR;
    const int nvec = dim / W;
    const V* wr = reinterpret_cast<const V*>(w);

    // Every lane loads -- rows past the end re-read row 0, indices past the row
    // its last vector: a load under a per-lane test makes the compiler wait for
    // it before issuing the next one, which had put a wait for the (cached)
    // weight load ahead of every row's HBM loads.  The weight is issued first:
    // loads complete in order, so the wait for the rows covers it.
    V xv[RPT][NV], wv[NV];
    V dv[ADD ? RPT : 1][ADD ? NV : 1];
#pragma unroll
    for (int k = 0; k < NV; ++k) wv[k] = wr[min(rl + k * TPR, nvec - 1)];  // cached: shared by every row
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int row = row0 + r;
        const V* xr = reinterpret_cast<const V*>(x + (size_t)(row < rows ? row : 0) * dim);
        const V* dr = reinterpret_cast<const V*>(ADD ? d + (size_t)(row < rows ? row : 0) * dim : d);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int vi = min(rl + k * TPR, nvec - 1);
            xv[r][k] = load<NT>(xr + vi);
            if constexpr (ADD) dv[r][k] = load<NT>(dr + vi);
        }
    }
    __builtin_amdgcn_sched_barrier(0);   // every load issued before any arithmetic

    // Values stay in D precision (exact for the rounded sum) to halve the
    // register footprint of binary16 rows; they are widened again for output.
    // Every lane computes; lanes past the row add fmaf(0, 0, ss) == ss.  (With
    // the arithmetic under a per-lane test the compiler moved the d loads into
    // it, behind the wait for x.)
    float ss[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        ss[r] = 0.0f;
        const bool row_ok = row0 + r < rows;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int vi = rl + k * TPR;
            const bool ok = row_ok && vi < nvec;
#pragma unroll
            for (int e = 0; e < W; ++e) {
                float a = to_f32(xv[r][k].v[e]);
                if constexpr (ADD) {
                    a = a + to_f32(dv[r][k].v[e]);
                    xv[r][k].v[e] = from_f32<D>(a);
                    a = to_f32(xv[r][k].v[e]);
                }
                a = ok ? a : 0.0f;
                ss[r] = fmaf(a, a, ss[r]);
            }
            // the rounded sum x' is final: store it now, before the row's
            // reduction (measured 0.7% faster than with y)
            if (ADD && ok)
                store<NT>(reinterpret_cast<V*>(x + (size_t)(row0 + r) * dim) + vi, xv[r][k]);
        }
        ss[r] = wave_sum(ss[r]);
    }
    if constexpr (WPR > 1) {
        __shared__ float red[BLOCK / kWave][RPT];
#pragma unroll
        for (int r = 0; r < RPT; ++r)
            if ((tid & (kWave - 1)) == 0) red[tid / kWave][r] = ss[r];
        __syncthreads();
        const int w0 = (tid / TPR) * WPR;
#pragma unroll
        for (int r = 0; r < RPT; ++r) {
            ss[r] = 0.0f;
#pragma unroll
            for (int i = 0; i < WPR; ++i) ss[r] += red[w0 + i][r];
        }
    }

#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int row = row0 + r;
        if (row >= rows) continue;
        const float inv = 1.0f / sqrtf(ss[r] / (float)dim + eps);
        V* orow = reinterpret_cast<V*>(out + (size_t)row * dim);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int vi = rl + k * TPR;
            if (vi < nvec) {
                V y;
#pragma unroll
                for (int e = 0; e < W; ++e)
                    y.v[e] = from_f32<D>((to_f32(xv[r][k].v[e]) * inv) * to_f32(wv[k].v[e]));
                // plain RMSNorm writes y through (sc1 nt): 25.8 -> 24.3 us at
                // 8192 x 4096 binary16 on MI355X; with the fused add it measured
                // no faster (x' and y both 0.5% either way), so it keeps NT
                if constexpr (!ADD && NT) store_wt(uniform(orow), (uint32_t)vi * (uint32_t)sizeof(V), y);
                else store<NT>(orow + vi, y);
            }
        }
    }
}

// One wavefront per row (launched with grid = rows, 64-thread workgroups): the
// row's NV vectors per lane are loaded, reduced with the wave64 butterfly alone
// (no LDS, no barrier) and written.  Used below 4096 rows, where one small
// workgroup per row fills the chip better than row groups.
template <typename D, int NV, bool ADD>
__global__ __launch_bounds__(kWave) void rmsnorm_wave(D* x, const D* __restrict__ d,
                                                     const D* __restrict__ w,
                                                     D* __restrict__ out, int dim, float eps) {
    constexpr int W = vec16<D>();
    using V = Vec<D, W>;
    const int rl = threadIdx.x;
    const int nvec = dim / W;
    const size_t row = blockIdx.x;
    const V* wr = reinterpret_cast<const V*>(w);
    const V* xr = reinterpret_cast<const V*>(x + row * dim);
    const V* dr = reinterpret_cast<const V*>(ADD ? d + row * dim : d);
    // every lane loads (indices past the row re-read its last vector), the
    // shared weight first, as in rmsnorm_rows
    V cx[NV], cd[ADD ? NV : 1], wv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) wv[k] = wr[min(rl + k * kWave, nvec - 1)];   // cached
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int vi = min(rl + k * kWave, nvec - 1);
        cx[k] = load<true>(xr + vi);
        if constexpr (ADD) cd[k] = load<true>(dr + vi);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load issued before any arithmetic
    float ss = 0.0f;   // every lane computes; lanes past the row add fmaf(0, 0, ss)
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const bool ok = rl + k * kWave < nvec;
#pragma unroll
        for (int e = 0; e < W; ++e) {
            float a = to_f32(cx[k].v[e]);
            if constexpr (ADD) {
                a = a + to_f32(cd[k].v[e]);
                cx[k].v[e] = from_f32<D>(a);
                a = to_f32(cx[k].v[e]);
            }
            a = ok ? a : 0.0f;
            ss = fmaf(a, a, ss);
        }
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    V* xw = reinterpret_cast<V*>(x + row * dim);
    V* orow = reinterpret_cast<V*>(out + row * dim);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int vi = rl + k * kWave;
        if (vi < nvec) {
            V y;
#pragma unroll
            for (int e = 0; e < W; ++e)
                y.v[e] = from_f32<D>((to_f32(cx[k].v[e]) * inv) * to_f32(wv[k].v[e]));
            if constexpr (ADD) store<true>(xw + vi, cx[k]);
            store<true>(orow + vi, y);
        }
    }
}

// Rows of any length whose starts need not be 16-byte aligned (x, d and out at one
// offset modulo 16): WPR wavefronts per row, each lane NV of the aligned 16-byte
// vectors that cover the row, the first starting p elements before it.  Elements
// outside the row add nothing to the sum and are not written: the row's first and
// last vectors, shared with the neighbouring rows, are stored element by element.
// The weights of a vector's columns c0 .. c0 + W - 1 are two aligned vectors of w
// (w at its own offset pw) shifted by s = (pw + c0) mod W, which is the same for
// every vector of a row; the first and last pair are clamped to w's covering
// vectors, which changes only weights of columns outside the row.  (An aligned
// 16-byte vector never crosses a page, so the covering loads stay within mapped
// memory.)
// One row per workgroup of blockDim.x = 64 * wpr threads (wpr <= 16, chosen by the
// host as the fewest wavefronts whose NV vectors per lane cover the row, so few
// lanes sit idle and as many rows as fit stay in flight per CU).
constexpr int kAnyMaxWaves = 16;

template <typename D, int NV, bool ADD>
__global__ __launch_bounds__(kWave * kAnyMaxWaves) void rmsnorm_any(
    D* x, const D* __restrict__ d, const D* __restrict__ w, D* __restrict__ out, int dim, float eps) {
    constexpr int W = vec16<D>();
    using V = Vec<D, W>;

    const int tid = threadIdx.x;
    const int TPR = blockDim.x;
    const int row = blockIdx.x;   // grid.x == rows
    const int rl = tid;
    const size_t roff = (size_t)row * (size_t)dim;
    const int p = (int)((reinterpret_cast<uintptr_t>(x + roff) & 15) / sizeof(D));
    const int nvec = (p + dim + W - 1) / W;
    const V* xr = reinterpret_cast<const V*>(x + roff - p);
    const V* dr = reinterpret_cast<const V*>(ADD ? d + roff - p : d);

    const int pw = (int)((reinterpret_cast<uintptr_t>(w) & 15) / sizeof(D));
    const V* wa = reinterpret_cast<const V*>(w - pw);
    const int wlast = (pw + dim - 1) / W;   // w's last covering vector
    const int sh = (pw - p + W) % W;
    V xv[NV], dv[ADD ? NV : 1], w0[NV], w1[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {   // the shared weight first (cached), then the row
        const int ja = (pw + min(rl + k * TPR, nvec - 1) * W - p + W) / W - 1;   // floor, >= -1
        w0[k] = wa[min(max(ja, 0), wlast)];
        w1[k] = wa[min(ja + 1, wlast)];
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int vi = min(rl + k * TPR, nvec - 1);
        xv[k] = load<true>(xr + vi);
        if constexpr (ADD) dv[k] = load<true>(dr + vi);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load issued before any arithmetic
    V wv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) wv[k] = take_at(sh, w0[k], w1[k]);

    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int vi = rl + k * TPR;
#pragma unroll
        for (int e = 0; e < W; ++e) {
            float a = to_f32(xv[k].v[e]);
            if constexpr (ADD) {
                a = a + to_f32(dv[k].v[e]);
                xv[k].v[e] = from_f32<D>(a);
                a = to_f32(xv[k].v[e]);
            }
            const int c = vi * W + e - p;
            a = c >= 0 && c < dim ? a : 0.0f;   // vectors past the row: c >= dim
            ss = fmaf(a, a, ss);
        }
    }
    ss = wave_sum(ss);
    const int wpr = TPR / kWave;   // uniform
    if (wpr > 1) {
        __shared__ float red[kAnyMaxWaves];
        if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
        __syncthreads();
        ss = 0.0f;
        for (int i = 0; i < wpr; ++i) ss += red[i];
    }
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int vi = rl + k * TPR;
        if (vi < nvec) {
            V y;
#pragma unroll
            for (int e = 0; e < W; ++e) y.v[e] = from_f32<D>((to_f32(xv[k].v[e]) * inv) * to_f32(wv[k].v[e]));
            if (vi * W >= p && vi * W + W - p <= dim) {
                if constexpr (ADD) store<true>(reinterpret_cast<V*>(x + roff - p) + vi, xv[k]);
                store<true>(reinterpret_cast<V*>(out + roff - p) + vi, y);
            } else {   // shared with a neighbouring row: this row's elements only
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    const int c = vi * W + e - p;
                    if (c >= 0 && c < dim) {
                        if constexpr (ADD) x[roff + c] = xv[k].v[e];
                        out[roff + c] = y.v[e];
                    }
                }
            }
        }
    }
}

template <typename D, int NV, bool ADD>
hipError_t launch_any(D* x, const D* d, const D* w, D* out, int rows, int nv, int dim, float eps,
                      hipStream_t stream) {
    const int wpr = (nv + NV * kWave - 1) / (NV * kWave);   // <= kAnyMaxWaves by the caller's choice of NV
    hipLaunchKernelGGL((rmsnorm_any<D, NV, ADD>), dim3((unsigned)rows), dim3(kWave * wpr), 0, stream, x, d, w,
                       out, dim, eps);
    return hipGetLastError();
}

// Block-per-row loop for any dim / alignment.  Same arithmetic; x' is written
// in the first pass and re-read by the same thread in the second.
template <typename D, bool ADD>
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_generic(
    D* x, const D* __restrict__ d, const D* __restrict__ w, D* __restrict__ out,
    int rows, int dim, float eps) {
    const int row = blockIdx.x;  // grid.x == rows
    (void)rows;
    const int tid = threadIdx.x;
    const size_t roff = (size_t)row * (size_t)dim;
    float ss = 0.0f;
    for (int i = tid; i < dim; i += kBlock) {
        float a = to_f32(x[roff + i]);
        if constexpr (ADD) {
            a = round_to<D>(a + to_f32(d[roff + i]));
            x[roff + i] = from_f32<D>(a);
        }
        ss = fmaf(a, a, ss);
    }
    ss = wave_sum(ss);
    __shared__ float red[kBlock / kWave];
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = ss;
    __syncthreads();
    ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kBlock / kWave; ++i) ss += red[i];
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = tid; i < dim; i += kBlock) {
        const float a = to_f32(x[roff + i]);
        out[roff + i] = from_f32<D>((a * inv) * to_f32(w[i]));
    }
}

template <typename D, int NV, int WPR, bool ADD, int RPT = 1>
hipError_t launch_fast(D* x, const D* d, const D* w, D* out, int rows, int dim, float eps,
                       hipStream_t stream) {
    constexpr int BLOCK = WPR <= 4 ? kBlock : kWave * WPR;
    constexpr int RPB = BLOCK / (kWave * WPR) * RPT;
    const unsigned grid = qlh::blocks_for(rows, RPB);
    hipLaunchKernelGGL((rmsnorm_rows<D, NV, WPR, RPT, ADD>), dim3(grid), dim3(BLOCK), 0, stream,
                       x, d, w, out, rows, dim, eps);
    return hipGetLastError();
}

constexpr int kSmallRows = 4096;

template <typename D, bool ADD>
hipError_t rmsnorm_dispatch(D* x, const D* d, const D* w, D* out, int rows, int dim,
                            float eps, hipStream_t stream) {
    QL_CHECK_ARG(rows >= 0 && dim >= 0);
    if (rows == 0) return hipSuccess;
    QL_CHECK_ARG(dim > 0);
    QL_CHECK_ARG(x && w && out && (!ADD || d));
    constexpr int W = vec16<D>();
    const bool vec_ok = dim % W == 0 && qlh::aligned16(x) && qlh::aligned16(w) &&
                        qlh::aligned16(out) && (!ADD || qlh::aligned16(d));
    const int nvec = dim / W;
    if (vec_ok && rows < kSmallRows && nvec <= 512) {
        // Few rows (e.g. 2048 x 2048 fp32): one single-wavefront workgroup per
        // row, no cross-wave exchange -- measured faster than spreading rows
        // over 512-thread groups when the whole problem is a few tens of MB.
        const unsigned grid = (unsigned)rows;
        if (nvec <= 64)
            hipLaunchKernelGGL((rmsnorm_wave<D, 1, ADD>), dim3(grid), dim3(kWave), 0, stream, x,
                               d, w, out, dim, eps);
        else if (nvec <= 128)
            hipLaunchKernelGGL((rmsnorm_wave<D, 2, ADD>), dim3(grid), dim3(kWave), 0, stream, x,
                               d, w, out, dim, eps);
        else if (nvec <= 256)
            hipLaunchKernelGGL((rmsnorm_wave<D, 4, ADD>), dim3(grid), dim3(kWave), 0, stream, x,
                               d, w, out, dim, eps);
        else
            hipLaunchKernelGGL((rmsnorm_wave<D, 8, ADD>), dim3(grid), dim3(kWave), 0, stream, x,
                               d, w, out, dim, eps);
        return hipGetLastError();
    }
    if (vec_ok) {
        if (nvec <= 64) return launch_fast<D, 1, 1, ADD>(x, d, w, out, rows, dim, eps, stream);
        if constexpr (!ADD) {
            // Plain RMSNorm reads one row, not two: two 16-byte vectors per
            // lane over half the wavefronts keep as many bytes in flight per
            // lane as the fused kernel's x and d.  Measured on MI355X (8192
            // rows, rotating buffers): binary16 4096 wide 24.3 -> 23.1 us, 8192
            // wide 52.2 -> 44.6, 1024 wide 7.8 -> 6.8; fp32 4096 wide 51.6 ->
            // 44.4; 2048 wide equal.
            if (nvec <= 128) return launch_fast<D, 2, 1, ADD>(x, d, w, out, rows, dim, eps, stream);
            if (nvec <= 256) return launch_fast<D, 2, 2, ADD>(x, d, w, out, rows, dim, eps, stream);
            if (nvec <= 512) return launch_fast<D, 2, 4, ADD>(x, d, w, out, rows, dim, eps, stream);
            if (nvec <= 1024) return launch_fast<D, 2, 8, ADD>(x, d, w, out, rows, dim, eps, stream);
        } else {
            // The fused add: a row over as many wavefronts as it has 64-vector
            // chunks (up to 16), one 16-byte vector per lane (more waves in
            // flight, shorter reduction tails; two vectors per lane measured
            // 0.1-1.9% slower at 1024-8192 wide).
            if (nvec <= 128) return launch_fast<D, 1, 2, ADD>(x, d, w, out, rows, dim, eps, stream);
            if (nvec <= 256) return launch_fast<D, 1, 4, ADD>(x, d, w, out, rows, dim, eps, stream);
            if (nvec <= 512) return launch_fast<D, 1, 8, ADD>(x, d, w, out, rows, dim, eps, stream);
            if (nvec <= 1024) return launch_fast<D, 1, 16, ADD>(x, d, w, out, rows, dim, eps, stream);
        }
        // wider rows, both: 16 wavefronts, 2-8 vectors per lane
        if (nvec <= 2048) return launch_fast<D, 2, 16, ADD>(x, d, w, out, rows, dim, eps, stream);
        if (nvec <= 4096) return launch_fast<D, 4, 16, ADD>(x, d, w, out, rows, dim, eps, stream);
        if (nvec <= 8192) return launch_fast<D, 8, 16, ADD>(x, d, w, out, rows, dim, eps, stream);
    }
    // other lengths or offsets: the covering aligned vectors of each row, when x, d and
    // out share their offset mod 16 (at most (dim + 2W - 2) / W vectors a row).  As on
    // the aligned path, the fused add takes one vector per lane and plain RMSNorm two,
    // over as many wavefronts as cover the row (up to 16), then 2-8 over 16.
    const uintptr_t xa = reinterpret_cast<uintptr_t>(x);
    const bool any = (xa & (sizeof(D) - 1)) == 0 && ((xa - reinterpret_cast<uintptr_t>(out)) & 15) == 0 &&
                     (!ADD || ((xa - reinterpret_cast<uintptr_t>(d)) & 15) == 0);
    const int nv = (dim + 2 * W - 2) / W;
    if (any) {
        if (nv <= (ADD ? 1024 : 64)) return launch_any<D, 1, ADD>(x, d, w, out, rows, nv, dim, eps, stream);
        if (nv <= 2048) return launch_any<D, 2, ADD>(x, d, w, out, rows, nv, dim, eps, stream);
        if (nv <= 4096) return launch_any<D, 4, ADD>(x, d, w, out, rows, nv, dim, eps, stream);
        if (nv <= 8192) return launch_any<D, 8, ADD>(x, d, w, out, rows, nv, dim, eps, stream);
    }
    hipLaunchKernelGGL((rmsnorm_rows_generic<D, ADD>), dim3((unsigned)rows), dim3(kBlock), 0,
                       stream, x, d, w, out, rows, dim, eps);
    return hipGetLastError();
}

}  // namespace

extern "C" hipError_t ql_rmsnorm_f32(const float* x, const float* w, float* out, int rows,
                                     int dim, float eps, hipStream_t stream) {
    return rmsnorm_dispatch<float, false>(const_cast<float*>(x), nullptr, w, out, rows, dim,
                                          eps, stream);
}

extern "C" hipError_t ql_rmsnorm_f16(const uint16_t* x, const uint16_t* w, uint16_t* out,
                                     int rows, int dim, float eps, hipStream_t stream) {
    return rmsnorm_dispatch<_Float16, false>(
        reinterpret_cast<_Float16*>(const_cast<uint16_t*>(x)), nullptr,
        reinterpret_cast<const _Float16*>(w), reinterpret_cast<_Float16*>(out), rows, dim,
        eps, stream);
}

extern "C" hipError_t ql_add_rmsnorm_f32(float* x, const float* d, const float* w,
                                         float* out, int rows, int dim, float eps,
                                         hipStream_t stream) {
    return rmsnorm_dispatch<float, true>(x, d, w, out, rows, dim, eps, stream);
}

extern "C" hipError_t ql_add_rmsnorm_f16(uint16_t* x, const uint16_t* d, const uint16_t* w,
                                         uint16_t* out, int rows, int dim, float eps,
                                         hipStream_t stream) {
    return rmsnorm_dispatch<_Float16, true>(
        reinterpret_cast<_Float16*>(x), reinterpret_cast<const _Float16*>(d),
        reinterpret_cast<const _Float16*>(w), reinterpret_cast<_Float16*>(out), rows, dim,
        eps, stream);
}
