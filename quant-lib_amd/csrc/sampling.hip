// sampling.hip -- greedy token selection over rows of logits.
//
// argmax_kernel (src/continuous_batch.cu:12-25) picks, for one row, the first
// index whose value is strictly greater than every earlier one and than the
// start value -1e20f (:15); NaN never compares greater, and a row with nothing
// above -1e20f gives 0.  (The fp16 engine's argmax_kernel,
// src/fp16_forward.cu:259-283, starts from -FLT_MAX instead: the two agree on
// every row that holds a value above -1e20f, which every binary16 row with a
// finite value does.)  Here one workgroup handles one
// row of a batch: each lane keeps its first strict maximum over a strided pass
// (16-byte loads when the row allows), then (value, index) pairs are reduced
// preferring the larger value and, on equal values, the smaller index -- the
// same answer as the sequential scan.
#include "ql_common.hpp"
#include "quantlib_amd.h"

#include <math.h>
#include <limits.h>

namespace {

using namespace ql;

constexpr float kStart = -1e20f;   // src/continuous_batch.cu:15

__device__ __forceinline__ void better(float& v, int& i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

template <typename D, bool VEC>
__global__ __launch_bounds__(kBlock) void argmax_rows(const D* __restrict__ x, int cols, int64_t ld,
                                                      int32_t* __restrict__ out) {
    const D* row = x + (size_t)blockIdx.x * (size_t)ld;
    float best = kStart;
    int idx = INT_MAX;   // none yet
    if constexpr (VEC) {
        constexpr int W = vec16<D>();
        const int nv = cols / W;
        for (int c = threadIdx.x; c < nv; c += kBlock) {
            const Vec<D, W> v = load<true>(reinterpret_cast<const Vec<D, W>*>(row) + c);
#pragma unroll
            for (int e = 0; e < W; ++e) {
                const float f = to_f32(v.v[e]);
                if (f > best) {
                    best = f;
                    idx = c * W + e;
                }
            }
        }
        for (int c = nv * W + threadIdx.x; c < cols; c += kBlock) {
            const float f = to_f32(row[c]);
            if (f > best) {
                best = f;
                idx = c;
            }
        }
    } else {
        for (int c = threadIdx.x; c < cols; c += kBlock) {
            const float f = to_f32(row[c]);
            if (f > best) {
                best = f;
                idx = c;
            }
        }
    }
    // lanes that saw nothing above the start keep (kStart, INT_MAX) and never win a tie
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(best, o, kWave);
        const int i2 = __shfl_xor(idx, o, kWave);
        better(best, idx, v2, i2);
    }
    __shared__ float sv[kBlock / kWave];
    __shared__ int si[kBlock / kWave];
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        sv[wave] = best;
        si[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kBlock / kWave; ++w) better(best, idx, sv[w], si[w]);
        out[blockIdx.x] = idx == INT_MAX ? 0 : idx;
    }
}

template <typename D>
hipError_t argmax_launch(const D* x, int rows, int cols, int64_t ld, int32_t* out,
                         hipStream_t stream) {
    QL_CHECK_ARG(rows >= 0 && cols > 0 && ld >= cols && rows <= 0x7fffffff);
    if (rows == 0) return hipSuccess;
    QL_CHECK_ARG(x && out);
    const bool vec = qlh::aligned16(x) && (ld * (int64_t)sizeof(D)) % 16 == 0;
    if (vec) {
        hipLaunchKernelGGL((argmax_rows<D, true>), dim3(rows), dim3(kBlock), 0, stream, x, cols, ld, out);
    } else {
        hipLaunchKernelGGL((argmax_rows<D, false>), dim3(rows), dim3(kBlock), 0, stream, x, cols, ld, out);
    }
    return hipGetLastError();
}

}  // namespace

extern "C" hipError_t ql_argmax_f32(const float* logits, int rows, int cols, int64_t ld,
                                    int32_t* out, hipStream_t stream) {
    return argmax_launch<float>(logits, rows, cols, ld, out, stream);
}

extern "C" hipError_t ql_argmax_f16(const uint16_t* logits, int rows, int cols, int64_t ld,
                                    int32_t* out, hipStream_t stream) {
    return argmax_launch<_Float16>(reinterpret_cast<const _Float16*>(logits), rows, cols, ld, out,
                                   stream);
}
