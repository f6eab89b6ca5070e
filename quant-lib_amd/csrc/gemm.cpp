// gemm.cpp -- the fp16 library GEMM used by the layer engine and the FP8 GEMM's
// large-M path: y[M, N] = x[M, K] W[N, K]^T (row-major, weights [out, in]),
// fp16 in/out, fp32 accumulation, on hipBLASLt.
//
// Column-major view for the library: y^T (N x M) = op(A) op(B) with A = W stored
// K x N and transposed, B = x stored K x M.  Plans (descriptors + the heuristic's
// first algorithm) are cached per (device, M, N, K); each (device, stream) pair
// gets its own workspace so GEMMs on different streams never share one.  The
// handle, plans and workspaces are created on first use and live until the
// process ends.
#include "quantlib_amd.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace {

constexpr size_t kWorkspace = 64u << 20;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

struct Device {
    hipblasLtHandle_t lt = nullptr;
    std::map<std::tuple<int, int, int>, Plan> plans;
    std::map<hipStream_t, void*> workspaces;
};

std::mutex g_mu;
std::map<int, Device> g_devices;

hipError_t make_plan(Device& d, int M, int N, int K, Plan& p) {
    const hipblasOperation_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
    if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
        return hipErrorUnknown;
    if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16F, (uint64_t)K, (uint64_t)N, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16F, (uint64_t)K, (uint64_t)M, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.c, HIP_R_16F, (uint64_t)N, (uint64_t)M, N) != HIPBLAS_STATUS_SUCCESS)
        return hipErrorUnknown;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return hipErrorUnknown;
    const uint64_t ws = kWorkspace;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    hipblasLtMatmulHeuristicResult_t res{};
    int n = 0;
    const hipblasStatus_t st =
        hipblasLtMatmulAlgoGetHeuristic(d.lt, p.desc, p.a, p.b, p.c, p.c, pref, 1, &res, &n);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || n < 1 || res.workspaceSize > kWorkspace) return hipErrorNotSupported;
    p.algo = res.algo;
    return hipSuccess;
}

}  // namespace

extern "C" hipError_t ql_gemm_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, int M, int N,
                                  int K, hipStream_t stream) {
    if (M < 0 || N < 0 || K < 0) return hipErrorInvalidValue;
    if (M == 0 || N == 0) return hipSuccess;
    if (!x || !w || !y || K == 0) return hipErrorInvalidValue;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return hipErrorNoDevice;
    Plan plan;
    void* ws = nullptr;
    hipblasLtHandle_t lt = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        Device& d = g_devices[dev];
        if (!d.lt && hipblasLtCreate(&d.lt) != HIPBLAS_STATUS_SUCCESS) {
            d.lt = nullptr;
            return hipErrorNotInitialized;
        }
        auto key = std::make_tuple(M, N, K);
        auto it = d.plans.find(key);
        if (it == d.plans.end()) {
            Plan p;
            const hipError_t e = make_plan(d, M, N, K, p);
            if (e != hipSuccess) return e;
            it = d.plans.emplace(key, p).first;
        }
        plan = it->second;
        void*& slot = d.workspaces[stream];
        if (!slot && hipMalloc(&slot, kWorkspace) != hipSuccess) {
            slot = nullptr;
            return hipErrorOutOfMemory;
        }
        ws = slot;
        lt = d.lt;
    }
    const float alpha = 1.0f, beta = 0.0f;
    const hipblasStatus_t st = hipblasLtMatmul(lt, plan.desc, &alpha, w, plan.a, x, plan.b, &beta, y, plan.c,
                                               y, plan.c, &plan.algo, ws, kWorkspace, stream);
    return st == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorLaunchFailure;
}
