// gemm.cpp -- the fp16 library GEMM used by the layer engine and the FP8 GEMM's
// large-M path: y[M, N] = x[M, K] W[N, K]^T (row-major, weights [out, in]),
// fp16 in/out, fp32 accumulation, on hipBLASLt.
//
// Column-major view for the library: y^T (N x M) = op(A) op(B) with A = W stored
// K x N and transposed, B = x stored K x M.  Plans (descriptors + the heuristic's
// first algorithm) are cached per (device, M, N, K); each (device, stream) pair
// gets its own workspace so GEMMs on different streams never share one.  The
// handle, plans and workspaces are created on first use and live until the
// process ends.  ql_gemm_tune_f16 replaces a shape's algorithm by the fastest of
// the heuristic's candidates, timed on scratch operands.
#include "quantlib_amd.h"

#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <chrono>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

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

constexpr int kTuneCandidates = 32;      // heuristic results timed by ql_gemm_tune_f16
constexpr size_t kTuneWeightBytes = 512u << 20;   // rotated weight copies: past the MALL
constexpr int kTuneMaxCopies = 8;
constexpr int kTuneReps = 10;
constexpr int kTuneFinalists = 4;       // re-timed with the heuristic's first choice
constexpr int kTuneRounds = 3;
constexpr double kTuneMargin = 0.03;    // a replacement must be this much faster

// The heuristic's first `want` algorithms for a plan's descriptors that fit the workspace.
hipError_t candidates(Device& d, const Plan& p, int want,
                      std::vector<hipblasLtMatmulHeuristicResult_t>& out) {
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return hipErrorUnknown;
    const uint64_t ws = kWorkspace;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    std::vector<hipblasLtMatmulHeuristicResult_t> res((size_t)want);
    int n = 0;
    const hipblasStatus_t st =
        hipblasLtMatmulAlgoGetHeuristic(d.lt, p.desc, p.a, p.b, p.c, p.c, pref, want, res.data(), &n);
    hipblasLtMatmulPreferenceDestroy(pref);
    out.clear();
    if (st != HIPBLAS_STATUS_SUCCESS) return hipErrorNotSupported;
    for (int i = 0; i < n; ++i)
        if (res[(size_t)i].workspaceSize <= kWorkspace) out.push_back(res[(size_t)i]);
    return out.empty() ? hipErrorNotSupported : hipSuccess;
}

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
    std::vector<hipblasLtMatmulHeuristicResult_t> res;
    const hipError_t e = candidates(d, p, 1, res);
    if (e != hipSuccess) return e;
    p.algo = res[0].algo;
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

namespace {

// Scratch device memory of the tuner, released on every return path.
struct Scratch {
    void* p = nullptr;
    ~Scratch() {
        if (p) (void)hipFree(p);
    }
};

// Waits for the stream when it leaves scope (before the scratch it uses is freed).
struct StreamDrain {
    hipStream_t s;
    ~StreamDrain() { (void)hipStreamSynchronize(s); }
};

}  // namespace

extern "C" hipError_t ql_gemm_tune_f16(int M, int N, int K, hipStream_t stream) {
    if (M <= 0 || N <= 0 || K <= 0) return hipErrorInvalidValue;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return hipErrorNoDevice;
    Plan plan;
    hipblasLtHandle_t lt = nullptr;
    std::vector<hipblasLtMatmulHeuristicResult_t> cands;
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
        lt = d.lt;
        const hipError_t e = candidates(d, plan, kTuneCandidates, cands);
        if (e != hipSuccess) return e;
    }
    // operands: x, y, and enough weight copies that each timed launch streams its
    // weights from HBM, as in a multi-layer step
    const size_t xb = (size_t)M * K * 2, yb = (size_t)M * N * 2, wb = (size_t)N * K * 2;
    const int copies = (int)std::min<size_t>(kTuneMaxCopies, std::max<size_t>(1, (kTuneWeightBytes + wb - 1) / wb));
    Scratch xs, ys, ws_, wks;
    hipError_t e = hipMalloc(&xs.p, xb);
    if (e == hipSuccess) e = hipMalloc(&ys.p, yb);
    if (e == hipSuccess) e = hipMalloc(&ws_.p, wb * (size_t)copies);
    if (e == hipSuccess) e = hipMalloc(&wks.p, kWorkspace);
    if (e != hipSuccess) return e;
    const StreamDrain drain{stream};   // destroyed first: nothing in flight when the scratch is freed
    // small binary16 values (0x1111 = 6.5e-4): finite products and sums
    if ((e = hipMemsetAsync(xs.p, 0x11, xb, stream)) != hipSuccess) return e;
    if ((e = hipMemsetAsync(ws_.p, 0x11, wb * (size_t)copies, stream)) != hipSuccess) return e;
    const float alpha = 1.0f, beta = 0.0f;
    auto run = [&](const hipblasLtMatmulAlgo_t& algo, int i) {
        const char* w = static_cast<const char*>(ws_.p) + (size_t)(i % copies) * wb;
        return hipblasLtMatmul(lt, plan.desc, &alpha, w, plan.a, xs.p, plan.b, &beta, ys.p, plan.c, ys.p,
                               plan.c, &algo, wks.p, kWorkspace, stream) == HIPBLAS_STATUS_SUCCESS;
    };
    // time one candidate: kTuneReps launches over the weight copies, host wall clock
    // from the first launch to the stream's completion, so a candidate that launches
    // more kernels (e.g. a split-K reduction) pays their launch cost (-1: unsupported)
    auto time_of = [&](const hipblasLtMatmulAlgo_t& algo, float& ms) -> hipError_t {
        ms = -1.0f;
        if (!run(algo, 0) || !run(algo, 1)) return hipSuccess;   // warm-up; unsupported: skip
        hipError_t r = hipStreamSynchronize(stream);
        if (r != hipSuccess) return r;
        const auto t0 = std::chrono::steady_clock::now();
        bool ok = true;
        for (int i = 0; i < kTuneReps && ok; ++i) ok = run(algo, i + 2);
        if ((r = hipStreamSynchronize(stream)) != hipSuccess) return r;
        const auto t1 = std::chrono::steady_clock::now();
        if (ok) ms = std::chrono::duration<float, std::milli>(t1 - t0).count();
        return hipSuccess;
    };
    // first pass over every candidate, then the fastest few and the heuristic's
    // first choice again in alternating rounds; the first choice is kept unless
    // another one is faster by more than kTuneMargin over the rounds
    std::vector<std::pair<float, int>> first;
    for (int i = 0; i < (int)cands.size(); ++i) {
        float ms;
        if ((e = time_of(cands[(size_t)i].algo, ms)) != hipSuccess) return e;
        if (ms >= 0.0f) first.emplace_back(ms, i);
    }
    if (first.empty()) return hipErrorNotSupported;
    std::sort(first.begin(), first.end());
    std::vector<int> finalists = {0};
    for (size_t i = 0; i < first.size() && finalists.size() < (size_t)kTuneFinalists + 1; ++i)
        if (first[i].second != 0) finalists.push_back(first[i].second);
    std::vector<double> total(finalists.size(), 0.0);
    std::vector<bool> valid(finalists.size(), true);
    for (int round = 0; round < kTuneRounds; ++round)
        for (size_t f = 0; f < finalists.size(); ++f) {
            float ms;
            if ((e = time_of(cands[(size_t)finalists[f]].algo, ms)) != hipSuccess) return e;
            if (ms < 0.0f) valid[f] = false;
            total[f] += ms;
        }
    size_t pick = 0;
    for (size_t f = 1; f < finalists.size(); ++f)
        if (valid[f] && (!valid[pick] || total[f] < total[pick])) pick = f;
    if (pick != 0 && valid[0] && total[pick] * (1.0 + kTuneMargin) > total[0]) pick = 0;
    const float best = valid[pick] ? (float)total[pick] : -1.0f;
    const hipblasLtMatmulAlgo_t best_algo = cands[(size_t)finalists[pick]].algo;
    if (best < 0.0f) return hipErrorNotSupported;
    std::lock_guard<std::mutex> lock(g_mu);
    g_devices[dev].plans[std::make_tuple(M, N, K)].algo = best_algo;
    return hipSuccess;
}
