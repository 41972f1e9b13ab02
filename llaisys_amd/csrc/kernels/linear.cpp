// Y = X W^T (+ bias) (+ Y) through the library GEMM (weights in the
// reference's [out_features, in_features] row-major layout, README.md:195-210).
//
// Row-major Y[M,N] = X[M,K] W[N,K]^T is, read column-major, Y^T = W^T' X^T'
// with W's buffer as a K x N column-major matrix used transposed and X's as
// K x M used as is: one "TN" GEMM, m = N, n = M, k = K, fp32 accumulation.
//
// hipBLASLt runs it, with the bias as its BIAS epilogue (added before the one
// rounding) and the residual as C = D, beta = 1. For decode-sized M the
// library's first heuristic choice is often not its fastest kernel for these
// skinny shapes, so the first call of each (dtype, M, N, K, bias) times the
// top candidates on the caller's stream (into a scratch output, each run
// after a 512 MiB write that evicts the weights from L2 and the MALL, as a
// model's layers see them) and keeps the fastest. LLAISYS_GEMM_AUTOTUNE=0, or
// a stream under graph capture, keeps the first choice. rocBLAS is the
// fallback when hipBLASLt offers no kernel.
#include "launch.hpp"

#include "../common.hpp"
#include "../device/hip_check.hpp"

#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>

#include <cstdlib>
#include <map>
#include <memory>
#include <tuple>
#include <unordered_map>
#include <vector>

namespace llaisys::kernels {

namespace {

#define ROCBLAS_CHECK(expr)                                                                  \
    do {                                                                                     \
        rocblas_status s__ = (expr);                                                         \
        if (s__ != rocblas_status_success) LLAISYS_RAISE("rocBLAS error " << rocblas_status_to_string(s__) << " from " #expr); \
    } while (0)

#define LT_CHECK(expr)                                                                       \
    do {                                                                                     \
        hipblasStatus_t s__ = (expr);                                                        \
        if (s__ != HIPBLAS_STATUS_SUCCESS) LLAISYS_RAISE("hipBLASLt error " << int(s__) << " from " #expr); \
    } while (0)

constexpr int kTuneMaxM = 256;          // autotune decode-sized GEMMs only
constexpr int kTuneCandidates = 16;      // heuristic candidates timed per shape
constexpr int kTuneCandidatesWide = 64;  // ... for weight matrices of >= kWideElems elements
constexpr long long kWideElems = 1 << 20;
constexpr size_t kWorkspaceBytes = 32u << 20;
constexpr size_t kFlushBytes = size_t(512) << 20;   // > L2 + MALL

int currentDevice() {
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    return dev;
}

// One rocBLAS handle per (thread, device); never destroyed (handles outlive any
// thread-exit ordering against the HIP runtime's own teardown).
rocblas_handle rocblasHandle() {
    thread_local std::unordered_map<int, rocblas_handle> handles;
    const int dev = currentDevice();
    auto it = handles.find(dev);
    if (it != handles.end()) return it->second;
    rocblas_handle h = nullptr;
    ROCBLAS_CHECK(rocblas_create_handle(&h));
    handles.emplace(dev, h);
    return h;
}

rocblas_datatype rocType(ElemType t) {
    switch (t) {
    case ElemType::F32: return rocblas_datatype_f32_r;
    case ElemType::F16: return rocblas_datatype_f16_r;
    case ElemType::BF16: return rocblas_datatype_bf16_r;
    }
    return rocblas_datatype_f32_r;
}

hipDataType ltType(ElemType t) {
    switch (t) {
    case ElemType::F32: return HIP_R_32F;
    case ElemType::F16: return HIP_R_16F;
    case ElemType::BF16: return HIP_R_16BF;
    }
    return HIP_R_32F;
}

size_t elemBytes(ElemType t) { return t == ElemType::F32 ? 4 : 2; }

// A prepared GEMM: descriptors plus the chosen kernel (ok == false: use rocBLAS).
struct LtGemm {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
};

// Per (thread, device): handle, workspace, tuning scratch, prepared GEMMs.
// Kept for the life of the thread (like the rocBLAS handle).
struct LtContext {
    hipblasLtHandle_t handle = nullptr;
    void *workspace = nullptr;
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    std::map<std::tuple<int, int, int, int, bool>, LtGemm> gemms;
    // Autotuned kernel per (type, M bucket, N, K, bias): a serving loop sees
    // a new M almost every step, and each exact shape reuses its bucket's pick.
    std::map<std::tuple<int, int, int, int, bool>, hipblasLtMatmulAlgo_t> tuned;
};

// M buckets of the autotune: the next power of two.
int tuneBucket(int M) {
    int b = 1;
    while (b < M) b <<= 1;
    return b;
}

LtContext &ltContext() {
    thread_local std::unordered_map<int, std::unique_ptr<LtContext>> contexts;
    const int dev = currentDevice();
    auto &ctx = contexts[dev];
    if (!ctx) {
        ctx = std::make_unique<LtContext>();
        LT_CHECK(hipblasLtCreate(&ctx->handle));
        HIP_CHECK(hipMalloc(&ctx->workspace, kWorkspaceBytes));
    }
    return *ctx;
}

bool autotuneEnabled() {
    const char *e = std::getenv("LLAISYS_GEMM_AUTOTUNE");
    return !(e && e[0] == '0');
}

void runLt(LtContext &ctx, const LtGemm &g, const hipblasLtMatmulAlgo_t &algo, void *y, const void *x, const void *w,
           float beta, hipStream_t s) {
    const float alpha = 1.f;
    LT_CHECK(hipblasLtMatmul(ctx.handle, g.desc, &alpha, w, g.a, x, g.b, &beta, y, g.c, y, g.c, &algo, ctx.workspace,
                             kWorkspaceBytes, s));
}

LtGemm &prepare(LtContext &ctx, ElemType t, int M, int N, int K, const void *bias, const void *x, const void *w,
                hipStream_t s) {
    const auto key = std::make_tuple(int(t), M, N, K, bias != nullptr);
    auto found = ctx.gemms.find(key);
    if (found != ctx.gemms.end()) return found->second;
    LtGemm &g = ctx.gemms[key];
    const hipDataType dt = ltType(t);
    LT_CHECK(hipblasLtMatmulDescCreate(&g.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    LT_CHECK(hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
    LT_CHECK(hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
    if (bias) {
        const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
        LT_CHECK(hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)));
        LT_CHECK(hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &dt, sizeof(dt)));
        // the pointer is set per call
    }
    LT_CHECK(hipblasLtMatrixLayoutCreate(&g.a, dt, K, N, K));
    LT_CHECK(hipblasLtMatrixLayoutCreate(&g.b, dt, K, M, K));
    LT_CHECK(hipblasLtMatrixLayoutCreate(&g.c, dt, N, M, N));
    hipblasLtMatmulPreference_t pref = nullptr;
    LT_CHECK(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t wsz = kWorkspaceBytes;
    LT_CHECK(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz, sizeof(wsz)));
    // The large decode-step weight GEMMs search wider (measured 4.5 % faster
    // for the Qwen2-1.5B step); small shapes keep the short list.
    const int want = (long long)N * K >= kWideElems ? kTuneCandidatesWide : kTuneCandidates;
    std::vector<hipblasLtMatmulHeuristicResult_t> res(want);
    int got = 0;
    const hipblasStatus_t hs = hipblasLtMatmulAlgoGetHeuristic(ctx.handle, g.desc, g.a, g.b, g.c, g.c, pref, want,
                                                               res.data(), &got);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (hs != HIPBLAS_STATUS_SUCCESS || got <= 0) return g; // rocBLAS fallback
    // Only candidates the library confirms for this problem and workspace run.
    std::vector<hipblasLtMatmulAlgo_t> algos;
    for (int i = 0; i < got; ++i) {
        if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > kWorkspaceBytes) continue;
        const float one = 1.f;
        size_t need = 0;
        if (hipblaslt_ext::matmulIsAlgoSupported(ctx.handle, g.desc, &one, g.a, g.b, &one, g.c, g.c, res[i].algo,
                                                 need) != HIPBLAS_STATUS_SUCCESS ||
            need > kWorkspaceBytes)
            continue;
        algos.push_back(res[i].algo);
    }
    if (algos.empty()) return g; // rocBLAS fallback
    g.algo = algos[0];
    g.ok = true;
    got = int(algos.size());
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    HIP_CHECK(hipStreamIsCapturing(s, &capture));
    if (got == 1 || M > kTuneMaxM || !autotuneEnabled()) return g;
    const auto bucket = std::make_tuple(int(t), tuneBucket(M), N, K, bias != nullptr);
    auto pick = ctx.tuned.find(bucket);
    if (pick != ctx.tuned.end()) {
        // The bucket's pick, if the library confirms it for this exact shape.
        const float one = 1.f;
        size_t need = 0;
        hipblasLtMatmulAlgo_t a = pick->second;
        if (hipblaslt_ext::matmulIsAlgoSupported(ctx.handle, g.desc, &one, g.a, g.b, &one, g.c, g.c, a, need) ==
                HIPBLAS_STATUS_SUCCESS &&
            need <= kWorkspaceBytes)
            g.algo = a;
        return g;
    }
    if (capture != hipStreamCaptureStatusNone) return g;

    // Time the candidates into a scratch output (the caller's Y, possibly a
    // residual being accumulated, is not touched), each run from cold caches.
    const size_t ybytes = size_t(M) * N * elemBytes(t);
    if (ybytes > ctx.scratch_bytes) {
        HIP_CHECK(hipStreamSynchronize(s));
        if (ctx.scratch) HIP_CHECK(hipFree(ctx.scratch));
        HIP_CHECK(hipMalloc(&ctx.scratch, ybytes));
        ctx.scratch_bytes = ybytes;
    }
    void *flush = nullptr;
    HIP_CHECK(hipMalloc(&flush, kFlushBytes));
    if (bias)
        LT_CHECK(hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)));
    constexpr int kReps = 3;
    hipEvent_t ev[2 * kReps];
    for (auto &e : ev) HIP_CHECK(hipEventCreate(&e));
    float best = 1e30f;
    for (int i = 0; i < got; ++i) {
        const float alpha = 1.f, beta = 0.f;
        if (hipblasLtMatmul(ctx.handle, g.desc, &alpha, w, g.a, x, g.b, &beta, ctx.scratch, g.c, ctx.scratch, g.c,
                            &algos[i], ctx.workspace, kWorkspaceBytes, s) != HIPBLAS_STATUS_SUCCESS)
            continue;
        for (int r = 0; r < kReps; ++r) {
            HIP_CHECK(hipMemsetAsync(flush, r, kFlushBytes, s));
            HIP_CHECK(hipEventRecord(ev[2 * r], s));
            runLt(ctx, g, algos[i], ctx.scratch, x, w, 0.f, s);
            HIP_CHECK(hipEventRecord(ev[2 * r + 1], s));
        }
        HIP_CHECK(hipEventSynchronize(ev[2 * kReps - 1]));
        float total = 0.f;
        for (int r = 0; r < kReps; ++r) {
            float ms = 0.f;
            HIP_CHECK(hipEventElapsedTime(&ms, ev[2 * r], ev[2 * r + 1]));
            total += ms;
        }
        if (total < best) {
            best = total;
            g.algo = algos[i];
        }
    }
    for (auto &e : ev) HIP_CHECK(hipEventDestroy(e));
    HIP_CHECK(hipStreamSynchronize(s));
    HIP_CHECK(hipFree(flush));
    ctx.tuned[bucket] = g.algo;
    return g;
}

} // namespace

void linear(void *y, const void *x, const void *w, const void *bias, ElemType t, int M, int N, int K, void *stream,
            bool accumulate) {
    if (M == 0 || N == 0) return;
    auto s = static_cast<hipStream_t>(stream);
    LtContext &ctx = ltContext();
    LtGemm &g = prepare(ctx, t, M, N, K, bias, x, w, s);
    if (g.ok) {
        if (bias)
            LT_CHECK(hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)));
        runLt(ctx, g, g.algo, y, x, w, accumulate ? 1.f : 0.f, s);
        return;
    }
    // rocBLAS: the bias enters as C (Y preset to the bias rows, beta = 1) so the
    // result is still rounded once.
    if (bias) {
        if (accumulate) {
            addBias(y, bias, t, size_t(M), size_t(N), stream);
        } else {
            fillRows(y, bias, t, size_t(M), size_t(N), stream);
        }
    }
    rocblas_handle h = rocblasHandle();
    ROCBLAS_CHECK(rocblas_set_stream(h, s));
    const float alpha = 1.f, beta = (accumulate || bias) ? 1.f : 0.f;
    const rocblas_datatype dt = rocType(t);
    ROCBLAS_CHECK(rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, N, M, K, &alpha, w, dt, K, x,
                                  dt, K, &beta, y, dt, N, y, dt, N, rocblas_datatype_f32_r, rocblas_gemm_algo_standard,
                                  0, 0));
}

} // namespace llaisys::kernels
