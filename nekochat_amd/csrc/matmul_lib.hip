// The plain F16 weight matmul at prefill sizes on hipBLASLt, the vendor GEMM library -- the one case
// where a library kernel measured faster than this library's own MFMA kernels (Qwen3-4B prefill,
// T = 8192, f32 output: q/k/v 226 vs 263 us, o 156 vs 212, gate/up 719 vs 833, down 342 vs 457).
// y[t][n] (+)= x[t] . W[n] (+ bias[n]) is the column-major product D = op(A) B (+ C) with
//   A = the weight rows: row-major [N][K] = column-major K x N (lda = row_bytes / 2), op(A) = A^T;
//   B = the activations: row-major [T][K] = column-major K x T (ldb = x_stride);
//   D = y: row-major [T][N] = column-major N x T (ldd = y_stride), f32 or f16;
// NEKO_MM_ACCUMULATE as beta = 1 with C = D; the bias through the library's bias epilogue. The
// products are exact (f16 x f16) and summed in f32 in the library's order, so the results meet the
// same bound as the own kernels' (a different order of the same f32 sum). GELU, FP8 / FP4 rows, f32
// activations, decode sizes and the allocation-free entry point keep the own kernels.
#include <hipblaslt/hipblaslt.h>

#include <array>
#include <map>

#include "internal.h"

namespace neko_hip {

namespace {

// One product shape's descriptors and chosen algorithm.
struct LtPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
    bool ok = false;  // false: the library has no algorithm for it (the own kernels run)
};

// Workspace the library may use per call (its stream-K kernels keep partial tiles there).
constexpr size_t kLtMaxWorkspace = size_t{64} << 20;

void destroy_plan(LtPlan& p) {
    if (p.desc) (void)hipblasLtMatmulDescDestroy(p.desc);
    if (p.a) (void)hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) (void)hipblasLtMatrixLayoutDestroy(p.b);
    if (p.d) (void)hipblasLtMatrixLayoutDestroy(p.d);
    p = LtPlan{};
}

}  // namespace

struct LtState {
    hipblasLtHandle_t handle = nullptr;
    bool failed = false;  // the handle could not be created: never try again on this context
    // key: T, N, K, lda, ldb, ldd, y_dtype, bias, accumulate
    std::map<std::array<int64_t, 9>, LtPlan> plans;
};

void lt_release(neko_hip_ctx* ctx) {
    if (!ctx->lt) return;
    for (auto& kv : ctx->lt->plans) destroy_plan(kv.second);
    if (ctx->lt->handle) (void)hipblasLtDestroy(ctx->lt->handle);
    delete ctx->lt;
    ctx->lt = nullptr;
}

namespace {

#define LT_TRY(call)                                          \
    do {                                                      \
        if ((call) != HIPBLAS_STATUS_SUCCESS) return false;   \
    } while (0)

bool make_plan(hipblasLtHandle_t h, LtPlan& p, int64_t T, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldd,
               int y_dtype, bool bias) {
    const hipDataType yt = y_dtype == NEKO_DT_F16 ? HIP_R_16F : HIP_R_32F;
    LT_TRY(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    LT_TRY(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
    LT_TRY(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
    if (bias) {
        const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
        const hipDataType bt = HIP_R_32F;
        LT_TRY(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)));
        LT_TRY(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)));
    }
    LT_TRY(hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16F, static_cast<uint64_t>(K), static_cast<uint64_t>(N), lda));
    LT_TRY(hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16F, static_cast<uint64_t>(K), static_cast<uint64_t>(T), ldb));
    LT_TRY(hipblasLtMatrixLayoutCreate(&p.d, yt, static_cast<uint64_t>(N), static_cast<uint64_t>(T), ldd));
    hipblasLtMatmulPreference_t pref = nullptr;
    LT_TRY(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t max_ws = kLtMaxWorkspace;
    hipblasLtMatmulHeuristicResult_t res[1];
    int n = 0;
    const bool found =
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &max_ws, sizeof(max_ws)) ==
            HIPBLAS_STATUS_SUCCESS &&
        hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.d, p.d, pref, 1, res, &n) == HIPBLAS_STATUS_SUCCESS &&
        n > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize <= kLtMaxWorkspace;
    (void)hipblasLtMatmulPreferenceDestroy(pref);
    if (!found) return false;
    p.algo = res[0].algo;
    p.ws = res[0].workspaceSize;
    return true;
}

}  // namespace

int lt_matmul(neko_hip_ctx* ctx, const void* x, int64_t x_stride, int64_t T, int64_t K, const void* w, int64_t row_bytes,
              int64_t N, const float* bias, void* y, int64_t y_stride, int flags, int y_dtype, bool* done) {
    *done = false;
    if (!ctx->lt) ctx->lt = new LtState;
    LtState& s = *ctx->lt;
    if (s.failed) return NEKO_OK;
    if (!s.handle && hipblasLtCreate(&s.handle) != HIPBLAS_STATUS_SUCCESS) {
        s.handle = nullptr;
        s.failed = true;
        return NEKO_OK;
    }
    const bool has_bias = bias != nullptr, acc = (flags & NEKO_MM_ACCUMULATE) != 0;
    const int64_t lda = row_bytes / 2;
    const std::array<int64_t, 9> key{T, N, K, lda, x_stride, y_stride, y_dtype, has_bias, acc};
    auto it = s.plans.find(key);
    if (it == s.plans.end()) {
        LtPlan p;
        p.ok = make_plan(s.handle, p, T, N, K, lda, x_stride, y_stride, y_dtype, has_bias);
        if (!p.ok) destroy_plan(p);
        it = s.plans.emplace(key, p).first;
    }
    LtPlan& p = it->second;
    if (!p.ok) return NEKO_OK;
    void* ws = nullptr;
    if (p.ws > 0)
        if (int rc = workspace(ctx, p.ws, &ws, 0)) return rc;
    if (has_bias &&
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)) !=
            HIPBLAS_STATUS_SUCCESS)
        return fail(ctx, NEKO_ERR_HIP, "neko_hip_matmul: hipblasLtMatmulDescSetAttribute(bias) failed");
    const float alpha = 1.0f, beta = acc ? 1.0f : 0.0f;
    const hipblasStatus_t st =
        hipblasLtMatmul(s.handle, p.desc, &alpha, w, p.a, x, p.b, &beta, y, p.d, y, p.d, &p.algo, ws, p.ws, ctx->stream);
    if (st != HIPBLAS_STATUS_SUCCESS)
        return fail(ctx, NEKO_ERR_HIP, "neko_hip_matmul: hipblasLtMatmul failed (status %d)", static_cast<int>(st));
    *done = true;
    return after_launch(ctx, "neko_hip_matmul");
}

}  // namespace neko_hip
