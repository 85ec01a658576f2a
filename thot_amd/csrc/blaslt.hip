// Plain GEMMs through hipBLASLt.  The Linear forward and its two gradient
// products are library GEMMs (no gathers, no fused epilogue beyond a bias),
// so they go to the vendor GEMM; the fused and gathering GEMMs (implicit
// convolutions, the column path's layout epilogues, split-K partial stores)
// stay on the hand-written kernels.  One handle, one 32 MiB workspace and a
// plan cache (descriptor, layouts, heuristic algorithm per shape) per
// context.
#include "common.hpp"
#include "blaslt.hpp"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>

namespace nott {
namespace blas {
namespace {

constexpr size_t kWsBytes = 32u << 20;

using Key = std::tuple<int, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int, int, int, int64_t, int64_t,
                       int64_t, int64_t>;

struct Plan {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
};

struct State {
    hipblasLtHandle_t h = nullptr;
    void* ws = nullptr;
    bool broken = false;
    std::map<Key, Plan> plans;
};

State* state(nott_ctx ctx) {
    if (!ctx->blas) {
        State* s = new State();
        if (hipblasLtCreate(&s->h) != HIPBLAS_STATUS_SUCCESS || hipMalloc(&s->ws, kWsBytes) != hipSuccess) {
            s->broken = true;
        }
        ctx->blas = s;
    }
    return static_cast<State*>(ctx->blas);
}

void destroy_plan(Plan& p) {
    if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
    if (p.d) hipblasLtMatrixLayoutDestroy(p.d);
    if (p.op) hipblasLtMatmulDescDestroy(p.op);
}

Plan make_plan(State* s, bool ta, bool tb, int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldd,
               hipDataType ab, hipDataType dt, bool bias, int64_t batch, int64_t sa, int64_t sb, int64_t sd) {
    Plan p;
    if (hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return p;
    const int32_t opa = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N, opb = tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa));
    hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof(opb));
    if (bias) {
        const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
        const int32_t bt = HIP_R_32F;
        hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi));
        hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt));
    }
    // Column-major layouts: op(A) is m×k, op(B) is k×n, D is m×n.
    if (hipblasLtMatrixLayoutCreate(&p.a, ab, ta ? k : m, ta ? m : k, lda) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.b, ab, tb ? n : k, tb ? k : n, ldb) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p.d, dt, m, n, ldd) != HIPBLAS_STATUS_SUCCESS)
        return p;
    if (batch > 1) {
        const int32_t bc = (int32_t)batch;
        const int64_t strides[3] = {sa, sb, sd};
        hipblasLtMatrixLayout_t ls[3] = {p.a, p.b, p.d};
        for (int i = 0; i < 3; ++i) {
            hipblasLtMatrixLayoutSetAttribute(ls[i], HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc));
            hipblasLtMatrixLayoutSetAttribute(ls[i], HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &strides[i],
                                              sizeof(strides[i]));
        }
    }
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return p;
    const uint64_t wsb = kWsBytes;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
    hipblasLtMatmulHeuristicResult_t res[1];
    int got = 0;
    const hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(s->h, p.op, p.a, p.b, p.d, p.d, pref, 1, res, &got);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st == HIPBLAS_STATUS_SUCCESS && got > 0) {
        p.algo = res[0].algo;
        p.ok = true;
    }
    return p;
}

}  // namespace

int gemm(nott_ctx ctx, bool ta, bool tb, int64_t m, int64_t n, int64_t k, const void* A, int64_t lda, const void* B,
         int64_t ldb, hipDataType ab, void* D, int64_t ldd, hipDataType dt, float beta, const float* bias, int64_t batch,
         int64_t sa, int64_t sb, int64_t sd) {
    if (m <= 0 || n <= 0 || k <= 0 || batch <= 0 || batch > 0x7fffffff) return NOTT_ERR_UNSUPPORTED;
    State* s = state(ctx);
    if (s->broken) return NOTT_ERR_UNSUPPORTED;
    const Key key{ta, tb, m, n, k, lda, ldb, ldd, (int)ab, (int)dt, bias != nullptr, batch, sa, sb, sd};
    auto it = s->plans.find(key);
    if (it == s->plans.end())
        it = s->plans.emplace(key, make_plan(s, ta, tb, m, n, k, lda, ldb, ldd, ab, dt, bias != nullptr, batch, sa, sb,
                                             sd)).first;
    Plan& p = it->second;
    if (!p.ok) return NOTT_ERR_UNSUPPORTED;
    if (bias) hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
    const float alpha = 1.f;
    const hipblasStatus_t st = hipblasLtMatmul(s->h, p.op, &alpha, A, p.a, B, p.b, &beta, D, p.d, D, p.d, &p.algo,
                                               s->ws, kWsBytes, ctx->stream);
    if (st != HIPBLAS_STATUS_SUCCESS) return fail(ctx, NOTT_ERR_HIP, "hipblasLtMatmul failed");
    return launch_status(ctx, "hipblasLt gemm");
}

void release(nott_ctx ctx) {
    if (!ctx->blas) return;
    State* s = static_cast<State*>(ctx->blas);
    for (auto& kv : s->plans) destroy_plan(kv.second);
    if (s->h) hipblasLtDestroy(s->h);
    if (s->ws) (void)hipFree(s->ws);
    delete s;
    ctx->blas = nullptr;
}

}  // namespace blas
}  // namespace nott
