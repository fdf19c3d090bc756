// Plain bf16 / f16 products on hipBLASLt.
//
// A 16-bit matmul with no epilogue is a library GEMM: the reference HIP lane
// runs it on hipblasGemmEx with a binary32 compute type and a 16-bit result
// (crates/chelis-backend-hip/runtime/chelis_hip_runtime.h:92-170), and on
// gfx950 hipBLASLt's tuned kernels outrun this library's own 128-tile
// kernel on whole-chip shapes (4096^3 bf16: 0.33 of the dense peak for
// gemm16_deep_kernel). The products it takes here: one matrix (no batch
// axes), no bias, activation, residual or causal structure, the default
// mode (the exact flag keeps the tree path), each operand with one unit
// stride and a leading dimension of whole 16-byte runs, the output
// row-major. Its accumulation runs in binary32 in its own order, so the
// result stays within the bound every 16-bit product here is held to (one
// 16-bit rounding of the exact value plus the binary32 accumulation
// error); anything else, or any hipBLASLt failure, stays on the MFMA tiles.
//
// Row-major C = A B is the column-major C^T = B^T A^T: hipBLASLt's first
// operand is B as stored (N x K, or K x N transposed), its second A (K x M,
// or M x K transposed), its output C^T (N x M) with C's row pitch.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "gemm.h"

namespace chelis {
namespace {

constexpr size_t kLtWorkspace = size_t(32) << 20;
constexpr int kLtDevices = 64;

struct LtPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t lx = nullptr, ly = nullptr, ld = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
};

using LtKey = std::tuple<int, int64_t, int64_t, int64_t, int, int, int64_t, int64_t, int64_t>;

struct LtDevice {
    hipblasLtHandle_t handle = nullptr;
    void *workspace = nullptr;
    bool unusable = false;
    std::map<LtKey, LtPlan> plans;
};

std::mutex g_lt_mutex;
LtDevice g_lt[kLtDevices];

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The plan of one shape and layout: descriptors and the heuristic's first
// algorithm; ok = false when hipBLASLt offers none.
LtPlan make_plan(hipblasLtHandle_t h, hipDataType t, int64_t M, int64_t N, int64_t K, hipblasOperation_t opx,
                 hipblasOperation_t opy, int64_t ldx, int64_t ldy, int64_t ldc) {
    LtPlan pl;
    if (hipblasLtMatmulDescCreate(&pl.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return pl;
    const int32_t ox = opx, oy = opy;
    hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ox, sizeof ox);
    hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &oy, sizeof oy);
    const bool nx = opx == HIPBLAS_OP_N, ny = opy == HIPBLAS_OP_N;
    if (hipblasLtMatrixLayoutCreate(&pl.lx, t, nx ? N : K, nx ? K : N, ldx) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&pl.ly, t, ny ? K : M, ny ? M : K, ldy) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&pl.ld, t, N, M, ldc) != HIPBLAS_STATUS_SUCCESS)
        return pl;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return pl;
    const uint64_t ws = kLtWorkspace;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof ws);
    hipblasLtMatmulHeuristicResult_t res[1];
    int returned = 0;
    const hipblasStatus_t s =
        hipblasLtMatmulAlgoGetHeuristic(h, pl.desc, pl.lx, pl.ly, pl.ld, pl.ld, pref, 1, res, &returned);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (s == HIPBLAS_STATUS_SUCCESS && returned > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS &&
        res[0].workspaceSize <= kLtWorkspace) {
        pl.algo = res[0].algo;
        pl.ok = true;
    }
    return pl;
}

}  // namespace

bool gemm16_lt(chelis_dtype dt, const GemmProblem &p, hipStream_t st) {
    if (p.nb0 * p.nb1 != 1 || p.nbz || p.bias || p.act != CHELIS_ACT_NONE || p.resid || p.causal) return false;
    if (p.M < 256 || p.N < 256 || p.K < 256) return false;  // small products: the tiles' own launch is cheaper
    if (p.scn != 1 || p.scm < p.N || p.scm % 8 || !aligned16(p.c)) return false;
    hipblasOperation_t opx, opy;
    int64_t ldx, ldy;
    if (p.sbn == 1) {
        opx = HIPBLAS_OP_N, ldx = p.sbk;  // B row-major: B^T is N x K column-major
    } else if (p.sbk == 1) {
        opx = HIPBLAS_OP_T, ldx = p.sbn;  // B along K: stored K x N column-major
    } else {
        return false;
    }
    if (p.sak == 1) {
        opy = HIPBLAS_OP_N, ldy = p.sam;  // A row-major: A^T is K x M column-major
    } else if (p.sam == 1) {
        opy = HIPBLAS_OP_T, ldy = p.sak;
    } else {
        return false;
    }
    if (ldx % 8 || ldy % 8 || !aligned16(p.a) || !aligned16(p.b)) return false;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kLtDevices) return false;
    const hipDataType t = dt == CHELIS_DTYPE_BF16 ? HIP_R_16BF : HIP_R_16F;
    std::lock_guard<std::mutex> lock(g_lt_mutex);
    LtDevice &d = g_lt[device];
    if (d.unusable) return false;
    if (!d.handle) {
        if (hipblasLtCreate(&d.handle) != HIPBLAS_STATUS_SUCCESS || device_malloc(&d.workspace, kLtWorkspace) != hipSuccess) {
            d.unusable = true;
            return false;
        }
    }
    const LtKey key{(int)dt, p.M, p.N, p.K, (int)opx, (int)opy, ldx, ldy, p.scm};
    auto it = d.plans.find(key);
    if (it == d.plans.end()) it = d.plans.emplace(key, make_plan(d.handle, t, p.M, p.N, p.K, opx, opy, ldx, ldy, p.scm)).first;
    const LtPlan &pl = it->second;
    if (!pl.ok) return false;
    const float alpha = 1.0f, beta = 0.0f;
    return hipblasLtMatmul(d.handle, pl.desc, &alpha, p.b, pl.lx, p.a, pl.ly, &beta, p.c, pl.ld, p.c, pl.ld, &pl.algo,
                           d.workspace, kLtWorkspace, st) == HIPBLAS_STATUS_SUCCESS;
}

}  // namespace chelis
