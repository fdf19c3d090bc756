// chelis_hip_matmul / chelis_hip_linear: validate the packets, reduce them
// to one GemmProblem and pick the kernel family.
//
// Dispatch (the reference sends every BlasMatmul to hipBLAS,
// crates/chelis-backend-hip/src/emit.rs:4718-4842):
//   K <= 32                      -> tree_thread (short K, bit-exact)
//   M == 1 or N == 1             -> tree_wave   (GEMV, HBM bound, bit-exact),
//                                   or tree_panel when the matrix has at
//                                   most 64 outputs and is stored along them
//   min(M, N) <= 64 and (CHELIS_MATMUL_EXACT or min(M, N) < 16)
//                                -> tree_panel  (narrow side on the lanes,
//                                   bit-exact)
//   CHELIS_MATMUL_EXACT          -> tree_tiled  (bit-exact, any other shape)
//   otherwise                    -> MFMA tiles  (dense; rounding differs
//                                   from the canonical tree)
// bf16 / f16 (every shape): MFMA 16x16x32 tiles with a binary32
// accumulator; with CHELIS_MATMUL_EXACT (or K == 0) the operands are
// widened to binary32, the binary32 dispatch above runs exact, and the
// result is encoded once - the C lane's decode / tree / encode, bit-exact.
#include "gemm.h"

#include <algorithm>

namespace chelis {
namespace {

struct Mat {
    int64_t rows, cols, srow, scol;  // the trailing 2-D view
    int32_t nbatch;                  // leading axes (<= 2)
    int64_t bext[2], bstr[2];
};

// View a packet as [batch..., rows, cols]; a rank-1 operand is a row
// (as_row) or a column.
bool as_mat(const chelis_gpu_tensor *t, bool as_row, Mat *m) {
    *m = Mat{};
    if (t->rank < 1) return false;
    if (t->rank == 1) {
        if (as_row) {
            m->rows = 1, m->cols = t->shape[0], m->srow = 0, m->scol = t->strides[0];
        } else {
            m->rows = t->shape[0], m->cols = 1, m->srow = t->strides[0], m->scol = 0;
        }
        m->nbatch = 0;
        return true;
    }
    const int32_t r = t->rank;
    m->rows = t->shape[r - 2], m->cols = t->shape[r - 1];
    m->srow = t->strides[r - 2], m->scol = t->strides[r - 1];
    m->nbatch = r - 2;
    if (m->nbatch > 2) return false;
    for (int32_t i = 0; i < m->nbatch; ++i) m->bext[i] = t->shape[i], m->bstr[i] = t->strides[i];
    return true;
}

// Distinct indices of a view must address distinct elements (no write races).
bool non_overlapping(const chelis_gpu_tensor *t) {
    int32_t idx[8];
    int32_t n = 0;
    for (int32_t a = 0; a < t->rank; ++a)
        if (t->shape[a] > 1) idx[n++] = a;
    std::sort(idx, idx + n, [&](int32_t x, int32_t y) { return t->strides[x] < t->strides[y]; });
    int64_t span = 1;
    for (int32_t i = 0; i < n; ++i) {
        const int64_t s = t->strides[idx[i]];
        if (s < span) return false;
        span = s * t->shape[idx[i]];
    }
    return true;
}

int32_t build_problem(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b, const chelis_gpu_tensor *c,
                      GemmProblem *p, const char *what) {
    int32_t s;
    if ((s = check_tensor(a, "a")) || (s = check_tensor(b, "b")) || (s = check_tensor(c, "c"))) return s;
    if (!(is_float(a->dtype) || is_narrow16(a->dtype)) || a->dtype != b->dtype || a->dtype != c->dtype)
        return set_error(CHELIS_HIP_EDOMAIN, "%s: a, b and c must share an f32, f64, bf16 or f16 dtype", what);
    Mat ma, mb;
    if (!as_mat(a, true, &ma) || !as_mat(b, false, &mb))
        return set_error(CHELIS_HIP_EUNSUPPORTED, "%s: operands need rank 1..4", what);
    if (ma.cols != mb.rows)
        return set_error(CHELIS_HIP_EDOMAIN, "%s: contraction extents differ (%lld vs %lld)", what,
                         (long long)ma.cols, (long long)mb.rows);
    // expected result shape: broadcast batch, then [M] [N] (dropped for rank-1 operands)
    const int32_t nb = std::max(ma.nbatch, mb.nbatch);
    int64_t bext[2] = {1, 1}, sa[2] = {0, 0}, sb[2] = {0, 0};
    for (int32_t i = 0; i < nb; ++i) {
        const int32_t ia = i - (nb - ma.nbatch), ib = i - (nb - mb.nbatch);
        const int64_t ea = ia >= 0 ? ma.bext[ia] : 1, eb = ib >= 0 ? mb.bext[ib] : 1;
        if (ea != eb && ea != 1 && eb != 1) return set_error(CHELIS_HIP_EDOMAIN, "%s: batch axes do not broadcast", what);
        bext[2 - nb + i] = std::max(ea, eb);
        sa[2 - nb + i] = (ia >= 0 && ea != 1) ? ma.bstr[ia] : 0;
        sb[2 - nb + i] = (ib >= 0 && eb != 1) ? mb.bstr[ib] : 0;
    }
    int64_t want[8];
    int32_t wr = 0;
    for (int32_t i = 0; i < nb; ++i) want[wr++] = bext[2 - nb + i];
    if (a->rank > 1) want[wr++] = ma.rows;
    if (b->rank > 1) want[wr++] = mb.cols;
    if (c->rank != wr) return set_error(CHELIS_HIP_EDOMAIN, "%s: result rank %d, expected %d", what, c->rank, wr);
    for (int32_t i = 0; i < wr; ++i)
        if (c->shape[i] != want[i]) return set_error(CHELIS_HIP_EDOMAIN, "%s: result axis %d has the wrong extent", what, i);
    if (!non_overlapping(c)) return set_error(CHELIS_HIP_EDOMAIN, "%s: result view overlaps itself", what);
    // result strides per role
    int64_t scm = 0, scn = 0, sc[2] = {0, 0};
    {
        int32_t ax = 0;
        for (int32_t i = 0; i < nb; ++i) sc[2 - nb + i] = c->strides[ax++];
        if (a->rank > 1) scm = c->strides[ax++];
        if (b->rank > 1) scn = c->strides[ax++];
    }
    *p = GemmProblem{};
    p->a = a->data, p->b = b->data, p->c = c->data;
    p->M = ma.rows, p->N = mb.cols, p->K = ma.cols;
    p->sam = ma.srow, p->sak = ma.scol, p->sbk = mb.srow, p->sbn = mb.scol, p->scm = scm, p->scn = scn;
    p->nb0 = bext[0], p->nb1 = bext[1];
    p->sa0 = sa[0], p->sa1 = sa[1], p->sb0 = sb[0], p->sb1 = sb[1], p->sc0 = sc[0], p->sc1 = sc[1];
    p->gelu_fast = exact_mode() ? 0 : 1;
    return CHELIS_HIP_OK;
}

int32_t dispatch(chelis_dtype dt, const GemmProblem &p, int32_t flags);

// The exact 16-bit matmul: widen both operands to contiguous binary32,
// run the binary32 canonical-tree dispatch, encode the result into c.
int32_t dispatch_narrow_exact(chelis_dtype dt, const GemmProblem &p, hipStream_t st) {
    const int64_t nz0 = p.nb0, nz1 = p.nb1, M = p.M, N = p.N, K = p.K;
    const size_t ab = sizeof(float) * (size_t)(nz0 * nz1 * M * K) + 16,
                 bb = sizeof(float) * (size_t)(nz0 * nz1 * K * N) + 16,
                 cb = sizeof(float) * (size_t)(nz0 * nz1 * M * N) + 16;
    float *a32 = static_cast<float *>(scratch_alloc(ab));
    float *b32 = static_cast<float *>(scratch_alloc(bb));
    float *c32 = static_cast<float *>(scratch_alloc(cb));
    int32_t s = CHELIS_HIP_OK;
    if (!a32 || !b32 || !c32) s = set_error(CHELIS_HIP_EHIP, "matmul: scratch allocation failed");
    if (!s) s = widen16(dt, p.a, a32, nz0, nz1, M, K, p.sa0, p.sa1, p.sam, p.sak, st);
    if (!s) s = widen16(dt, p.b, b32, nz0, nz1, K, N, p.sb0, p.sb1, p.sbk, p.sbn, st);
    if (!s) {
        GemmProblem q{};
        q.a = a32, q.b = b32, q.c = c32;
        q.M = M, q.N = N, q.K = K;
        q.sam = K, q.sak = 1, q.sbk = N, q.sbn = 1, q.scm = N, q.scn = 1;
        q.nb0 = nz0, q.nb1 = nz1;
        q.sa0 = nz1 * M * K, q.sa1 = M * K, q.sb0 = nz1 * K * N, q.sb1 = K * N, q.sc0 = nz1 * M * N, q.sc1 = M * N;
        s = dispatch(CHELIS_DTYPE_F32, q, CHELIS_MATMUL_EXACT);
    }
    if (!s) s = narrow16(dt, c32, p.c, nz0, nz1, M, N, p.sc0, p.sc1, p.scm, p.scn, st);
    if (a32) scratch_free(a32, ab);
    if (b32) scratch_free(b32, bb);
    if (c32) scratch_free(c32, cb);
    return s;
}

int32_t dispatch(chelis_dtype dt, const GemmProblem &p, int32_t flags) {
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    if (p.M == 0 || p.N == 0 || p.nb0 == 0 || p.nb1 == 0) return CHELIS_HIP_OK;
    if (exact_mode()) flags |= CHELIS_MATMUL_EXACT;
    if (is_narrow16(dt)) {
        if ((flags & CHELIS_MATMUL_EXACT) || p.K == 0) return dispatch_narrow_exact(dt, p, st);
        if (gemm16_lt(dt, p, st)) return CHELIS_HIP_OK;
        return gemm_mfma16(dt, p, st);
    }
    const bool f64 = dt == CHELIS_DTYPE_F64;
    const int64_t narrow = std::min(p.M, p.N);
    if (p.K <= 32) return gemm_tree_thread(dt, p, st);
    if (p.M == 1 || p.N == 1) {
        // a matrix of at most 64 outputs stored along the output axis: the
        // column panel puts the outputs on the lanes and reads whole rows
        if (p.N == 1 && p.M > 1 && p.M <= 64 && p.sak != 1 && p.sam == 1) return gemm_tree_panel(dt, p, st);
        if (p.M == 1 && p.N > 1 && p.N <= 64 && p.sbk != 1 && p.sbn == 1) return gemm_tree_panel(dt, p, st);
        return gemm_tree_wave(dt, p, st);
    }
    const bool exact = flags & CHELIS_MATMUL_EXACT;
    // A narrow side of 16..64 (the skinny 8192x64x4096 of config 3c) runs
    // on the matrix cores within the GEMM tolerance, where the tree panel is
    // bit-exact but bound by its separate multiply and add (329 us against a
    // 55 us f64 FMA floor); the exact flag keeps the tree
    if (narrow <= 64 && (exact || narrow < 16)) return gemm_tree_panel(dt, p, st);
    if (exact) return gemm_tree_tiled(dt, p, st);
    return gemm_mfma(dt, p, st);
}

// True when dispatch sends p to the MFMA tiles.
bool takes_mfma(chelis_dtype dt, const GemmProblem &p) {
    if (is_narrow16(dt) || (dt != CHELIS_DTYPE_F32 && dt != CHELIS_DTYPE_F64)) return false;
    if (exact_mode() || p.K <= 32 || p.M == 1 || p.N == 1) return false;
    return std::min(p.M, p.N) >= 16 && p.M > 0 && p.N > 0 && p.nb0 > 0 && p.nb1 > 0;
}

// A [M, N] contiguous view of part's first slice, for build_problem (the
// packet points into this object, which is not copied).
struct SliceView {
    int64_t shape[2], strides[2];
    chelis_gpu_tensor t{};
    SliceView(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b, void *part) {
        shape[0] = a->shape[a->rank - 2];
        shape[1] = b->shape[b->rank - 1];
        strides[0] = shape[1];
        strides[1] = 1;
        t.data = part;
        t.dtype = a->dtype;
        t.rank = 2;
        t.shape = shape;
        t.strides = strides;
        t.count = shape[0] * shape[1];
        t.byte_capacity = t.count * dtype_width(a->dtype);
    }
    SliceView(const SliceView &) = delete;
};

}  // namespace

int32_t linear_multi_b(const chelis_gpu_tensor *a, const chelis_gpu_tensor *const *b,
                       const chelis_gpu_tensor *const *bias, int32_t n, const chelis_gpu_tensor *c) {
    if (n < 1 || n > kMaxBatchPtrs || !a || !b || !bias || !c || a->rank != 2 || c->rank != 3 || c->shape[0] != n)
        return set_error(CHELIS_HIP_EDOMAIN, "linear_multi_b: a [M,K], n <= %d weights, c [n,M,N]", kMaxBatchPtrs);
    bool same = true;
    for (int32_t i = 0; i < n; ++i) {
        if (int32_t s = check_tensor(b[i], "b")) return s;
        if (int32_t s = check_tensor(bias[i], "bias")) return s;
        same = same && b[i]->rank == 2 && same_shape(b[i], b[0]) && b[i]->strides[0] == b[0]->strides[0] &&
               b[i]->strides[1] == b[0]->strides[1] && b[i]->dtype == a->dtype && bias[i]->rank == 1 &&
               bias[i]->dtype == a->dtype && bias[i]->shape[0] == b[0]->shape[1] &&
               bias[i]->strides[0] == bias[0]->strides[0] &&
               (reinterpret_cast<uintptr_t>(b[i]->data) & 15) == (reinterpret_cast<uintptr_t>(b[0]->data) & 15);
    }
    if (!same) return set_error(CHELIS_HIP_EDOMAIN, "linear_multi_b: weights and biases must match in shape and strides");
    // the batch view of a (stride 0) and of the first weight; the problem
    // then reads weight and bias i at their own addresses
    const int64_t a_sh[3] = {n, a->shape[0], a->shape[1]}, a_st[3] = {0, a->strides[0], a->strides[1]};
    const int64_t b_sh[3] = {n, b[0]->shape[0], b[0]->shape[1]}, b_st[3] = {0, b[0]->strides[0], b[0]->strides[1]};
    chelis_gpu_tensor a3 = *a, b3 = *b[0];
    a3.rank = 3, a3.shape = a_sh, a3.strides = a_st, a3.count = n * a->count;
    b3.rank = 3, b3.shape = b_sh, b3.strides = b_st, b3.count = n * b[0]->count;
    GemmProblem p;
    if (int32_t s = build_problem(&a3, &b3, c, &p, "linear")) return s;
    if (!takes_mfma(a->dtype, p)) {
        // one launch per weight, each into its slice of c
        for (int32_t i = 0; i < n; ++i) {
            const int64_t sh[2] = {c->shape[1], c->shape[2]}, st[2] = {c->strides[1], c->strides[2]};
            chelis_gpu_tensor ci = *c;
            ci.data = static_cast<char *>(c->data) + i * c->strides[0] * dtype_width(c->dtype);
            ci.rank = 2, ci.shape = sh, ci.strides = st, ci.count = sh[0] * sh[1];
            ci.byte_capacity = c->byte_capacity - i * c->strides[0] * dtype_width(c->dtype);
            if (int32_t s = chelis_hip_linear(a, b[i], bias[i], CHELIS_ACT_NONE, nullptr, &ci, 0)) return s;
        }
        return CHELIS_HIP_OK;
    }
    p.nbz = n;
    for (int32_t i = 0; i < n; ++i) p.bz[i] = b[i]->data, p.biasz[i] = bias[i]->data;
    p.bias = bias[0]->data;
    p.sbias = bias[0]->strides[0];
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    return gemm_mfma(a->dtype, p, st);
}

int64_t matmul_slice_count(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b) {
    if (!a || !b || a->rank != 2 || b->rank != 2) return 1;
    // a stand-in address: only the problem's shape is read
    static int64_t dummy[1];
    const SliceView c(a, b, dummy);
    GemmProblem p;
    if (build_problem(a, b, &c.t, &p, "matmul")) return 1;
    return takes_mfma(a->dtype, p) ? gemm_mfma_slice_count(a->dtype, p) : 1;
}

int32_t matmul_slices(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b, void *part, int64_t slices) {
    if (!a || !b || a->rank != 2 || b->rank != 2)
        return set_error(CHELIS_HIP_EDOMAIN, "matmul slices: two matrices required");
    const SliceView c(a, b, part);
    GemmProblem p;
    if (int32_t s = build_problem(a, b, &c.t, &p, "matmul")) return s;
    const int64_t ks = takes_mfma(a->dtype, p) ? gemm_mfma_slice_count(a->dtype, p) : 1;
    if (ks != slices) return set_error(CHELIS_HIP_EDOMAIN, "matmul slices: %lld slices, not %lld", (long long)ks,
                                       (long long)slices);
    if (ks == 1 && !takes_mfma(a->dtype, p)) return dispatch(a->dtype, p, 0);
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    return gemm_mfma_slices(a->dtype, p, part, st);
}

int32_t matmul_causal(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b, const chelis_gpu_tensor *c,
                      int32_t mode) {
    GemmProblem p;
    if (int32_t s = build_problem(a, b, c, &p, "matmul")) return s;
    p.causal = mode;
    return dispatch(a->dtype, p, 0);
}

}  // namespace chelis

using namespace chelis;


extern "C" int32_t chelis_hip_matmul(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                                     const chelis_gpu_tensor *c, int32_t flags) {
    const ModeScope mode;
    GemmProblem p;
    if (int32_t s = build_problem(a, b, c, &p, "matmul")) return s;
    if (flags & ~CHELIS_MATMUL_EXACT) return set_error(CHELIS_HIP_EDOMAIN, "matmul: unknown flags %d", flags);
    return dispatch(a->dtype, p, flags);
}

extern "C" int32_t chelis_hip_linear(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b,
                                     const chelis_gpu_tensor *bias, int32_t activation,
                                     const chelis_gpu_tensor *residual, const chelis_gpu_tensor *c, int32_t flags) {
    const ModeScope mode;
    GemmProblem p;
    if (int32_t s = build_problem(a, b, c, &p, "linear")) return s;
    if (flags & ~CHELIS_MATMUL_EXACT) return set_error(CHELIS_HIP_EDOMAIN, "linear: unknown flags %d", flags);
    if (activation < CHELIS_ACT_NONE || activation > CHELIS_ACT_GELU)
        return set_error(CHELIS_HIP_EDOMAIN, "linear: unknown activation %d", activation);
    if (a->rank < 2 || b->rank < 2) return set_error(CHELIS_HIP_EDOMAIN, "linear: a and b need rank >= 2");
    if (is_narrow16(a->dtype))
        return set_error(CHELIS_HIP_EUNSUPPORTED, "linear: bf16/f16 matmuls take no fused epilogue (use matmul)");
    p.act = activation;
    if (bias) {
        if (int32_t s = check_tensor(bias, "bias")) return s;
        // [N], or [batch..., N] over the result's batch axes (c is [batch..., M, N])
        const int32_t nbatch = c->rank - 2;
        bool ok = bias->dtype == a->dtype && bias->rank >= 1 && bias->shape[bias->rank - 1] == p.N;
        if (ok && bias->rank > 1) {
            ok = bias->rank == nbatch + 1;
            for (int32_t i = 0; ok && i < nbatch; ++i) ok = bias->shape[i] == c->shape[i];
        }
        if (!ok)
            return set_error(CHELIS_HIP_EDOMAIN, "linear: bias must be [N] or [batch..., N] of the operand dtype");
        p.bias = bias->data;
        p.sbias = bias->strides[bias->rank - 1];
        if (bias->rank > 1) {
            // batch axes are right-aligned in the problem: one axis is z1, two are z0, z1
            p.sbias1 = bias->strides[bias->rank - 2];
            p.sbias0 = bias->rank > 2 ? bias->strides[bias->rank - 3] : 0;
        }
    }
    if (residual) {
        if (int32_t s = check_tensor(residual, "residual")) return s;
        if (residual->dtype != a->dtype || !same_shape(residual, c))
            return set_error(CHELIS_HIP_EDOMAIN, "linear: residual must match the result");
        const int32_t r = residual->rank;
        p.resid = residual->data;
        p.srm = residual->strides[r - 2];
        p.srn = residual->strides[r - 1];
        p.sr0 = r >= 4 ? residual->strides[r - 4] : 0;
        p.sr1 = r >= 3 ? residual->strides[r - 3] : 0;
    }
    return dispatch(a->dtype, p, flags);
}
