// Internal interface between the matmul entry points (k_gemm.hip) and the
// kernel families that serve them: the MFMA tile kernels (k_gemm.hip) and
// the canonical-tree kernels (k_gemm_exact.hip).
#pragma once

#include "chain.h"

namespace chelis {

constexpr int kMaxBatchPtrs = 4;

// One contraction c[z][m][n] = sum_k a[z][m][k] * b[z][k][n] over a batch of
// up to two axes (z = z0 * nb1 + z1). Strides are in elements; every view
// is already validated against its byte capacity on the host.
struct GemmProblem {
    const void *a, *b;
    void *c;
    int64_t M, N, K;
    int64_t sam, sak, sbk, sbn, scm, scn;
    int64_t nb0, nb1;                       // batch extents (1 when absent)
    int64_t sa0, sa1, sb0, sb1, sc0, sc1;   // batch strides
    // fused epilogue (graph order): v = mm; v = v + bias[n]; act; v = resid + v
    const void *bias;
    int64_t sbias, sbias0, sbias1;  // along n, batch axis 0, batch axis 1
    int32_t act;
    const void *resid;
    int64_t srm, srn, sr0, sr1;
    // Causal attention structure (honoured by the MFMA tiles, ignored - so
    // computed in full - elsewhere): 1 = only entries with n <= m are used
    // downstream, tiles wholly above the diagonal are skipped and left as
    // they were; 2 = a[m][k] is zero for k > m, the contraction of a row
    // tile stops after its last row.
    int32_t causal;
    // Batches whose B operand and bias sit at unrelated addresses (the Q, K
    // and V weights): nbz > 0 makes batch z read B at bz[z] and its bias at
    // biasz[z] (each with batch 0's strides). Only the MFMA tiles take such
    // a problem (linear_multi_b).
    int32_t nbz;
    const void *bz[kMaxBatchPtrs];
    const void *biasz[kMaxBatchPtrs];
    // binary32 GELU epilogue in the default mode: gelu_fast_f32 (the Phi
    // graph for the inputs it does not serve) instead of the graph
    int32_t gelu_fast;
};

// Epilogue of one output element, each step finalized at the dtype so the
// bits equal the unfused graph's (mm, add bias, relu/gelu, add residual).
// GELU = false instances serve launches whose activation is not GELU: a
// kernel that holds many outputs per lane would otherwise carry the GELU
// graph's registers (and code) through its whole main loop.
// The epilogue's arithmetic on values already loaded (b: the bias element,
// r: the residual element, each used only when the problem has it).
template <typename T, bool GELU = true, class Tabs = ErfcTablesConst>
__device__ inline T epilogue_values(T acc, const GemmProblem &p, bool has_bias, T b, T r,
                                    const Tabs &tb = Tabs{}) {
    T v = canon(acc);
    if (has_bias) v = canon(v + b);
    if (p.act == CHELIS_ACT_RELU) {
        v = v < T(0) ? T(0) : v;
    } else if (GELU && p.act == CHELIS_ACT_GELU) {
        bool slow = true;
        T g = v;
        if constexpr (sizeof(T) == 4)
            if (p.gelu_fast) g = gelu_fast_f32(v, slow);
        v = slow ? gelu_one_t<T>(v, tb) : g;
    }
    if (p.resid) v = canon(r + v);
    return v;
}

template <typename T, bool GELU = true, class Tabs = ErfcTablesConst>
__device__ inline T gemm_epilogue(T acc, const GemmProblem &p, int64_t z0, int64_t z1, int64_t m, int64_t n,
                                  const Tabs &tb = Tabs{}) {
    const T *bias = static_cast<const T *>(p.nbz ? p.biasz[z0 * p.nb1 + z1] : p.bias);
    const T b = bias ? bias[(p.nbz ? 0 : z0 * p.sbias0 + z1 * p.sbias1) + n * p.sbias] : T(0);
    const T r = p.resid ? static_cast<const T *>(p.resid)[z0 * p.sr0 + z1 * p.sr1 + m * p.srm + n * p.srn] : T(0);
    return epilogue_values<T, GELU>(acc, p, bias != nullptr, b, r, tb);
}

int32_t gemm_mfma(chelis_dtype dt, const GemmProblem &p, hipStream_t st);
// A plain 16-bit product on hipBLASLt when it takes the shape and layout
// (gemm_lt.cpp); false leaves it to the MFMA tiles.
bool gemm16_lt(chelis_dtype dt, const GemmProblem &p, hipStream_t st);
// The MFMA tiles' raw sums as K slices, part[slice][z][m][n] (no epilogue,
// no combine; one slice when the product is not split), and their count.
int64_t gemm_mfma_slice_count(chelis_dtype dt, const GemmProblem &p);
int32_t gemm_mfma_slices(chelis_dtype dt, const GemmProblem &p, void *part, hipStream_t st);
// c[i] = a . b[i] + bias[i] (i < n <= kMaxBatchPtrs; the b[i] alike in
// shape and strides, c a [n, M, N] block): one batched MFMA launch over the
// n weights where they sit, or n linear launches where the dispatch takes
// another kernel.
int32_t linear_multi_b(const chelis_gpu_tensor *a, const chelis_gpu_tensor *const *b,
                       const chelis_gpu_tensor *const *bias, int32_t n, const chelis_gpu_tensor *c);
// c = a . b of two matrices as raw K slices for a consumer that sums them
// in slice order itself (then finalizes: canon, epilogue): part holds
// matmul_slice_count(a, b) contiguous [M, N] slices. Whatever the dispatch
// routes elsewhere (tree kernels, the exact flag) is one finished slice.
int64_t matmul_slice_count(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b);
int32_t matmul_slices(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b, void *part, int64_t slices);
// bf16 / f16 operands and result, binary32 accumulation (k_gemm16.hip).
int32_t gemm_mfma16(chelis_dtype dt, const GemmProblem &p, hipStream_t st);
// 16-bit [nz0][nz1][rows][cols] view <-> contiguous binary32 (the exact
// 16-bit matmul runs the binary32 canonical tree between them).
int32_t widen16(chelis_dtype dt, const void *src, float *dst, int64_t nz0, int64_t nz1, int64_t rows, int64_t cols,
                int64_t s0, int64_t s1, int64_t sr, int64_t sc, hipStream_t st);
int32_t narrow16(chelis_dtype dt, const float *src, void *dst, int64_t nz0, int64_t nz1, int64_t rows, int64_t cols,
                 int64_t s0, int64_t s1, int64_t sr, int64_t sc, hipStream_t st);
// Causal attention fused in one launch (k_attention.hip): o = softmax(
// where(key <= row, q.k^T * scale, -inf)).v over f32 [batch, heads, seq, 64]
// views, seq a multiple of 64; o must not overlap q, k or v.
bool attention_causal_fits(const chelis_gpu_tensor *q, const chelis_gpu_tensor *k, const chelis_gpu_tensor *v,
                           const chelis_gpu_tensor *o);
int32_t attention_causal(const chelis_gpu_tensor *q, const chelis_gpu_tensor *k, const chelis_gpu_tensor *v,
                         double scale, const chelis_gpu_tensor *o);
// The linear-regression step r = X.w - y, grad = X^T.r / n, loss =
// tree(r * r) / n in two launches, bit-identical to the unfused graph
// (k_linreg.hip); linreg_fused_fits: d <= 32 and rows of X contiguous.
bool linreg_fused_fits(const chelis_gpu_tensor *X, const chelis_gpu_tensor *w);
int32_t linreg_fused(const chelis_gpu_tensor *X, const chelis_gpu_tensor *w, const chelis_gpu_tensor *y,
                     const chelis_gpu_tensor *grad, const chelis_gpu_tensor *loss, hipStream_t st);
// The MLP step between and after its two wide products (k_mlp.hip),
// bit-identical to the unfused launches. mlp_head_tail: from x.W1's raw K
// slices (z1, [z1_slices][B][H]) to d, g_z2, nl, g_d (the input of the
// x^T.g_d product) and the tail's row-block totals in part
// (mlp_part_bytes). mlp_finish, after x^T.g_d (gw1, [gw1_slices][I][H]):
// the W1, W2, b1, b2 updates and the loss. All pointers are contiguous f32
// device arrays ([B,H] d, gd; [H,O] W2; [B,O] onehot, gz2; [B] nl); key is
// the KEY tensor's storage.
struct MlpNarrow {
    int64_t B, I, H, O;
    const float *z1;
    int64_t z1_slices;
    const float *gw1;
    int64_t gw1_slices;
    const float *w1, *w2, *b2, *onehot, *b1;
    const uint64_t *key;
    float *d, *gz2, *nl, *gd, *part;
    float *w1_out, *w2_out, *b1_out, *b2_out, *loss;
    float rate, lr;
};
bool mlp_narrow_fits(int64_t B, int64_t I, int64_t H, int64_t O);
size_t mlp_part_bytes(int64_t B, int64_t H);
int32_t mlp_head_tail(const MlpNarrow &m, hipStream_t st);
int32_t mlp_finish(const MlpNarrow &m, hipStream_t st);
// The MLP training step (chelis_prog_mlp_train_step) at a given dropout
// rate and learning rate: five launches where mlp_narrow_fits, else the
// launch-per-region form; the same bits either way.
int32_t mlp_train_step_run(const chelis_gpu_tensor *const *in, int32_t n_in, const chelis_gpu_tensor *const *out,
                           int32_t n_out, float rate, float lr);
// c = a . b for attention with the causal mode above (programs only).
int32_t matmul_causal(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b, const chelis_gpu_tensor *c,
                      int32_t mode);
// Canonical-tree kernels: bit-exact with the [05-OP-30] matmul.
int32_t gemm_tree_wave(chelis_dtype dt, const GemmProblem &p, hipStream_t st);    // one wave per output
int32_t gemm_tree_tiled(chelis_dtype dt, const GemmProblem &p, hipStream_t st);   // narrow N, long K
int32_t gemm_tree_thread(chelis_dtype dt, const GemmProblem &p, hipStream_t st);  // short K
int32_t gemm_tree_panel(chelis_dtype dt, const GemmProblem &p, hipStream_t st);   // min(M, N) <= 64

}  // namespace chelis
