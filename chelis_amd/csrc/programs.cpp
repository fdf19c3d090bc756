// Configuration programs as generated entries: each is the launch sequence
// the HIP backend emits for the program's fused DAG, one region launcher
// per fused region, on the library stream (include/chelis_programs.h).
//
// Intermediates live in one stream-ordered workspace per call (the
// library's cached scratch blocks, recycled in stream order on the library
// stream), in place of the reference's per-call slot allocations
// (crates/chelis-backend-hip/src/emit.rs:3162).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <vector>

#include "chelis_programs.h"
#include "gemm.h"
#include "hip_common.h"

namespace chelis {
namespace {

// A contiguous or strided packet over device memory this file manages.
struct Pkt {
    int64_t shape[4] = {0, 0, 0, 0}, strides[4] = {0, 0, 0, 0};
    chelis_gpu_tensor t{};
    Pkt() = default;
    Pkt(void *data, chelis_dtype dt, std::initializer_list<int64_t> sh) {
        int32_t r = 0;
        for (int64_t e : sh) shape[r++] = e;
        int64_t acc = 1;
        for (int32_t a = r; a-- > 0;) {
            strides[a] = acc;
            acc *= shape[a];
        }
        init(data, dt, r, acc, acc * dtype_width(dt));
    }
    Pkt(void *data, chelis_dtype dt, std::initializer_list<int64_t> sh, std::initializer_list<int64_t> st,
        int64_t capacity) {
        int32_t r = 0;
        int64_t count = 1;
        for (int64_t e : sh) shape[r++] = e, count *= e;
        r = 0;
        for (int64_t s : st) strides[r++] = s;
        init(data, dt, r, count, capacity);
    }
    void init(void *data, chelis_dtype dt, int32_t rank, int64_t count, int64_t capacity) {
        t.data = data;
        t.shape = shape;
        t.strides = strides;
        t.count = count;
        t.byte_capacity = capacity;
        t.rank = rank;
        t.dtype = dt;
        t.ownership = 0;
    }
    Pkt(const Pkt &o) { *this = o; }
    Pkt &operator=(const Pkt &o) {
        std::memcpy(shape, o.shape, sizeof shape);
        std::memcpy(strides, o.strides, sizeof strides);
        t = o.t;
        t.shape = shape;
        t.strides = strides;
        return *this;
    }
    const chelis_gpu_tensor *operator&() const { return &t; }
};

// One stream-ordered scratch block carved into 256-byte aligned pieces.
class Workspace {
public:
    explicit Workspace(hipStream_t) {}
    ~Workspace() { scratch_free(base_, size_); }
    size_t reserve(int64_t bytes) {
        const size_t off = size_;
        size_ += (static_cast<size_t>(bytes) + 255) & ~size_t(255);
        return off;
    }
    int32_t commit() {
        if (size_ && !(base_ = scratch_alloc(size_)))
            return set_error(CHELIS_HIP_EHIP, "workspace: cannot allocate %zu bytes", size_);
        return CHELIS_HIP_OK;
    }
    void *at(size_t off) const { return static_cast<char *>(base_) + off; }

private:
    void *base_ = nullptr;
    size_t size_ = 0;
};

chelis_fused_chain chain(std::initializer_list<chelis_fused_step> steps) {
    chelis_fused_chain c{};
    c.n_steps = 0;
    for (const chelis_fused_step &s : steps) c.steps[c.n_steps++] = s;
    return c;
}
chelis_fused_step step(int op, int32_t a0, int32_t a1 = 0, double imm = 0.0) {
    chelis_fused_step s{};
    s.op = (uint8_t)op;
    s.args[0] = a0;
    s.args[1] = a1;
    s.imm = imm;
    return s;
}
constexpr int32_t prev(int32_t k) { return -(k + 1); }

#define TRY(expr)                                 \
    do {                                          \
        if (int32_t chelis_s_ = (expr)) return chelis_s_; \
    } while (0)

bool shape_is(const chelis_gpu_tensor *t, std::initializer_list<int64_t> sh, chelis_dtype dt) {
    if (!t || t->dtype != dt || t->rank != (int32_t)sh.size()) return false;
    int32_t a = 0;
    for (int64_t e : sh)
        if (t->shape[a++] != e) return false;
    return true;
}

int32_t check_all(const chelis_gpu_tensor *const *ts, int32_t n, const char *what) {
    if (!ts) return set_error(CHELIS_HIP_EDOMAIN, "%s: null packet array", what);
    for (int32_t i = 0; i < n; ++i)
        if (int32_t s = check_tensor(ts[i], what)) return s;
    return CHELIS_HIP_OK;
}

// y = x / extent at the dtype (mean = tree sum / extent, [05-OP-11]).
int32_t divide_by(const chelis_gpu_tensor *x, double extent, const chelis_gpu_tensor *y) {
    const chelis_fused_chain c = chain({step(CHELIS_FUSED_CONST, 0, 0, extent), step(CHELIS_FUSED_DIV, 0, prev(0))});
    const chelis_gpu_tensor *in[1] = {x};
    return chelis_hip_fused_elementwise(&c, in, 1, y);
}

}  // namespace
}  // namespace chelis

using namespace chelis;

// ------------------------------------------------------------------ linreg
extern "C" int32_t chelis_prog_linreg_step(const chelis_gpu_tensor *const *in, int32_t n_in,
                                           const chelis_gpu_tensor *const *out, int32_t n_out) {
    const ModeScope mode;
    if (n_in != 3 || n_out != 2) return set_error(CHELIS_HIP_EDOMAIN, "linreg_step: 3 inputs, 2 outputs");
    TRY(check_all(in, 3, "linreg_step input"));
    TRY(check_all(out, 2, "linreg_step output"));
    const chelis_gpu_tensor *X = in[0], *w = in[1], *y = in[2];
    if (X->rank != 2) return set_error(CHELIS_HIP_EDOMAIN, "linreg_step: X must be [n, d]");
    const int64_t n = X->shape[0], d = X->shape[1];
    const chelis_dtype dt = X->dtype;
    if (!is_float(dt) || !shape_is(w, {d}, dt) || !shape_is(y, {n}, dt) || !shape_is(out[0], {d}, dt) ||
        !shape_is(out[1], {}, dt))
        return set_error(CHELIS_HIP_EDOMAIN, "linreg_step: shapes/dtypes must be X[n,d], w[d], y[n] -> grad[d], loss[]");
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    // two launches (row blocks, then the joins) where d <= 32; the same bits
    // as the launch-per-region form below
    if (linreg_fused_fits(X, w)) return linreg_fused(X, w, y, out[0], out[1], st);
    Workspace ws(st);
    const size_t o_r = ws.reserve(n * dtype_width(dt)), o_g = ws.reserve(d * dtype_width(dt));
    TRY(ws.commit());
    const Pkt r(ws.at(o_r), dt, {n}), g(ws.at(o_g), dt, {d});
    const Pkt Xt(X->data, dt, {d, n}, {X->strides[1], X->strides[0]}, X->byte_capacity);
    // r = X.w - y
    TRY(chelis_hip_matmul(X, w, &r, 0));
    const chelis_fused_chain sub = chain({step(CHELIS_FUSED_SUB, 0, 1)});
    const chelis_gpu_tensor *ry[2] = {&r, y};
    TRY(chelis_hip_fused_elementwise(&sub, ry, 2, &r));
    // grad = X^T.r / n
    TRY(chelis_hip_matmul(&Xt, &r, &g, 0));
    TRY(divide_by(&g, (double)n, out[0]));
    // loss = tree_sum(r * r) / n
    const chelis_fused_chain sq = chain({step(CHELIS_FUSED_MUL, 0, 0)});
    const chelis_gpu_tensor *rr[1] = {&r};
    TRY(chelis_hip_reduce(CHELIS_REDUCE_SUM, &sq, rr, 1, 0, out[1]));
    TRY(divide_by(out[1], (double)n, out[1]));
    return CHELIS_HIP_OK;
}

// ------------------------------------------------------------------ transformer block
extern "C" int32_t chelis_prog_transformer_block(const chelis_gpu_tensor *const *in, int32_t n_in,
                                                 const chelis_gpu_tensor *const *out, int32_t n_out) {
    const ModeScope mode;
    if (n_in != 17 || n_out != 1) return set_error(CHELIS_HIP_EDOMAIN, "transformer_block: 17 inputs, 1 output");
    TRY(check_all(in, 17, "transformer_block input"));
    TRY(check_all(out, 1, "transformer_block output"));
    const chelis_gpu_tensor *x = in[0];
    const chelis_gpu_tensor *const *P = in + 1;
    if (x->rank != 3) return set_error(CHELIS_HIP_EDOMAIN, "transformer_block: x must be [batch, seq, d_model]");
    const int64_t B = x->shape[0], S = x->shape[1], D = x->shape[2];
    const chelis_dtype dt = x->dtype;
    constexpr int64_t DH = 64;
    if (dt != CHELIS_DTYPE_F32 && dt != CHELIS_DTYPE_F64) return set_error(CHELIS_HIP_EDOMAIN, "transformer_block: f32/f64");
    if (D % DH) return set_error(CHELIS_HIP_EDOMAIN, "transformer_block: d_model must be a multiple of 64");
    const int64_t H = D / DH, F = P[12]->rank == 2 ? P[12]->shape[1] : -1, R = B * S;
    const bool ok = shape_is(P[0], {D}, dt) && shape_is(P[1], {D}, dt) && shape_is(P[2], {D, D}, dt) &&
                    shape_is(P[3], {D}, dt) && shape_is(P[4], {D, D}, dt) && shape_is(P[5], {D}, dt) &&
                    shape_is(P[6], {D, D}, dt) && shape_is(P[7], {D}, dt) && shape_is(P[8], {D, D}, dt) &&
                    shape_is(P[9], {D}, dt) && shape_is(P[10], {D}, dt) && shape_is(P[11], {D}, dt) &&
                    shape_is(P[12], {D, F}, dt) && shape_is(P[13], {F}, dt) && shape_is(P[14], {F, D}, dt) &&
                    shape_is(P[15], {D}, dt) && shape_is(out[0], {B, S, D}, dt);
    if (!ok) return set_error(CHELIS_HIP_EDOMAIN, "transformer_block: parameter shapes do not match x");
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    const int64_t w = dtype_width(dt);
    // The Q, K and V projections run as one batch of three products that
    // reads each weight and bias where it sits, the three results landing
    // in one [3, B*S, D] block (measured at [4096,1024] x [1024,1024]: 255
    // us for the batch of three on 128-tiles against 3 x 90 us).
    // attention as one fused launch where it applies (binary32, seq a
    // multiple of 64), else scores, causal softmax and P.V
    const bool fused = dt == CHELIS_DTYPE_F32 && S % 64 == 0;
    Workspace ws(st);
    const size_t o_h = ws.reserve(R * D * w), o_qkv = ws.reserve(3 * R * D * w),
                 o_s = ws.reserve(fused ? 0 : B * H * S * S * w),
                 o_o = ws.reserve(R * D * w), o_x1 = ws.reserve(R * D * w), o_f = ws.reserve(R * F * w);
    TRY(ws.commit());
    const Pkt x2(x->data, dt, {R, D}, {x->strides[1], x->strides[2]}, x->byte_capacity);
    char *qkv = static_cast<char *>(ws.at(o_qkv));
    const Pkt h(ws.at(o_h), dt, {R, D}), q(qkv, dt, {R, D}), k(qkv + R * D * w, dt, {R, D}),
        v(qkv + 2 * R * D * w, dt, {R, D}), o(ws.at(o_o), dt, {R, D}), x1(ws.at(o_x1), dt, {R, D}),
        f(ws.at(o_f), dt, {R, F});
    const Pkt s(ws.at(o_s), dt, {B, H, S, S});
    const int64_t cap = R * D * w;
    // per-head views of [B, S, H, DH] storage as [B, H, S, DH] (and K^T as [B, H, DH, S])
    const Pkt qh(q.t.data, dt, {B, H, S, DH}, {S * D, DH, D, 1}, cap);
    const Pkt kt(k.t.data, dt, {B, H, DH, S}, {S * D, DH, 1, D}, cap);
    const Pkt vh(v.t.data, dt, {B, H, S, DH}, {S * D, DH, D, 1}, cap);
    const Pkt oh(o.t.data, dt, {B, H, S, DH}, {S * D, DH, D, 1}, cap);
    const Pkt y2(out[0]->data, dt, {R, D}, {out[0]->strides[1], out[0]->strides[2]}, out[0]->byte_capacity);
    if (x->strides[0] != S * x->strides[1] || out[0]->strides[0] != S * out[0]->strides[1])
        return set_error(CHELIS_HIP_EUNSUPPORTED, "transformer_block: batch and seq axes of x/y must collapse");
    // attention
    TRY(chelis_hip_layer_norm(&x2, P[0], P[1], 1e-5, &h));
    {
        const chelis_gpu_tensor *wqkv[3] = {P[2], P[4], P[6]}, *bqkv[3] = {P[3], P[5], P[7]};
        const Pkt qkv3(qkv, dt, {3, R, D});
        TRY(linear_multi_b(&h.t, wqkv, bqkv, 3, &qkv3.t));
    }
    const Pkt kh(k.t.data, dt, {B, H, S, DH}, {S * D, DH, D, 1}, cap);
    if (fused && attention_causal_fits(&qh.t, &kh.t, &vh.t, &oh.t)) {
        TRY(attention_causal(&qh.t, &kh.t, &vh.t, 1.0 / 8.0, &oh.t));
    } else {
        // causal: score tiles above the diagonal are masked to -inf by the
        // softmax without being read, and P is exactly +0 there, so those
        // tiles and contraction terms are skipped
        if (fused) return set_error(CHELIS_HIP_EUNSUPPORTED, "transformer_block: attention operands misaligned");
        TRY(matmul_causal(&qh, &kt, &s, 1));
        TRY(chelis_hip_scaled_masked_softmax(&s, 1.0 / 8.0, 1, &s));
        TRY(matmul_causal(&s, &vh, &oh, 2));
    }
    TRY(chelis_hip_linear(&o, P[8], P[9], CHELIS_ACT_NONE, &x2, &x1, 0));
    // feed-forward
    TRY(chelis_hip_layer_norm(&x1, P[10], P[11], 1e-5, &h));
    TRY(chelis_hip_linear(&h, P[12], P[13], CHELIS_ACT_GELU, nullptr, &f, 0));
    TRY(chelis_hip_linear(&f, P[14], P[15], CHELIS_ACT_NONE, &x1, &y2, 0));
    return CHELIS_HIP_OK;
}

// ------------------------------------------------------------------ MLP train step
namespace {

// The step in five launches: x.W1 as raw K slices, the head and the tail
// of the narrow part (k_mlp.hip), x^T.g_d as raw K slices, and the finish
// (W1 update from the slices, the tail's join, the other updates, the loss).
int32_t mlp_fused(const chelis_gpu_tensor *x, const chelis_gpu_tensor *oh, const chelis_gpu_tensor *w1,
                  const chelis_gpu_tensor *b1, const chelis_gpu_tensor *w2, const chelis_gpu_tensor *b2,
                  const uint64_t *kdev, const chelis_gpu_tensor *const *out, int64_t Bt, int64_t I, int64_t Hd,
                  int64_t O, float rate, float lr, hipStream_t st) {
    const chelis_dtype dt = CHELIS_DTYPE_F32;
    const Pkt xT(x->data, dt, {I, Bt}, {x->strides[1], x->strides[0]}, x->byte_capacity);
    Workspace ws(st);
    const size_t o_d = ws.reserve(Bt * Hd * 4), o_gd = ws.reserve(Bt * Hd * 4), o_gz2 = ws.reserve(Bt * O * 4),
                 o_nl = ws.reserve(Bt * 4), o_part = ws.reserve(mlp_part_bytes(Bt, Hd));
    // the slice count reads only shapes: any non-null address stands in for g_d
    const Pkt gd_probe(x->data, dt, {Bt, Hd});
    const int64_t ks1 = matmul_slice_count(x, w1), ks2 = matmul_slice_count(&xT.t, &gd_probe.t);
    const size_t o_z1 = ws.reserve(ks1 * Bt * Hd * 4), o_gw1 = ws.reserve(ks2 * I * Hd * 4);
    TRY(ws.commit());
    const Pkt gd(ws.at(o_gd), dt, {Bt, Hd});
    MlpNarrow m{};
    m.B = Bt, m.I = I, m.H = Hd, m.O = O;
    m.z1 = static_cast<const float *>(ws.at(o_z1)), m.z1_slices = ks1;
    m.gw1 = static_cast<const float *>(ws.at(o_gw1)), m.gw1_slices = ks2;
    m.w1 = static_cast<const float *>(w1->data), m.w2 = static_cast<const float *>(w2->data);
    m.b2 = static_cast<const float *>(b2->data), m.onehot = static_cast<const float *>(oh->data);
    m.b1 = static_cast<const float *>(b1->data), m.key = kdev;
    m.d = static_cast<float *>(ws.at(o_d)), m.gz2 = static_cast<float *>(ws.at(o_gz2));
    m.nl = static_cast<float *>(ws.at(o_nl)), m.gd = static_cast<float *>(gd.t.data);
    m.part = static_cast<float *>(ws.at(o_part));
    m.w1_out = static_cast<float *>(out[1]->data), m.b1_out = static_cast<float *>(out[2]->data);
    m.w2_out = static_cast<float *>(out[3]->data), m.b2_out = static_cast<float *>(out[4]->data);
    m.loss = static_cast<float *>(out[0]->data);
    m.rate = rate, m.lr = lr;
    TRY(matmul_slices(x, w1, ws.at(o_z1), ks1));
    TRY(mlp_head_tail(m, st));
    TRY(matmul_slices(&xT.t, &gd.t, ws.at(o_gw1), ks2));
    return mlp_finish(m, st);
}

}  // namespace

extern "C" int32_t chelis_prog_mlp_train_step(const chelis_gpu_tensor *const *in, int32_t n_in,
                                              const chelis_gpu_tensor *const *out, int32_t n_out) {
    // the configuration's dropout rate and learning rate (mnist.ch form)
    return chelis::mlp_train_step_run(in, n_in, out, n_out, 0.1f, 0.01f);
}

int32_t chelis::mlp_train_step_run(const chelis_gpu_tensor *const *in, int32_t n_in,
                                   const chelis_gpu_tensor *const *out, int32_t n_out, float rate, float lr) {
    const ModeScope mode;
    if (n_in != 7 || n_out != 5) return set_error(CHELIS_HIP_EDOMAIN, "mlp_train_step: 7 inputs, 5 outputs");
    TRY(check_all(in, 7, "mlp_train_step input"));
    TRY(check_all(out, 5, "mlp_train_step output"));
    const chelis_gpu_tensor *x = in[0], *oh = in[1], *w1 = in[2], *b1 = in[3], *w2 = in[4], *b2 = in[5], *key = in[6];
    const chelis_dtype dt = CHELIS_DTYPE_F32;
    if (x->rank != 2 || w1->rank != 2 || w2->rank != 2)
        return set_error(CHELIS_HIP_EDOMAIN, "mlp_train_step: x, w1, w2 must be matrices");
    const int64_t Bt = x->shape[0], I = x->shape[1], Hd = w1->shape[1], O = w2->shape[1];
    const bool ok = shape_is(x, {Bt, I}, dt) && shape_is(oh, {Bt, O}, dt) && shape_is(w1, {I, Hd}, dt) &&
                    shape_is(b1, {Hd}, dt) && shape_is(w2, {Hd, O}, dt) && shape_is(b2, {O}, dt) &&
                    shape_is(key, {}, CHELIS_DTYPE_KEY) && shape_is(out[0], {}, dt) && shape_is(out[1], {I, Hd}, dt) &&
                    shape_is(out[2], {Hd}, dt) && shape_is(out[3], {Hd, O}, dt) && shape_is(out[4], {O}, dt);
    if (!ok) return set_error(CHELIS_HIP_EDOMAIN, "mlp_train_step: shapes/dtypes do not match the program");
    for (int32_t i = 1; i < 5; ++i)
        if (!is_contiguous(out[i])) return set_error(CHELIS_HIP_EUNSUPPORTED, "mlp_train_step: outputs must be contiguous");
    if (!(rate >= 0.0f && rate < 1.0f)) return set_error(CHELIS_HIP_EDOMAIN, "mlp_train_step: rate outside [0, 1)");
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    // the dropout kernels read the key from its tensor on the device
    const uint64_t *kdev = static_cast<const uint64_t *>(key->data);
    if (mlp_narrow_fits(Bt, I, Hd, O) && is_contiguous(oh) && is_contiguous(w1) && is_contiguous(w2) &&
        is_contiguous(b1) && is_contiguous(b2))
        return mlp_fused(x, oh, w1, b1, w2, b2, kdev, out, Bt, I, Hd, O, rate, lr, st);
    Workspace ws(st);
    const size_t o_hd = ws.reserve(Bt * Hd * 4), o_d = ws.reserve(Bt * Hd * 4), o_z2 = ws.reserve(Bt * O * 4),
                 o_p = ws.reserve(Bt * O * 4), o_nl = ws.reserve(Bt * 4), o_gp = ws.reserve(Bt * O * 4),
                 o_gz2 = ws.reserve(Bt * O * 4), o_gd = ws.reserve(Bt * Hd * 4), o_gw2 = ws.reserve(Hd * O * 4),
                 o_gb2 = ws.reserve(O * 4), o_gw1 = ws.reserve(I * Hd * 4), o_gb1 = ws.reserve(Hd * 4),
                 o_tot = ws.reserve(4);
    TRY(ws.commit());
    const Pkt hd(ws.at(o_hd), dt, {Bt, Hd}), d(ws.at(o_d), dt, {Bt, Hd}), z2(ws.at(o_z2), dt, {Bt, O}),
        p(ws.at(o_p), dt, {Bt, O}), nl(ws.at(o_nl), dt, {Bt}), gp(ws.at(o_gp), dt, {Bt, O}),
        gz2(ws.at(o_gz2), dt, {Bt, O}), gd(ws.at(o_gd), dt, {Bt, Hd}), gw2(ws.at(o_gw2), dt, {Hd, O}),
        gb2(ws.at(o_gb2), dt, {O}), gw1(ws.at(o_gw1), dt, {I, Hd}), gb1(ws.at(o_gb1), dt, {Hd}),
        tot(ws.at(o_tot), dt, {});
    const Pkt dT(d.t.data, dt, {Hd, Bt}, {1, Hd}, Bt * Hd * 4);
    const Pkt w2T(w2->data, dt, {O, Hd}, {w2->strides[1], w2->strides[0]}, w2->byte_capacity);
    const Pkt xT(x->data, dt, {I, Bt}, {x->strides[1], x->strides[0]}, x->byte_capacity);
    // forward: hd = relu(x.w1 + b1); d = dropout(hd); z2 = d.w2 + b2; p = softmax(z2)
    TRY(chelis_hip_linear(x, w1, b1, CHELIS_ACT_RELU, nullptr, &hd, 0));
    TRY(dropout_device_key(kdev, &hd, rate, &d));
    TRY(chelis_hip_linear(&d, w2, b2, CHELIS_ACT_NONE, nullptr, &z2, 0));
    TRY(chelis_hip_softmax(&z2, &p));
    // loss = mean(-sum(log(p) * onehot, 1))
    const chelis_fused_chain lpo = chain({step(CHELIS_FUSED_LOG, 0), step(CHELIS_FUSED_MUL, prev(0), 1)});
    const chelis_gpu_tensor *po[2] = {&p, oh};
    TRY(chelis_hip_reduce(CHELIS_REDUCE_SUM, &lpo, po, 2, 1, &nl));
    const chelis_fused_chain neg = chain({step(CHELIS_FUSED_NEG, 0)});
    const chelis_gpu_tensor *nl1[1] = {&nl};
    TRY(chelis_hip_fused_elementwise(&neg, nl1, 1, &nl));
    const chelis_gpu_tensor *nl2[1] = {&nl};
    TRY(chelis_hip_reduce(CHELIS_REDUCE_SUM, nullptr, nl2, 1, 0, &tot));
    TRY(divide_by(&tot, (double)Bt, out[0]));
    // backward: g_p = (-(1/B) * onehot) / p; g_z2 = p * (g_p - sum(g_p * p))
    const float g_nl = 1.0f / (float)Bt;
    const chelis_fused_chain gpc =
        chain({step(CHELIS_FUSED_CONST, 0, 0, (double)(-g_nl)), step(CHELIS_FUSED_MUL, prev(0), 0),
               step(CHELIS_FUSED_DIV, prev(1), 1)});
    const chelis_gpu_tensor *op[2] = {oh, &p};
    TRY(chelis_hip_fused_elementwise(&gpc, op, 2, &gp));
    TRY(chelis_hip_softmax_adjoint(&p, &gp, &gz2));
    const chelis_gpu_tensor *g2[1] = {&gz2};
    TRY(chelis_hip_reduce(CHELIS_REDUCE_SUM, nullptr, g2, 1, 0, &gb2));
    TRY(chelis_hip_matmul(&dT, &gz2, &gw2, 0));
    TRY(chelis_hip_matmul(&gz2, &w2T, &gd, 0));
    TRY(dropout_device_key(kdev, &gd, rate, &gd));
    TRY(chelis_hip_relu_adjoint(&hd, &gd, &gd));
    const chelis_gpu_tensor *g1[1] = {&gd};
    TRY(chelis_hip_reduce(CHELIS_REDUCE_SUM, nullptr, g1, 1, 0, &gb1));
    TRY(chelis_hip_matmul(&xT, &gd, &gw1, 0));
    // SGD: w' = w - lr * g
    const chelis_fused_chain sgd =
        chain({step(CHELIS_FUSED_CONST, 0, 0, (double)lr), step(CHELIS_FUSED_MUL, prev(0), 1),
               step(CHELIS_FUSED_SUB, 0, prev(1))});
    // the four parameter updates in one launch
    const chelis_gpu_tensor *pin[8] = {w1, &gw1, b1, &gb1, w2, &gw2, b2, &gb2};
    TRY(fused_elementwise_groups(&sgd, 2, pin, out + 1, 4));
    return CHELIS_HIP_OK;
}

// ------------------------------------------------------------------ generated-entry form
namespace {

[[noreturn]] void entry_trap(const char *what) {
    std::fprintf(stderr, "numeric trap: domain in %s at device entry: %s\n", what, chelis_hip_last_error());
    chelis_flush_and_exit_trap();
    std::abort();
}

using Prog = int32_t (*)(const chelis_gpu_tensor *const *, int32_t, const chelis_gpu_tensor *const *, int32_t);

chelis_device_tensor_owner *alloc_like(const std::vector<int64_t> &shape, chelis_dtype dt) {
    std::vector<chelis_scalar> sh;
    for (int64_t e : shape) sh.push_back(chelis_scalar_from_bits(CHELIS_DTYPE_I64, (uint64_t)e));
    chelis_scalar ex{};
    ex.dtype = dt;
    chelis_metadata_plan *plan = chelis_metadata_plan_new(
        chelis_scalar_from_bits(CHELIS_DTYPE_I64, (uint64_t)shape.size()), sh.empty() ? nullptr : sh.data(), ex);
    return chelis_device_tensor_alloc(plan);
}

// Run `prog` with inputs borrowed from owners and outputs freshly
// allocated with the given shapes; synchronizes before returning.
void run_entry(const char *what, Prog prog, const chelis_device_tensor_owner *const *inputs, int32_t n_in,
               chelis_device_tensor_owner **outputs, int32_t n_out,
               const std::vector<std::pair<std::vector<int64_t>, chelis_dtype>> &out_shapes) {
    if (!inputs || !outputs || n_out != (int32_t)out_shapes.size()) entry_trap(what);
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) entry_trap(what);
    std::vector<const chelis_gpu_tensor *> in(n_in);
    for (int32_t i = 0; i < n_in; ++i) {
        if (!inputs[i] || chelis_device_tensor_device(inputs[i]) != dev) entry_trap(what);
        in[i] = chelis_device_tensor_view(inputs[i]);
    }
    std::vector<const chelis_gpu_tensor *> outp(n_out);
    for (int32_t i = 0; i < n_out; ++i) {
        outputs[i] = alloc_like(out_shapes[i].first, out_shapes[i].second);
        outp[i] = chelis_device_tensor_view(outputs[i]);
    }
    if (prog(in.data(), n_in, outp.data(), n_out) != CHELIS_HIP_OK) entry_trap(what);
    if (chelis_hip_synchronize() != CHELIS_HIP_OK) entry_trap(what);
}

std::vector<int64_t> dims(const chelis_device_tensor_owner *o) {
    const chelis_gpu_tensor *t = chelis_device_tensor_view(o);
    return std::vector<int64_t>(t->shape, t->shape + t->rank);
}

}  // namespace

extern "C" void linreg_step_device(const chelis_device_tensor_owner *const *inputs, chelis_device_rank n_in,
                                   chelis_device_tensor_owner **outputs, chelis_device_rank n_out) {
    if (!inputs || n_in != 3 || !inputs[0]) entry_trap("linreg_step");
    const chelis_gpu_tensor *X = chelis_device_tensor_view(inputs[0]);
    if (X->rank != 2) entry_trap("linreg_step");
    run_entry("linreg_step", chelis_prog_linreg_step, inputs, n_in, outputs, n_out,
              {{{X->shape[1]}, X->dtype}, {{}, X->dtype}});
}

extern "C" void transformer_block_device(const chelis_device_tensor_owner *const *inputs, chelis_device_rank n_in,
                                         chelis_device_tensor_owner **outputs, chelis_device_rank n_out) {
    if (!inputs || n_in != 17 || !inputs[0]) entry_trap("transformer_block");
    run_entry("transformer_block", chelis_prog_transformer_block, inputs, n_in, outputs, n_out,
              {{dims(inputs[0]), chelis_device_tensor_view(inputs[0])->dtype}});
}

extern "C" void mlp_train_step_device(const chelis_device_tensor_owner *const *inputs, chelis_device_rank n_in,
                                      chelis_device_tensor_owner **outputs, chelis_device_rank n_out) {
    if (!inputs || n_in != 7) entry_trap("mlp_train_step");
    for (int32_t i = 0; i < 6; ++i)
        if (!inputs[i]) entry_trap("mlp_train_step");
    run_entry("mlp_train_step", chelis_prog_mlp_train_step, inputs, n_in, outputs, n_out,
              {{{}, CHELIS_DTYPE_F32},
               {dims(inputs[2]), CHELIS_DTYPE_F32},
               {dims(inputs[3]), CHELIS_DTYPE_F32},
               {dims(inputs[4]), CHELIS_DTYPE_F32},
               {dims(inputs[5]), CHELIS_DTYPE_F32}});
}

// ------------------------------------------------------------------ host-tensor entry form
// The generated `{f}(chelis_tensor **inputs, int n_in, chelis_tensor
// **outputs, int n_out)` (crates/chelis-backend-hip/src/emit.rs:667-808):
// a wrong count prints `{f}: expected N inputs, got M` and aborts; each
// host input is copied into a fresh device tensor (the PCIe crossing of a
// Load); the program runs as its `{f}_device` entry; each result comes back
// as a new host tensor from chelis_alloc, written under its write lease;
// the device is synchronized and every device tensor released before the
// call returns. Inputs stay owned by the caller.
namespace {

using DeviceEntry = void (*)(const chelis_device_tensor_owner *const *, chelis_device_rank,
                             chelis_device_tensor_owner **, chelis_device_rank);

void run_host_entry(const char *name, DeviceEntry entry, int expected_in, int expected_out, chelis_tensor **inputs,
                    int n_in, chelis_tensor **outputs, int n_out) {
    if (n_in != expected_in) {
        std::fprintf(stderr, "%s: expected %d inputs, got %d\n", name, expected_in, n_in);
        std::abort();
    }
    if (n_out != expected_out) {
        std::fprintf(stderr, "%s: expected %d outputs, got %d\n", name, expected_out, n_out);
        std::abort();
    }
    if (!inputs || !outputs) entry_trap(name);
    std::vector<chelis_device_tensor_owner *> device_in(n_in, nullptr);
    for (int i = 0; i < n_in; ++i) {
        const chelis_tensor *t = inputs[i];
        const int32_t rank = chelis_tensor_rank(t);
        std::vector<int64_t> shape(rank);
        for (int32_t a = 0; a < rank; ++a) shape[a] = chelis_tensor_shape(t, a);
        device_in[i] = alloc_like(shape, chelis_tensor_read_view(t).dtype);
        chelis_device_tensor_copy_from_host(device_in[i], t);
    }
    std::vector<chelis_device_tensor_owner *> device_out(n_out, nullptr);
    entry(device_in.data(), n_in, device_out.data(), n_out);
    for (int o = 0; o < n_out; ++o) {
        const chelis_gpu_tensor *v = chelis_device_tensor_view(device_out[o]);
        outputs[o] = chelis_alloc(v->rank, v->rank ? v->shape : nullptr, v->dtype);
        chelis_tensor_write *lease = chelis_tensor_begin_write(outputs[o]);
        chelis_device_tensor_copy_to_host(lease, device_out[o]);
        chelis_tensor_end_write(lease);
    }
    if (hipDeviceSynchronize() != hipSuccess) entry_trap(name);
    for (chelis_device_tensor_owner *t : device_out) chelis_device_tensor_release(t);
    for (chelis_device_tensor_owner *t : device_in) chelis_device_tensor_release(t);
}

}  // namespace

extern "C" void linreg_step(chelis_tensor **inputs, int n_in, chelis_tensor **outputs, int n_out) {
    run_host_entry("linreg_step", linreg_step_device, 3, 2, inputs, n_in, outputs, n_out);
}

extern "C" void transformer_block(chelis_tensor **inputs, int n_in, chelis_tensor **outputs, int n_out) {
    run_host_entry("transformer_block", transformer_block_device, 17, 1, inputs, n_in, outputs, n_out);
}

extern "C" void mlp_train_step(chelis_tensor **inputs, int n_in, chelis_tensor **outputs, int n_out) {
    run_host_entry("mlp_train_step", mlp_train_step_device, 7, 5, inputs, n_in, outputs, n_out);
}
