// The MLP training step (config 5) between and after its two wide products
// in three launches, bit-identical to the unfused launches they replace
// (and so to the C lane wherever those are):
//   head, one wave per batch row b, from x.W1's raw K slices:
//     hd = relu(sum_s z1[s] + b1)                     (the split-K combine and
//                                                      the linear epilogue)
//     d = dropout(key, hd, rate)
//     z2 = d.W2 + b2;  p = softmax(z2)
//     nl = -sum(log(p) * onehot);  g_p = (-(1/B) * onehot) / p
//     g_z2 = p * (g_p - sum(g_p * p))                 (softmax adjoint)
//     g_d = relu_adjoint(hd, dropout_replay(key, g_z2.W2^T))
//   tail, per 64-row block: its partial column sums of d^T.g_z2, g_d, g_z2
//     and nl;
//   finish, after x^T.g_d (raw K slices):
//     W1' = W1 - lr * sum_s gw1[s];  the row blocks of the tail joined:
//     W2' = W2 - lr * d^T.g_z2;  b1' = b1 - lr * sum_b g_d;
//     b2' = b2 - lr * sum_b g_z2;  loss = sum_b nl / B.
// Every sum is the canonical adjacent-pair tree over its leaves in index
// order, which equals the complete power-of-two tree over the leaves padded
// with -0.0 at the end (x + (-0.0) = x for every x): in-lane register trees
// over aligned runs, wave butterflies (wave_tree_sum) over 64 runs, aligned
// 64-row blocks joined as runs of sixteen and a carry stack. Every stored
// value is finalized with the canonical NaN, as the primitive it restates
// stores it.
//
// The kernels run once per compute unit and are bound by latency, not
// bandwidth: every global load a phase needs is issued before the first is
// used (a round trip to memory costs about a microsecond), loops over
// classes stay rolled and the per-element leaves (keyed unit, exp, log) are
// out-of-line calls, which keeps the code the units fetch cold to a few KiB.
#include "chain.h"
#include "gemm.h"

namespace chelis {
namespace {

constexpr int kMaxClasses = 16;      // classes a head lane row holds (padded tree of 16)
constexpr int kMaxRun = 16;          // hidden units per head lane: H <= 1024
constexpr int kW2Floats = kMaxClasses * 64 * kMaxRun;  // W2 staged in LDS: 64 KiB
constexpr int kOuts = kMaxClasses + 1;                 // tail outputs per hidden unit
constexpr int kJoinLevels = 12;      // carry stack over runs of 16 row blocks

struct MlpArgs {
    const float *z1, *w1, *w2, *b2, *oh, *b1, *gw1;
    const uint64_t *key;
    float *d, *gz2, *nl, *gd, *part;
    float *w1o, *w2o, *b1o, *b2o, *loss;
    int64_t B, H, I, z1_slices, gw1_slices, blocks;
    int O;
    bool vec;  // z1 slices, d and g_d rows load and store as float4
    float rate, g_pr, lr;
    uint64_t cut;  // dropout: keep when word >> 11 is at least this (dropout_cut)
    double inv_keep, inv_batch;
};

// Complete tree over N (a power of two) register values, adjacent pairs first.
template <int N>
__device__ inline float reg_tree(float (&a)[N]) {
#pragma unroll
    for (int s = 1; s < N; s <<= 1)
#pragma unroll
        for (int k = 0; k + s < N; k += 2 * s) a[k] = a[k] + a[k + s];
    return a[0];
}

// Reads through a buffer resource. The compiler turns `ok ? p[i] : x` into
// a branch around the load, with the wait for it inside, which serializes
// a run of such loads; a buffer load is never moved into a branch, so a
// run of them is issued back to back. Callers keep every index inside the
// buffer (no reliance on the out-of-range rule).
struct BufRead {
    __amdgpu_buffer_rsrc_t r;
    __device__ BufRead(const void *p, int64_t bytes)
        : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000)) {}
    __device__ float operator[](int64_t i) const {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)(i * 4), 0, 0));
    }
};

// Quotient at binary32: (double)v * (1 / (double)t) rounded once is the
// correctly rounded v / t (the quotient of two binary32 values is never
// within 2^-49 relative of a binary32 rounding midpoint).
__device__ inline float div32(float v, float t) { return quot_f32(v, 1.0 / (double)t); }

// Canonical tree over the 16 lanes of each DPP row (the first four levels
// of wave_tree_sum): every lane gets its row's total.
__device__ inline float row16_tree_sum(float x) {
    x = x + dpp_perm<kDppXor1>(x);
    x = x + dpp_perm<kDppXor2>(x);
    x = x + dpp_perm<kDppHalfMirror>(x);
    x = x + dpp_perm<kDppMirror>(x);
    return x;
}

__device__ inline float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// the word's top 53 bits, compared with the dropout cut-off (dropout_cut)
__device__ __noinline__ uint64_t word53(uint64_t key, uint64_t index) { return random_word(key, index) >> 11; }
// exp of x - max (<= 0 or NaN), correctly rounded
__device__ __noinline__ float exp_class(float x) { return expf_cr_nonpos(x); }
__device__ __noinline__ float log_class(float x) { return leaf_log<float>(x); }

// Raw x.W1 sums for row b, this lane's run, slice by slice: NS > 0 slices
// read together (every load issued before the first is used); NS = 0, any
// count, one slice after another into raw[0].
template <int L, int NS>
struct RawRun {
    float v[NS > 0 ? NS : 1][L];
};

template <int L>
__device__ inline void load_slice(const MlpArgs &a, const float *row, int64_t k0, bool vec, float (&v)[L]) {
    if (vec) {
#pragma unroll
        for (int i = 0; i < L; i += 4) {
            float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k0 + i < a.H) q = *reinterpret_cast<const float4 *>(row + i);
            v[i] = q.x, v[i + 1] = q.y, v[i + 2] = q.z, v[i + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < L; ++i) v[i] = k0 + i < a.H ? row[i] : 0.f;
    }
}

template <int L, int NS>
__device__ inline void load_raw(const MlpArgs &a, int64_t b, int64_t k0, bool vec, RawRun<L, NS> &r) {
    const float *row = a.z1 + b * a.H + k0;
    const int64_t slice = a.B * a.H;
    if constexpr (NS > 0) {
#pragma unroll
        for (int s = 0; s < NS; ++s) load_slice<L>(a, row + s * slice, k0, vec, r.v[s]);
    } else {
        load_slice<L>(a, row, k0, vec, r.v[0]);
        for (int64_t s = 1; s < a.z1_slices; ++s) {
            float t[L];
            load_slice<L>(a, row + s * slice, k0, vec, t);
#pragma unroll
            for (int i = 0; i < L; ++i) r.v[0][i] += t[i];
        }
    }
}

// hd: the slices added in slice order, then the linear epilogue (canon,
// + b1, relu) as the split-K combine applies it.
template <int L, int NS>
__device__ inline void hidden_run(const RawRun<L, NS> &r, const float (&b1v)[L], float (&hv)[L]) {
#pragma unroll
    for (int i = 0; i < L; ++i) {
        float acc = r.v[0][i];
#pragma unroll
        for (int s = 1; s < NS; ++s) acc += r.v[s][i];
        const float v = canon(canon(acc) + b1v[i]);
        hv[i] = v < 0.f ? 0.f : v;
    }
}

template <int L>
__device__ inline void store_run(float *row, int64_t H, int64_t k0, bool vec, const float (&v)[L]) {
    if (vec) {
#pragma unroll
        for (int i = 0; i < L; i += 4)
            if (k0 + i < H) *reinterpret_cast<float4 *>(row + k0 + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
    } else {
#pragma unroll
        for (int i = 0; i < L; ++i)
            if (k0 + i < H) row[k0 + i] = v[i];
    }
}

// One wave per batch row; lane l holds hidden units [l L, l L + L). The
// per-class steps (exp, log, the quotients) run once per class: class c in
// lane c of each 16-lane row, its row sums by row16_tree_sum.
template <int L, int NS>
__global__ __launch_bounds__(256) void mlp_head_kernel(MlpArgs a) {
    // W2 transposed as [class][i][lane]: hidden unit l L + i of class c at
    // c 64 L + i 64 + l, so a wave's reads of one (c, i) are 64 consecutive
    // words; -0.0 past H and for classes past O
    __shared__ float w2t[kW2Floats];
    __shared__ float b2s[kMaxClasses];
    constexpr int64_t HP = 64 * L;
    const int lane = threadIdx.x & 63, cl = lane & 15;
    const int64_t H = a.H;
    const int O = a.O;
    const int64_t k0 = (int64_t)lane * L;
    const bool vec = a.vec && L >= 4;
    int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    // set-up loads together: the first row's slices and one-hot entry (a
    // clamped row: no branch), b1 for this lane's run, the key, this
    // thread's W2 values, b2
    RawRun<L, NS> raw;
    const int64_t b_first = b < a.B ? b : a.B - 1;
    load_raw<L, NS>(a, b_first, k0, vec, raw);
    float ohv = a.oh[b_first * O + (cl < O ? cl : 0)];
    const BufRead b1b(a.b1, H * 4), w2b(a.w2, H * O * 4), b2b(a.b2, O * 4);
    float b1v[L];
#pragma unroll
    for (int i = 0; i < L; ++i) b1v[i] = b1b[k0 + i < H ? k0 + i : 0];
    const uint64_t key = *a.key;
    constexpr int kStage = (int)((HP + 255) / 256);
    float w2v[kStage][kMaxClasses];
#pragma unroll
    for (int it = 0; it < kStage; ++it) {
        const int64_t k = threadIdx.x + 256 * it;
#pragma unroll
        for (int c = 0; c < kMaxClasses; ++c) {
            const bool ok = c < O && k < H;
            const float v = w2b[ok ? k * O + c : 0];
            w2v[it][c] = ok ? v : -0.0f;
        }
    }
    const float b2v = b2b[threadIdx.x < O ? threadIdx.x : 0];
#pragma unroll
    for (int it = 0; it < kStage; ++it) {
        const int64_t k = threadIdx.x + 256 * it;
#pragma unroll
        for (int c = 0; c < kMaxClasses; ++c)
            if (k < HP) w2t[c * HP + (k % L) * 64 + k / L] = w2v[it][c];
    }
    if (threadIdx.x < kMaxClasses) b2s[threadIdx.x] = threadIdx.x < O ? b2v : 0.f;
    __syncthreads();
#pragma unroll 1
    for (; b < a.B; b += (int64_t)gridDim.x * 4) {
        float hv[L];
        hidden_run<L, NS>(raw, b1v, hv);
        const float ohc = cl < O ? ohv : 0.f;
        // dropout: mask and d for this lane's run
        float dv[L];
        uint32_t keep = 0;
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const bool kp = word53(key, (uint64_t)(b * H + k0 + i)) >= a.cut;
            keep |= (uint32_t)kp << i;
            dv[i] = kp ? canon(quot_f32(hv[i], a.inv_keep)) : 0.f;
        }
        store_run<L>(a.d + b * H, H, k0, vec, dv);
        // z2 = d.W2 + b2: per class, L products in a register tree, the wave
        // tree over the 64 runs (-0.0 past H); class c kept by lanes c mod 16
        float zc = 0.f, m = 0.f;
        bool mnan = false;
#pragma unroll 1
        for (int c = 0; c < O; ++c) {
            float t[L];
#pragma unroll
            for (int i = 0; i < L; ++i) t[i] = k0 + i < H ? dv[i] * w2t[c * HP + i * 64 + lane] : -0.0f;
            const float s = wave_tree_sum(reg_tree<L>(t));
            const float z = canon(canon(s) + b2s[c]);
            if (cl == c) zc = z;
            // [05-OP-12] max_reduce in class order: the first NaN, else the
            // maximum keeping the first representation among equals
            if (c == 0) {
                m = z;
                mnan = z != z;
            } else if (!mnan) {
                if (z != z) {
                    m = z;
                    mnan = true;
                } else if (z > m) {
                    m = z;
                }
            }
        }
        const bool in = cl < O;
        // softmax: exp(x - m), tree sum, quotient
        const float e = in ? exp_class(canon(zc - m)) : -0.0f;
        const float se = canon(row16_tree_sum(e));
        const float p = in ? canon(div32(e, se)) : 0.f;
        // nl = -tree(log(p) * onehot); g_p = (g_pr * onehot) / p
        const float lp = in ? canon(log_class(p) * ohc) : -0.0f;
        const float nl = canon(-row16_tree_sum(lp));
        const float gp = in ? canon(div32(canon(a.g_pr * ohc), p)) : 0.f;
        // softmax adjoint: p * (g_p - tree(g_p * p))
        const float sg = canon(row16_tree_sum(in ? canon(gp * p) : -0.0f));
        const float gz = in ? canon(p * canon(gp - sg)) : 0.f;
        if (lane < O) a.gz2[b * O + lane] = gz;
        if (lane == 0) a.nl[b] = nl;
        // g_d = g_z2.W2^T (tree over the classes, W2 -0.0 past O), dropout
        // replay, relu adjoint
        float gzs[kMaxClasses];
#pragma unroll
        for (int c = 0; c < kMaxClasses; ++c) gzs[c] = lane_value(gz, c);
        float gv[L];
#pragma unroll
        for (int i = 0; i < L; ++i) {
            float t[kMaxClasses];
#pragma unroll
            for (int c = 0; c < kMaxClasses; ++c) t[c] = gzs[c] * w2t[c * HP + i * 64 + lane];
            const float g = canon(reg_tree<kMaxClasses>(t));
            const float r = (keep >> i) & 1 ? canon(quot_f32(g, a.inv_keep)) : 0.f;
            gv[i] = 0.f < hv[i] ? r : 0.f;
        }
        store_run<L>(a.gd + b * H, H, k0, vec, gv);
        const int64_t bn = b + (int64_t)gridDim.x * 4;
        if (bn < a.B) {
            load_raw<L, NS>(a, bn, k0, vec, raw);
            ohv = a.oh[bn * O + (cl < O ? cl : 0)];
        }
    }
}

// Tail: workgroup (g, rb) sums rows [64 rb, 64 rb + 64) for column group g.
// Groups 0 .. G-2 hold hidden units [64 g, 64 g + 64) on the lanes with
// O + 1 outputs each (d^T.g_z2 per class, then sum g_d), the waves taking
// every fourth output; group G-1 holds sum g_z2 (lane c < O) and sum nl
// (lane O). Block totals go to part[g][rb][output][lane] (a wave's stores
// and the join's loads run along the lanes).
__global__ __launch_bounds__(256) void mlp_tail_kernel(MlpArgs a) {
    __shared__ float gzs[64][kOuts];
    __shared__ float tile[2][64][64];  // d and g_d rows of this block, this group's columns
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int O = a.O;
    const int64_t blocks = a.blocks;
    const int g = blockIdx.x, groups = gridDim.x;
    const bool extra = g == groups - 1;
    const int64_t rb = blockIdx.y, b0 = rb * 64;
    const int nrows = (int)min<int64_t>(64, a.B - b0);
    const int outs = extra ? 1 : O + 1;
    // stage g_z2 | nl rows, and the d and g_d tiles (0 past B and H); every
    // load is issued (at a valid address) before the first is used
    constexpr int kGz = (64 * kOuts + 255) / 256;
    const BufRead gzb(a.gz2, a.B * O * 4), nlb(a.nl, a.B * 4), db(a.d, a.B * a.H * 4), gdb(a.gd, a.B * a.H * 4);
    float gv[kGz];
#pragma unroll
    for (int u = 0; u < kGz; ++u) {
        const int e = threadIdx.x + 256 * u, r = e / kOuts, c = e % kOuts;
        const bool row = e < 64 * kOuts && r < nrows;
        const int64_t br = b0 + (row ? r : 0);
        const float xg = gzb[br * O + (c < O ? c : 0)], xn = nlb[br];
        gv[u] = row && c < O ? xg : (row && c == O ? xn : 0.f);
    }
    float dt[16], gt[16];
    const int64_t k = (int64_t)g * 64 + lane;
    const bool kin = !extra && k < a.H;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = wave + 4 * i;
        const bool ok = kin && r < nrows;
        const int64_t at = ok ? (b0 + r) * a.H + k : 0;
        const float x = db[at], y = gdb[at];
        dt[i] = ok ? x : 0.f;
        gt[i] = ok ? y : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kGz; ++u) {
        const int e = threadIdx.x + 256 * u;
        if (e < 64 * kOuts) gzs[e / kOuts][e % kOuts] = gv[u];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        tile[0][wave + 4 * i][lane] = dt[i];
        tile[1][wave + 4 * i][lane] = gt[i];
    }
    __syncthreads();
    float *part = a.part + (int64_t)g * kOuts * 64 * blocks;
    // a 64-leaf tree per output: four aligned 16-leaf register trees, then
    // (t0 + t1) + (t2 + t3); leaves past the rows are -0.0. Leaf r is
    // x[r] * f[r]: for d^T.g_z2, x the d tile and f the class column of
    // g_z2; for a plain sum f is 1 (x * 1 = x for every x, NaN aside, and
    // a NaN leaf makes the total NaN either way).
    for (int j = wave; j < outs; j += 4) {
        const bool mul = !extra && j < O;
        const float *xs = extra ? &gzs[0][lane <= O ? lane : O] : &tile[mul ? 0 : 1][0][lane];
        const int sx = extra ? kOuts : 64;
        const float *fs = &gzs[0][mul ? j : 0];
        float q[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            float t[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = h * 16 + i;
                const float f = fs[r * kOuts];
                const float leaf = xs[r * sx] * (mul ? f : 1.0f);
                t[i] = r < nrows ? leaf : -0.0f;
            }
            q[h] = reg_tree<16>(t);
        }
        part[(rb * kOuts + j) * 64 + lane] = (q[0] + q[1]) + (q[2] + q[3]);
    }
}

// Leaf i of a tree whose completed subtrees wait in lv (a carry stack of
// LV levels: leaf i absorbs one waiting subtree per trailing one bit; i <
// 2^LV - 1, so some level below LV takes the carry).
template <int LV>
__device__ inline void push_leaf(float (&lv)[LV], int64_t i, float carry) {
    bool done = false;
#pragma unroll
    for (int d = 0; d < LV; ++d) {
        if (!done) {
            if ((i >> d) & 1) {
                carry = lv[d] + carry;
            } else {
                lv[d] = carry;
                done = true;
            }
        }
    }
}

// The carry stack's total after n leaves: waiting subtrees folded lowest
// level (rightmost) first.
template <int LV>
__device__ inline float stack_total(const float (&lv)[LV], int64_t n) {
    float total = 0.f;
    bool found = false;
#pragma unroll
    for (int d = 0; d < LV; ++d)
        if ((n >> d) & 1) {
            total = found ? lv[d] + total : lv[d];
            found = true;
        }
    return total;
}

// Finish: the first G workgroups join the tail's row blocks of group g
// (thread t owns outputs t, t + 256, ...: at most five; their block totals
// read sixteen at a time, -0.0 past the last block, each run of sixteen a
// complete tree, the runs joined by a carry stack) and apply SGD to W2, b1,
// b2 and write the loss; the rest update W1 from the slices of x^T.g_d,
// four elements per thread.
template <int NS>
__global__ __launch_bounds__(256) void mlp_finish_kernel(MlpArgs a, int groups) {
    const int O = a.O;
    if ((int)blockIdx.x >= groups) {
        const int64_t n = a.I * a.H, slice = n;
        const int64_t e0 = ((int64_t)(blockIdx.x - groups) * 256 + threadIdx.x) * 4;
        if (e0 >= n) return;
        if (e0 + 4 <= n && a.vec) {
            // NS > 0: the slices read together, then added in slice order
            float4 g;
            if constexpr (NS > 0) {
                float4 v[NS];
#pragma unroll
                for (int s = 0; s < NS; ++s) v[s] = *reinterpret_cast<const float4 *>(a.gw1 + s * slice + e0);
                g = v[0];
#pragma unroll
                for (int s = 1; s < NS; ++s) g.x += v[s].x, g.y += v[s].y, g.z += v[s].z, g.w += v[s].w;
            } else {
                g = *reinterpret_cast<const float4 *>(a.gw1 + e0);
                for (int64_t s = 1; s < a.gw1_slices; ++s) {
                    const float4 v = *reinterpret_cast<const float4 *>(a.gw1 + s * slice + e0);
                    g.x += v.x, g.y += v.y, g.z += v.z, g.w += v.w;
                }
            }
            const float4 w = *reinterpret_cast<const float4 *>(a.w1 + e0);
            float4 o;
            o.x = canon(w.x - canon(a.lr * canon(g.x)));
            o.y = canon(w.y - canon(a.lr * canon(g.y)));
            o.z = canon(w.z - canon(a.lr * canon(g.z)));
            o.w = canon(w.w - canon(a.lr * canon(g.w)));
            *reinterpret_cast<float4 *>(a.w1o + e0) = o;
        } else {
            for (int64_t e = e0; e < n && e < e0 + 4; ++e) {
                float g = a.gw1[e];
                for (int64_t s = 1; s < a.gw1_slices; ++s) g += a.gw1[s * slice + e];
                a.w1o[e] = canon(a.w1[e] - canon(a.lr * canon(g)));
            }
        }
        return;
    }
    const int g = blockIdx.x;
    const bool extra = g == groups - 1;
    const int outs = extra ? 1 : O + 1;
    const int64_t blocks = a.blocks;
    const float *part = a.part + (int64_t)g * kOuts * 64 * blocks;
    const BufRead w2b(a.w2, a.H * O * 4), b1b(a.b1, a.H * 4), b2b(a.b2, O * 4), pb(part, kOuts * 64 * blocks * 4);
    float prm[5];
#pragma unroll
    for (int u = 0; u < 5; ++u) {
        const int e = threadIdx.x + 256 * u, j = e / 64, l = e % 64;
        const int64_t kk = (int64_t)g * 64 + l;
        const bool ok = e < outs * 64 && (extra ? l < O : kk < a.H);
        const float pw = w2b[ok && j < O ? kk * O + j : 0], p1 = b1b[ok ? kk : 0], p2 = b2b[ok && l < O ? l : 0];
        prm[u] = extra ? p2 : (j < O ? pw : p1);
    }
    float lvl[5][kJoinLevels];
#pragma unroll 1
    for (int64_t q0 = 0; q0 < blocks; q0 += 16) {
        float v[5][16];
#pragma unroll
        for (int u = 0; u < 5; ++u) {
            const int e = threadIdx.x + 256 * u;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const bool ok = e < outs * 64 && q0 + i < blocks;
                const float x = pb[ok ? (q0 + i) * kOuts * 64 + e : 0];
                v[u][i] = ok ? x : -0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < 5; ++u) push_leaf<kJoinLevels>(lvl[u], q0 / 16, reg_tree<16>(v[u]));
    }
    const int64_t runs = (blocks + 15) / 16;
#pragma unroll
    for (int u = 0; u < 5; ++u) {
        const int e = threadIdx.x + 256 * u, j = e / 64, l = e % 64;
        if (e >= outs * 64) continue;
        const float total = canon(stack_total<kJoinLevels>(lvl[u], runs));
        if (extra) {
            if (l < O) a.b2o[l] = canon(prm[u] - canon(a.lr * total));
            else if (l == O) *a.loss = canon(quot_f32(total, a.inv_batch));
        } else {
            const int64_t kk = (int64_t)g * 64 + l;
            if (kk >= a.H) continue;
            if (j < O) a.w2o[kk * O + j] = canon(prm[u] - canon(a.lr * total));
            else a.b1o[kk] = canon(prm[u] - canon(a.lr * total));
        }
    }
}

template <int L>
void launch_head(const MlpArgs &a, hipStream_t st) {
    const int64_t blocks = std::min<int64_t>((a.B + 3) / 4, 4 * (int64_t)std::max(device_cus(), 1));
    switch (a.z1_slices) {
        case 1: mlp_head_kernel<L, 1><<<(unsigned)blocks, 256, 0, st>>>(a); break;
        case 2: mlp_head_kernel<L, 2><<<(unsigned)blocks, 256, 0, st>>>(a); break;
        case 3: mlp_head_kernel<L, 3><<<(unsigned)blocks, 256, 0, st>>>(a); break;
        case 4: mlp_head_kernel<L, 4><<<(unsigned)blocks, 256, 0, st>>>(a); break;
        default: mlp_head_kernel<L, 0><<<(unsigned)blocks, 256, 0, st>>>(a); break;
    }
}

// Hidden units per lane in the head: the power of two that covers H with
// 64 lanes.
int64_t run_length(int64_t H) {
    int64_t L = 1;
    while (64 * L < H) L <<= 1;
    return L;
}

MlpArgs make_args(const MlpNarrow &m) {
    MlpArgs a{};
    a.z1 = m.z1, a.w1 = m.w1, a.w2 = m.w2, a.b2 = m.b2, a.oh = m.onehot, a.b1 = m.b1, a.gw1 = m.gw1;
    a.key = m.key;
    a.d = m.d, a.gz2 = m.gz2, a.nl = m.nl, a.gd = m.gd, a.part = m.part;
    a.w1o = m.w1_out, a.w2o = m.w2_out, a.b1o = m.b1_out, a.b2o = m.b2_out, a.loss = m.loss;
    a.B = m.B, a.H = m.H, a.I = m.I, a.O = (int)m.O;
    a.z1_slices = m.z1_slices, a.gw1_slices = m.gw1_slices;
    a.blocks = (m.B + 63) / 64;
    const auto al16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    a.vec = m.H % 4 == 0 && al16(m.z1) && al16(m.d) && al16(m.gd) && al16(m.w1) && al16(m.w1_out) &&
            (!m.gw1 || al16(m.gw1));
    a.rate = m.rate, a.lr = m.lr;
    // -(1 / B): finite and not NaN for B >= 1
    a.g_pr = -(1.0f / (float)m.B);
    a.inv_keep = 1.0 / (double)(1.0f - m.rate);
    a.cut = dropout_cut((double)m.rate, CHELIS_DTYPE_F32);
    a.inv_batch = 1.0 / (double)(float)m.B;
    return a;
}

}  // namespace

bool mlp_narrow_fits(int64_t B, int64_t I, int64_t H, int64_t O) {
    // buffer reads take 32-bit byte offsets; the join's carry stack holds
    // 2^kJoinLevels - 1 runs of sixteen row blocks
    return B >= 1 && H >= 1 && H <= 64 * kMaxRun && O >= 1 && O <= kMaxClasses && I >= 1 &&
           B * H * 4 < (int64_t(1) << 31) && I * H * 4 < (int64_t(1) << 31) &&
           (B + 63) / 64 <= 16 * ((int64_t(1) << kJoinLevels) - 1) && (B + 63) / 64 <= 65535;
}

size_t mlp_part_bytes(int64_t B, int64_t H) {
    return (size_t)((H + 63) / 64 + 1) * kOuts * 64 * ((B + 63) / 64) * sizeof(float);
}

int32_t mlp_head_tail(const MlpNarrow &m, hipStream_t st) {
    if (!mlp_narrow_fits(m.B, m.I, m.H, m.O) || m.z1_slices < 1)
        return set_error(CHELIS_HIP_EUNSUPPORTED, "mlp_train_step: narrow part shape");
    const MlpArgs a = make_args(m);
    const int64_t L = run_length(m.H);
    if (L <= 1) launch_head<1>(a, st);
    else if (L <= 2) launch_head<2>(a, st);
    else if (L <= 4) launch_head<4>(a, st);
    else if (L <= 8) launch_head<8>(a, st);
    else launch_head<16>(a, st);
    CHELIS_LAUNCH_CHECK();
    const int64_t groups = (m.H + 63) / 64 + 1;
    mlp_tail_kernel<<<dim3((unsigned)groups, (unsigned)a.blocks), 256, 0, st>>>(a);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

int32_t mlp_finish(const MlpNarrow &m, hipStream_t st) {
    if (!mlp_narrow_fits(m.B, m.I, m.H, m.O) || m.gw1_slices < 1)
        return set_error(CHELIS_HIP_EUNSUPPORTED, "mlp_train_step: narrow part shape");
    const MlpArgs a = make_args(m);
    const int groups = (int)((m.H + 63) / 64 + 1);
    const int64_t w1_blocks = (m.I * m.H + 1023) / 1024;
    const unsigned grid = (unsigned)(groups + w1_blocks);
    switch (m.gw1_slices) {
        case 1: mlp_finish_kernel<1><<<grid, 256, 0, st>>>(a, groups); break;
        case 2: mlp_finish_kernel<2><<<grid, 256, 0, st>>>(a, groups); break;
        case 3: mlp_finish_kernel<3><<<grid, 256, 0, st>>>(a, groups); break;
        case 4: mlp_finish_kernel<4><<<grid, 256, 0, st>>>(a, groups); break;
        case 5: mlp_finish_kernel<5><<<grid, 256, 0, st>>>(a, groups); break;
        case 6: mlp_finish_kernel<6><<<grid, 256, 0, st>>>(a, groups); break;
        default: mlp_finish_kernel<0><<<grid, 256, 0, st>>>(a, groups); break;
    }
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

}  // namespace chelis
