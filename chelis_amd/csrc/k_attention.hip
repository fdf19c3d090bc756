// Causal self-attention in one launch: for every (batch, head),
//   O = softmax(where(key <= row, (Q K^T) * scale, -inf)) V
// with binary32 operands and a head dimension of 64 - the lowering of the
// reference's attention (scores matmul, causal where, softmax, P.V) without
// its [S, S] score matrix ever reaching memory.
//
// A workgroup owns 64 query rows of one (batch, head); each of its four
// waves owns 16 of them and walks the key tiles 0..(its row tile) in order,
// keeping a running maximum and sum per row (the online softmax): for a key
// tile the wave forms S^T = K Q^T on the matrix cores, scales and masks it,
// exponentiates against the new running maximum, rescales its output
// accumulator, and adds P V. K and V tiles of 64 keys are staged through
// LDS, shared by the four waves; the next tile's loads are in flight while
// the current one is consumed.
//
// Operand layouts (v_mfma_f32_16x16x4_f32: A[i][k] from lane k*16 + i,
// B[k][j] from lane k*16 + j, C[4k' + r][j] in lane k'*16 + j, item r):
//   S^T block kb (keys 16kb.., rows of the wave): A = K[key][d], B = Q[row][d]
//     with, at MFMA step u, lane group q supplying d = 16q + u - so a lane
//     holds 16 consecutive d of its query row for the whole walk;
//   lane (q, j) then holds S^T[key 16kb + 4q + r][row j], r = 0..3, and its
//     row j's statistics combine across the lane groups (lanes j, j + 16,
//     j + 32, j + 48);
//   O^T block bd (d = 16bd..): A = V^T[d][key], B = P^T[key][row] at step
//     (kb, t) with lane group q supplying key 16kb + 4q + t: B is item t of
//     the S^T accumulator the lane already holds, and A a 4-key run of the
//     transposed V tile in LDS;
//   lane (q, j) ends with O^T[d 16bd + 4q + r][row j]: four consecutive d of
//     one output row, stored as one 16-byte write.
// Rounding differs from the unfused graph (the sums run in another order
// and the exponentials against running maxima); the result stays within
// the binary32 tolerance of the canonical-tree graph.
#include "hip_common.h"

namespace chelis {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 64;       // head dimension
constexpr int kT = 64;       // query rows per workgroup, keys per tile
constexpr int kPitch = 68;   // LDS row pitch in floats
constexpr int kThreads = 256;
constexpr int kMaxOrder = 32;  // q-tiles the round table covers

struct AttnArgs {
    const float *q, *k, *v;
    float *o;
    int64_t heads, S, qtiles, pairs;
    // element strides of [batch][head][seq] (the last axis is contiguous)
    int64_t q0, q1, qs, k0, k1, ks, v0, v1, vs, o0, o1, os;
    float scale;
    // round r (workgroups r * pairs ..) takes q-tile order[r] when
    // use_order, else the heaviest-first qtiles - 1 - r
    int32_t use_order;
    int8_t order[kMaxOrder];
};

__device__ inline f32x4 mma(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// Largest / sum over the four lane groups of a row (lanes j, j+16, j+32, j+48).
__device__ inline float row_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 16, 64));
    return fmaxf(x, __shfl_xor(x, 32, 64));
}
__device__ inline float row_sum(float x) {
    x += __shfl_xor(x, 16, 64);
    return x + __shfl_xor(x, 32, 64);
}

__global__ __launch_bounds__(kThreads, 2) void attention_causal_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) float Ks[kT][kPitch];  // [key][d]
    __shared__ __attribute__((aligned(16))) float Vt[kD][kPitch];  // [d][key]

    const int64_t round = (int64_t)blockIdx.x / a.pairs;
    const int64_t qt = a.use_order ? a.order[round] : a.qtiles - 1 - round;
    const int64_t z = (int64_t)blockIdx.x % a.pairs;
    const int64_t zb = z / a.heads, zh = z % a.heads;
    const float *Q = a.q + zb * a.q0 + zh * a.q1;
    const float *K = a.k + zb * a.k0 + zh * a.k1;
    const float *V = a.v + zb * a.v0 + zh * a.v1;
    float *O = a.o + zb * a.o0 + zh * a.o1;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, q = lane >> 4;
    const int64_t row = qt * kT + 16 * wave + j;  // this lane's query row

    // the 16 consecutive d of this lane's row from 16q
    float qf[16];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const float4 x = *reinterpret_cast<const float4 *>(Q + row * a.qs + 16 * q + 4 * h);
        qf[4 * h] = x.x;
        qf[4 * h + 1] = x.y;
        qf[4 * h + 2] = x.z;
        qf[4 * h + 3] = x.w;
    }

    // staging: thread t moves 4-float runs e = 4t + 1024i (i = 0..3) of the
    // 64 x 64 K and V tiles: key e / 64 = t / 16 + 16i, d e % 64 = 4 (t % 16).
    // The staging registers are written and read only in straight-line code
    // (through a lambda capturing them, the compiler kept the K half in
    // scratch memory and waited for the next tile's loads right after
    // issuing them, to store them there).
    const int skey = tid >> 4, sd = (tid & 15) * 4;
    const float *kbase = K + skey * a.ks + sd, *vbase = V + skey * a.vs + sd;
    const int64_t kstep = 16 * a.ks, vstep = 16 * a.vs;
    f32x4 kr0, kr1, kr2, kr3, vr0, vr1, vr2, vr3;
#define CHELIS_ATT_LOAD(kt)                                                                      \
    do {                                                                                         \
        const float *kp = kbase + (kt) * kT * a.ks, *vp = vbase + (kt) * kT * a.vs;              \
        kr0 = *reinterpret_cast<const f32x4 *>(kp);                                              \
        kr1 = *reinterpret_cast<const f32x4 *>(kp + kstep);                                      \
        kr2 = *reinterpret_cast<const f32x4 *>(kp + 2 * kstep);                                  \
        kr3 = *reinterpret_cast<const f32x4 *>(kp + 3 * kstep);                                  \
        vr0 = *reinterpret_cast<const f32x4 *>(vp);                                              \
        vr1 = *reinterpret_cast<const f32x4 *>(vp + vstep);                                      \
        vr2 = *reinterpret_cast<const f32x4 *>(vp + 2 * vstep);                                  \
        vr3 = *reinterpret_cast<const f32x4 *>(vp + 3 * vstep);                                  \
    } while (0)
#define CHELIS_ATT_STORE1(i, kr, vr)                                                             \
    do {                                                                                         \
        *reinterpret_cast<f32x4 *>(&Ks[skey + 16 * (i)][sd]) = kr;                               \
        Vt[sd][skey + 16 * (i)] = vr[0];                                                         \
        Vt[sd + 1][skey + 16 * (i)] = vr[1];                                                     \
        Vt[sd + 2][skey + 16 * (i)] = vr[2];                                                     \
        Vt[sd + 3][skey + 16 * (i)] = vr[3];                                                     \
    } while (0)
#define CHELIS_ATT_STORE()                                                                       \
    do {                                                                                         \
        CHELIS_ATT_STORE1(0, kr0, vr0);                                                          \
        CHELIS_ATT_STORE1(1, kr1, vr1);                                                          \
        CHELIS_ATT_STORE1(2, kr2, vr2);                                                          \
        CHELIS_ATT_STORE1(3, kr3, vr3);                                                          \
    } while (0)

    f32x4 acc_o[4];
#pragma unroll
    for (int bd = 0; bd < 4; ++bd) acc_o[bd] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    CHELIS_ATT_LOAD(0);
    CHELIS_ATT_STORE();
    __syncthreads();
    // Every load issued so far (the query row included) completes here, so
    // the loop header has nothing older to wait for: otherwise the wait the
    // compiler places there for the query row (its first use) also waits
    // for the next tile's loads on every iteration, and the prefetch never
    // overlaps the tile's arithmetic.
    __builtin_amdgcn_s_waitcnt(0);
    for (int64_t kt = 0; kt <= qt; ++kt) {
        if (kt < qt) CHELIS_ATT_LOAD(kt + 1);
        // On the diagonal tile, key block kb > wave lies wholly above this
        // wave's rows: its scores are masked to -inf below and its P.V terms
        // are skipped, as the tiles above the diagonal are.
        const bool diag = kt == qt;
        // S^T = K Q^T for the tile's four key blocks
        f32x4 s[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            s[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (diag && kb > wave) continue;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const float4 kf = *reinterpret_cast<const float4 *>(&Ks[16 * kb + j][16 * q + 4 * h]);
                s[kb] = mma(kf.x, qf[4 * h], s[kb]);
                s[kb] = mma(kf.y, qf[4 * h + 1], s[kb]);
                s[kb] = mma(kf.z, qf[4 * h + 2], s[kb]);
                s[kb] = mma(kf.w, qf[4 * h + 3], s[kb]);
            }
        }
        // scale, causal mask (the diagonal tile only), running statistics
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float x = s[kb][r] * a.scale;
                if (kt == qt && 16 * kb + 4 * q + r > 16 * wave + j) x = -INFINITY;
                s[kb][r] = x;
                mx = fmaxf(mx, x);
            }
        const float m_new = fmaxf(m_run, row_max(mx));  // key 0 <= row: finite
        const float alpha = expf(m_run - m_new);
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = expf(s[kb][r] - m_new);
                s[kb][r] = p;
                sum += p;
            }
        l_run = l_run * alpha + row_sum(sum);
        m_run = m_new;
#pragma unroll
        for (int bd = 0; bd < 4; ++bd) acc_o[bd] *= alpha;
        // O^T += V^T P^T
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            if (diag && kb > wave) continue;
#pragma unroll
            for (int bd = 0; bd < 4; ++bd) {
                const float4 vf = *reinterpret_cast<const float4 *>(&Vt[16 * bd + j][16 * kb + 4 * q]);
                acc_o[bd] = mma(vf.x, s[kb][0], acc_o[bd]);
                acc_o[bd] = mma(vf.y, s[kb][1], acc_o[bd]);
                acc_o[bd] = mma(vf.z, s[kb][2], acc_o[bd]);
                acc_o[bd] = mma(vf.w, s[kb][3], acc_o[bd]);
            }
        }
        if (kt < qt) {
            __syncthreads();  // every wave is done with this tile
            CHELIS_ATT_STORE();
            __syncthreads();
        }
    }
#undef CHELIS_ATT_STORE
#undef CHELIS_ATT_STORE1
#undef CHELIS_ATT_LOAD
    const float inv = 1.f / l_run;
#pragma unroll
    for (int bd = 0; bd < 4; ++bd) {
        const float4 y = {acc_o[bd][0] * inv, acc_o[bd][1] * inv, acc_o[bd][2] * inv, acc_o[bd][3] * inv};
        *reinterpret_cast<float4 *>(O + row * a.os + 16 * bd + 4 * q) = y;
    }
}

bool view4(const chelis_gpu_tensor *t, int64_t B, int64_t H, int64_t S) {
    return t && t->rank == 4 && t->shape && t->strides && t->dtype == CHELIS_DTYPE_F32 && t->shape[0] == B && t->shape[1] == H &&
           t->shape[2] == S && t->shape[3] == kD && t->strides[3] == 1 &&
           (reinterpret_cast<uintptr_t>(t->data) % 16) == 0 && t->strides[0] % 4 == 0 && t->strides[1] % 4 == 0 &&
           t->strides[2] % 4 == 0;
}

// The q-tile of each round of `pairs` workgroups. Workgroup b runs on CU
// b mod C when the whole grid is resident (the dispatcher deals workgroups
// round-robin over the XCDs and their CUs; four fit per CU), so when C is a
// multiple of pairs the rounds fall into g = C / pairs groups that share
// their CUs (round r in group r mod g). A q-tile t costs t + 1 key tiles:
// the tiles go heaviest first to the group with the least work so far, and
// each group takes its tiles heaviest first. B8 H16 S512 on 256 CUs: 18 key
// tiles on every CU, against 20 and 16 for heaviest-first rounds. Other
// geometries keep heaviest-first rounds.
void plan_rounds(AttnArgs &a, int64_t blocks, int cus) {
    a.use_order = 0;
    if (a.qtiles > kMaxOrder || a.pairs >= cus || cus % a.pairs != 0 || blocks > 4 * (int64_t)cus) return;
    const int g = (int)(cus / a.pairs);
    int64_t load[kMaxOrder] = {};
    int tiles[kMaxOrder][kMaxOrder], count[kMaxOrder] = {};
    for (int t = (int)a.qtiles - 1; t >= 0; --t) {
        int best = 0;
        for (int k = 1; k < g && k < kMaxOrder; ++k)
            if (load[k] < load[best]) best = k;
        load[best] += t + 1;
        tiles[best][count[best]++] = t;
    }
    int used[kMaxOrder] = {};
    for (int64_t r = 0; r < a.qtiles; ++r) {
        const int k = (int)(r % g);
        if (k >= kMaxOrder || used[k] >= count[k]) return;  // a group short of tiles: keep heaviest-first
        a.order[r] = (int8_t)tiles[k][used[k]++];
    }
    a.use_order = 1;
}

}  // namespace

bool attention_causal_fits(const chelis_gpu_tensor *q, const chelis_gpu_tensor *k, const chelis_gpu_tensor *v,
                           const chelis_gpu_tensor *o) {
    if (!q || q->rank != 4 || !q->shape) return false;
    const int64_t B = q->shape[0], H = q->shape[1], S = q->shape[2];
    return S > 0 && S % kT == 0 && B * H > 0 && view4(q, B, H, S) && view4(k, B, H, S) && view4(v, B, H, S) &&
           view4(o, B, H, S);
}

int32_t attention_causal(const chelis_gpu_tensor *q, const chelis_gpu_tensor *k, const chelis_gpu_tensor *v,
                         double scale, const chelis_gpu_tensor *o) {
    for (const chelis_gpu_tensor *t : {q, k, v, o})
        if (int32_t s = check_tensor(t, "attention")) return s;
    if (!attention_causal_fits(q, k, v, o))
        return set_error(CHELIS_HIP_EUNSUPPORTED,
                         "attention: f32 [batch, heads, seq, 64] views with seq a multiple of 64, the last axis "
                         "contiguous and 16-byte aligned rows");
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    AttnArgs a{};
    a.q = static_cast<const float *>(q->data);
    a.k = static_cast<const float *>(k->data);
    a.v = static_cast<const float *>(v->data);
    a.o = static_cast<float *>(o->data);
    a.heads = q->shape[1];
    a.S = q->shape[2];
    a.qtiles = a.S / kT;
    a.pairs = q->shape[0] * q->shape[1];
    a.q0 = q->strides[0], a.q1 = q->strides[1], a.qs = q->strides[2];
    a.k0 = k->strides[0], a.k1 = k->strides[1], a.ks = k->strides[2];
    a.v0 = v->strides[0], a.v1 = v->strides[1], a.vs = v->strides[2];
    a.o0 = o->strides[0], a.o1 = o->strides[1], a.os = o->strides[2];
    a.scale = (float)scale;
    const int64_t blocks = a.pairs * a.qtiles;
    if (!grid_fits(blocks, kThreads)) return set_error(CHELIS_HIP_EUNSUPPORTED, "attention: grid too large");
    plan_rounds(a, blocks, device_cus());
    attention_causal_kernel<<<(unsigned)blocks, kThreads, 0, st>>>(a);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

}  // namespace chelis

// No counterpart in the reference's C ABI: the fused form of its attention
// lowering (scores matmul, causal where, softmax, P.V), for callers and
// plans that hold the three as one region.
extern "C" int32_t chelis_hip_causal_attention(const chelis_gpu_tensor *q, const chelis_gpu_tensor *k,
                                               const chelis_gpu_tensor *v, double scale,
                                               const chelis_gpu_tensor *o) {
    return chelis::attention_causal(q, k, v, scale, o);
}
