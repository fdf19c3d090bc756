// Elementwise regions on gfx950: the FusedElem chain interpreter, GELU,
// ReLU and its adjoint, keyed dropout / replay / uniform_like.
//
// Bandwidth design: the unary maps (GELU, ReLU, dropout, uniform) move
// contiguous operands in 16-byte vectors (one float4 / double2 per lane per
// access, 1 KiB per wave instruction). The chain interpreter reads one
// element per lane (coalesced) and keeps its code small; shapes are
// collapsed on the host first, so the common case is a flat map (every
// operand contiguous with the output or a broadcast scalar) with no index
// arithmetic, and only genuinely strided views (row/column broadcast,
// permuted axes) pay for coordinates. A broadcast operand (stride 0) is
// re-read through L2/MALL, not materialized.
#include <type_traits>

#include "chain.h"
#include "narrow.h"
#include "strided.h"

namespace chelis {
namespace {

// Every kernel in this file runs 256 threads per workgroup (the launches
// below pass that count). Index arithmetic uses the constant: blockDim.x is
// read from the dispatch packet with a vector memory load at the start of
// each wave, a full memory round trip before a one-vector-per-thread wave
// can form its first address.
constexpr int kMapThreads = 256;

struct Operand {
    const void *p;
    int64_t st[kMaxRank];
};
struct Operands {
    int32_t n;
    Operand o[CHELIS_FUSED_MAX_INPUTS];
};

// The chain interpreter (run_chain, chain.h): one thread per element, the
// element's inputs and step results in a row of LDS slots. A launch is
// mostly a handful of small tensors, so the kernel is kept small: its code
// is fetched by every CU once per launch.

// Strided operands (any of the up-to-4 collapsed axes, broadcast by stride
// 0): the element's coordinates from its flat index, then one offset per
// operand.
template <typename T>
__global__ __launch_bounds__(256) void fused_chain_kernel(ChainDev ch, Operands ops, Shape sh, T *__restrict__ out,
                                                          int64_t count) {
    __shared__ T slots[256 * kSlotStride];
    T *slot = slots + threadIdx.x * kSlotStride;
    const int64_t stride = (int64_t)gridDim.x * kMapThreads;
    for (int64_t idx = (int64_t)blockIdx.x * kMapThreads + threadIdx.x; idx < count; idx += stride) {
        int64_t coord[kMaxRank];
        int64_t rem = idx;
#pragma unroll
        for (int a = kMaxRank - 1; a >= 0; --a) {
            if (a < sh.rank) {
                coord[a] = rem % sh.ext[a];
                rem /= sh.ext[a];
            } else {
                coord[a] = 0;
            }
        }
        T in[CHELIS_FUSED_MAX_INPUTS];
#pragma unroll
        for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k) {
            if (k < ops.n) {
                int64_t off = 0;
#pragma unroll
                for (int a = 0; a < kMaxRank; ++a) off += coord[a] * ops.o[k].st[a];
                in[k] = static_cast<const T *>(ops.o[k].p)[off];
            }
        }
#pragma unroll
        for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k)
            if (k < ops.n) slot[k] = in[k];
        out[idx] = run_chain<T>(ch, slot);
    }
}

// ---------------------------------------------------------------- narrow floats
// bf16 / f16 chains of sub, max_elem and min_elem, the steps the reference
// admits for 16-bit storage (crates/chelis-backend-hip/src/emit.rs:2292-2319,
// kernels.rs:2274-2310): each step reads 16-bit operands, works at binary32
// and stores 16 bits (narrow.h). Slots hold stored bits; the operands are
// gathered as in fused_chain_kernel.
template <Narrow K>
__device__ inline uint16_t run_narrow_chain(const ChainDev &ch, uint16_t *slot) {
    uint16_t v = 0;
#pragma unroll 1
    for (int s = 0; s < ch.n_steps; ++s) {
        const int a0 = ch.a0[s], a1 = ch.a1[s];
        const uint16_t x = slot[a0 >= 0 ? a0 : CHELIS_FUSED_MAX_INPUTS - a0 - 1];
        const uint16_t y = slot[a1 >= 0 ? a1 : CHELIS_FUSED_MAX_INPUTS - a1 - 1];
        const uint8_t op = ch.op[s];
        v = op == CHELIS_FUSED_SUB ? narrow_sub<K>(x, y)
                                   : (op == CHELIS_FUSED_MAX_ELEM ? narrow_max<K>(x, y) : narrow_min<K>(x, y));
        slot[CHELIS_FUSED_MAX_INPUTS + s] = v;
    }
    return v;
}

template <Narrow K>
__global__ __launch_bounds__(256) void narrow_chain_kernel(ChainDev ch, Operands ops, Shape sh,
                                                           uint16_t *__restrict__ out, int64_t count) {
    __shared__ uint16_t slots[256 * kSlotStride];
    uint16_t *slot = slots + threadIdx.x * kSlotStride;
    const int64_t stride = (int64_t)gridDim.x * kMapThreads;
    for (int64_t idx = (int64_t)blockIdx.x * kMapThreads + threadIdx.x; idx < count; idx += stride) {
        int64_t coord[kMaxRank];
        int64_t rem = idx;
#pragma unroll
        for (int a = kMaxRank - 1; a >= 0; --a) {
            if (a < sh.rank) {
                coord[a] = rem % sh.ext[a];
                rem /= sh.ext[a];
            } else {
                coord[a] = 0;
            }
        }
        uint16_t in[CHELIS_FUSED_MAX_INPUTS];
#pragma unroll
        for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k) {
            if (k < ops.n) {
                int64_t off = 0;
#pragma unroll
                for (int a = 0; a < kMaxRank; ++a) off += coord[a] * ops.o[k].st[a];
                in[k] = static_cast<const uint16_t *>(ops.o[k].p)[off];
            }
        }
#pragma unroll
        for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k)
            if (k < ops.n) slot[k] = in[k];
        out[idx] = run_narrow_chain<K>(ch, slot);
    }
}

// bf16 / f16 relu (ADJ = false) and its adjoint on contiguous operands,
// eight 16-bit values per 16-byte access (kernels.rs:1196-1260).
template <Narrow K, bool ADJ>
__global__ __launch_bounds__(256) void narrow_relu_kernel(const uint16_t *__restrict__ x,
                                                          const uint16_t *__restrict__ g, uint16_t *__restrict__ y,
                                                          int64_t n) {
    const int64_t nv = n / 8;
    const int64_t stride = (int64_t)gridDim.x * kMapThreads;
    for (int64_t v = (int64_t)blockIdx.x * kMapThreads + threadIdx.x; v < nv; v += stride) {
        uint4 xv = reinterpret_cast<const uint4 *>(x)[v], gv{}, yv;
        if constexpr (ADJ) gv = reinterpret_cast<const uint4 *>(g)[v];
        const uint16_t *xe = reinterpret_cast<const uint16_t *>(&xv);
        const uint16_t *ge = reinterpret_cast<const uint16_t *>(&gv);
        uint16_t *ye = reinterpret_cast<uint16_t *>(&yv);
#pragma unroll
        for (int i = 0; i < 8; ++i) ye[i] = ADJ ? narrow_relu_adjoint<K>(xe[i], ge[i]) : narrow_relu<K>(xe[i]);
        reinterpret_cast<uint4 *>(y)[v] = yv;
    }
    const int64_t t = nv * 8 + (int64_t)blockIdx.x * kMapThreads + threadIdx.x;
    if (t < n) y[t] = ADJ ? narrow_relu_adjoint<K>(x[t], g[t]) : narrow_relu<K>(x[t]);
}

// ---------------------------------------------------------------- flat maps
// Every operand either runs with the output (stride 1) or is one element
// broadcast to all (stride 0): no index arithmetic. One launch serves up to
// kMaxGroups independent (inputs, output) groups under the same chain (a
// program's parameter updates); block ranges select the group.
constexpr int kMaxGroups = 4;
struct FlatGroup {
    const void *in[CHELIS_FUSED_MAX_INPUTS];
    uint32_t bcast;  // bit k: input k is a single element broadcast to all
    void *out;
    int64_t count;
    int64_t first_block;  // the group's first block in the grid
};
struct FlatGroups {
    int32_t n, n_in;
    FlatGroup g[kMaxGroups];
};

template <typename T>
__global__ __launch_bounds__(256) void fused_flat_kernel(ChainDev ch, FlatGroups fg) {
    __shared__ T slots[256 * kSlotStride];
    int gi = 0;
#pragma unroll
    for (int k = 1; k < kMaxGroups; ++k)
        if (k < fg.n && (int64_t)blockIdx.x >= fg.g[k].first_block) gi = k;
    const FlatGroup &G = fg.g[gi];
    const int64_t i = ((int64_t)blockIdx.x - G.first_block) * 256 + threadIdx.x;
    if (i >= G.count) return;
    T *slot = slots + threadIdx.x * kSlotStride;
    // every load issued before the first slot store: one memory latency
    T in[CHELIS_FUSED_MAX_INPUTS];
#pragma unroll
    for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k)
        if (k < fg.n_in) in[k] = static_cast<const T *>(G.in[k])[((G.bcast >> k) & 1u) ? 0 : i];
#pragma unroll
    for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k)
        if (k < fg.n_in) slot[k] = in[k];
    static_cast<T *>(G.out)[i] = run_chain<T>(ch, slot);
}

// Flat maps over 16-byte vectors: each thread carries V = 16/sizeof(T)
// consecutive elements, so a wave has V times the bytes of the scalar form
// in flight, and each step's operation is chosen once for all V. The slots
// are slot-major in dynamic LDS ([n_in + n_steps][256] vectors: adjacent
// lanes read adjacent 16-byte words) and sized to the chain. Every
// non-broadcast input and the output start 16-byte aligned; a group's last
// partial vector is read and written element by element.
template <typename T>
__global__ __launch_bounds__(256) void fused_flat_vec_kernel(ChainDev ch, FlatGroups fg) {
    constexpr int V = 16 / sizeof(T);
    using Q = typename Vec16F<T>::type;
    extern __shared__ __align__(16) unsigned char flat_lds[];
    Q *slots = reinterpret_cast<Q *>(flat_lds);
    int gi = 0;
#pragma unroll
    for (int k = 1; k < kMaxGroups; ++k)
        if (k < fg.n && (int64_t)blockIdx.x >= fg.g[k].first_block) gi = k;
    const FlatGroup &G = fg.g[gi];
    const int64_t i0 = (((int64_t)blockIdx.x - G.first_block) * 256 + threadIdx.x) * V;
    if (i0 >= G.count) return;
    const bool full = i0 + V <= G.count;
    const int n_in = fg.n_in;
    // every load issued before the first slot store: one memory latency
    Q in[CHELIS_FUSED_MAX_INPUTS];
#pragma unroll
    for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k) {
        if (k < n_in) {
            const T *p = static_cast<const T *>(G.in[k]);
            T *e = reinterpret_cast<T *>(&in[k]);
            if ((G.bcast >> k) & 1u) {
                const T b = p[0];
#pragma unroll
                for (int j = 0; j < V; ++j) e[j] = b;
            } else if (full) {
                in[k] = load_nt16(p + i0);
            } else {
#pragma unroll
                for (int j = 0; j < V; ++j) e[j] = i0 + j < G.count ? p[i0 + j] : T(0);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < CHELIS_FUSED_MAX_INPUTS; ++k)
        if (k < n_in) slots[k * 256 + threadIdx.x] = in[k];
    T r[V];
    run_chain_vec<T, V>(ch, slots, n_in, threadIdx.x, r);
    T *out = static_cast<T *>(G.out);
    if (full) {
        Q rq;
#pragma unroll
        for (int j = 0; j < V; ++j) reinterpret_cast<T *>(&rq)[j] = r[j];
        store_nt16(out + i0, rq);
    } else {
#pragma unroll
        for (int j = 0; j < V; ++j)
            if (i0 + j < G.count) out[i0 + j] = r[j];
    }
}

// ---------------------------------------------------------------- unary maps
// Contiguous n-element maps with 16-byte vectors; the scalar tail is the
// last n % V elements.
template <typename T>
struct Vec16;
template <> struct Vec16<float> { using type = float4; static constexpr int V = 4; };
template <> struct Vec16<double> { using type = double2; static constexpr int V = 2; };

// GeluFast: binary32 GELU in the default mode (gelu_fast_f32, the graph
// for the inputs it does not serve); binary64 GELU is the graph in both.
enum class Unary : int { Gelu, Relu, ReluAdjoint, Dropout, Uniform, GeluFast };

struct UnaryArgs {
    uint64_t key;
    double p0, p1;            // dropout: rate; uniform: low, high
    const uint64_t *key_dev;  // when set, the key is read from device memory (a KEY tensor)
    double inv_keep;          // dropout, binary32: 1 / (double)(1 - (float)rate), set by the kernel
    uint64_t cut;             // dropout: an element whose word >> 11 is below it is dropped (dropout_cut)
};

template <typename T, Unary OP, class Tabs = ErfcTablesConst>
__device__ inline T unary_one(T x, T g, int64_t i, const UnaryArgs &u, const Tabs &tb = Tabs{}) {
    if constexpr (OP == Unary::Gelu) {
        return gelu_one_t<T>(x, tb);
    } else if constexpr (OP == Unary::GeluFast) {
        if constexpr (sizeof(T) == 4) {
            bool slow;
            T r = gelu_fast_f32(x, slow);
            if (slow) r = gelu_one_t<T>(x, ErfcTablesConst{});
            return r;
        } else {
            return gelu_one_t<T>(x, tb);
        }
    } else if constexpr (OP == Unary::Relu) {
        return x < T(0) ? T(0) : x;
    } else if constexpr (OP == Unary::ReluAdjoint) {
        return T(0) < x ? g : T(0);
    } else if constexpr (OP == Unary::Dropout) {
        // [05-OP-37]: the unit at the dtype's width against the rate, as the
        // integer comparison it is equivalent to (dropout_cut); a kept
        // element is x / (1 - rate) (binary32: through the binary64
        // reciprocal of the divisor, quot_f32, which rounds to the IEEE
        // quotient).
        // (word >> 11) < cut, as word < cut * 2^11 (no shift per element;
        // cut = 2^53, which drops every element, does not fit the product)
        const bool drop = (u.cut >> 53) != 0 || random_word(u.key, (uint64_t)i) < (u.cut << 11);
        if constexpr (sizeof(T) == 4) return drop ? T(0) : canon(quot_f32(x, u.inv_keep));
        else return drop ? T(0) : canon(x / (T(1) - (T)u.p0));
    } else {
        // [05-OP-8]: one fma(high - low, u, low) at the dtype.
        const T low = (T)u.p0, high = (T)u.p1;
        return canon(fma(high - low, (T)random_unit(u.key, (uint64_t)i), low));
    }
}

// 16-byte vectors as clang vector types: the nontemporal load and store
// builtins take those (not HIP's float4 / double2 structs).
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef double f64x2_t __attribute__((ext_vector_type(2)));
template <typename T> struct NtVec;
template <> struct NtVec<float> { using type = f32x4_t; };
template <> struct NtVec<double> { using type = f64x2_t; };

// One 16-byte vector per thread (grid-stride past 2^16 workgroups), loads
// and stores nontemporal: every element is read once and written once. The
// binary32 default-mode GELU evaluates a vector's four elements side by
// side and branches once to the graph for those gelu_fast_f32 does not
// serve. ([16384,4096] f32 at settled clocks: GELU 83 us here against
// 99-103 us as a resident grid streaming several vectors per thread, whose
// copy form alone took 85-124 us; a plain copy in this form 82.5 us with
// nontemporal accesses, 88.4 without.)
template <typename T, Unary OP>
__global__ __launch_bounds__(256) void unary_kernel(const T *__restrict__ x, const T *__restrict__ g,
                                                    T *__restrict__ y, int64_t n, UnaryArgs u) {
    if constexpr (OP == Unary::Dropout || OP == Unary::Uniform)
        if (u.key_dev) u.key = *u.key_dev;
    if constexpr (OP == Unary::Dropout) u.inv_keep = 1.0 / (double)(T(1) - (T)u.p0);
    // binary32 GELU reads its erfc and exp tables from LDS
    auto run = [&](const auto &tb) {
        using NV = typename NtVec<T>::type;
        constexpr int V = Vec16<T>::V;
        const int64_t nv = n / V;
        const int64_t stride = (int64_t)gridDim.x * kMapThreads;
        for (int64_t v = (int64_t)blockIdx.x * kMapThreads + threadIdx.x; v < nv; v += stride) {
            NV xv{}, gv{}, yv;
            if constexpr (OP != Unary::Uniform) xv = __builtin_nontemporal_load(reinterpret_cast<const NV *>(x) + v);
            if constexpr (OP == Unary::ReluAdjoint) gv = __builtin_nontemporal_load(reinterpret_cast<const NV *>(g) + v);
            if constexpr (OP == Unary::GeluFast && sizeof(T) == 4) {
                bool sl[V], any = false;
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    yv[i] = gelu_fast_f32(xv[i], sl[i]);
                    any = any || sl[i];
                }
                if (any)
#pragma unroll
                    for (int i = 0; i < V; ++i)
                        if (sl[i]) yv[i] = gelu_one_t<T>(xv[i], ErfcTablesConst{});
            } else {
#pragma unroll
                for (int i = 0; i < V; ++i) yv[i] = unary_one<T, OP>(xv[i], gv[i], v * V + i, u, tb);
            }
            __builtin_nontemporal_store(yv, reinterpret_cast<NV *>(y) + v);
        }
        // tail
        const int64_t t = nv * V + (int64_t)blockIdx.x * kMapThreads + threadIdx.x;
        if (t < n) {
            const T xe = (OP != Unary::Uniform) ? x[t] : T(0);
            const T ge = (OP == Unary::ReluAdjoint) ? g[t] : T(0);
            y[t] = unary_one<T, OP>(xe, ge, t, u, tb);
        }
    };
    if constexpr (OP == Unary::Gelu && sizeof(T) == 4) {
        __shared__ ErfcLdsStore gtab;
        gtab.fill<kMapThreads>();
        __syncthreads();
        run(gtab.tabs());
    } else {
        run(ErfcTablesConst{});
    }
}

// The exact-mode GELU, keyed dropout and uniform_like (VALU-heavy): a
// resident grid whose threads walk the vectors with a stride, the next
// vectors' loads issued before the current ones are evaluated, so each
// wave's memory traffic overlaps its own arithmetic. Loads and stores are
// nontemporal.
// vectors per buffer: each thread evaluates one buffer of kStreamBatch
// vectors while the other buffer's loads are in flight (a ping-pong, so no
// register moves); fewer for the register-heavy exact GELU
// (dropout, [16384,4096] f32 at settled clocks: 1 vector 106-110 us, 2
// vectors 107-110, 3 vectors 111-113, 4 vectors 109-111, 6 vectors 119)
template <Unary OP> constexpr int kStreamBatch = OP == Unary::Gelu ? 1 : OP == Unary::Dropout ? 2 : 3;

// the maps that take the resident streaming grid; the others run one vector
// per thread (unary_kernel)
template <Unary OP> constexpr bool kStreamed = OP == Unary::Gelu || OP == Unary::Dropout || OP == Unary::Uniform;

template <typename T, Unary OP>
__global__ __launch_bounds__(256) void unary_stream_kernel(const T *__restrict__ x, T *__restrict__ y, int64_t n,
                                                           UnaryArgs u) {
    if constexpr (OP == Unary::Dropout || OP == Unary::Uniform)
        if (u.key_dev) u.key = *u.key_dev;
    if constexpr (OP == Unary::Dropout) u.inv_keep = 1.0 / (double)(T(1) - (T)u.p0);
    constexpr bool reads = OP != Unary::Uniform;
    auto run = [&](const auto &tb) {
        using NV = typename NtVec<T>::type;
        constexpr int V = Vec16<T>::V;
        const int64_t nv = n / V;
        const int64_t stride = (int64_t)gridDim.x * kMapThreads;
        const NV *xv = reinterpret_cast<const NV *>(x);
        NV *yv = reinterpret_cast<NV *>(y);
        constexpr int B = kStreamBatch<OP>;
        const int64_t v0 = (int64_t)blockIdx.x * kMapThreads + threadIdx.x;
        // every load is issued (an index past the end reads the last vector,
        // which is not stored), so the wait counts are exact on every path
        auto load = [&](NV (&buf)[B], int64_t base) {
#pragma unroll
            for (int j = 0; j < B; ++j) {
                const int64_t v = base + j * stride;
                if (reads) buf[j] = __builtin_nontemporal_load(xv + (v < nv ? v : nv - 1));
            }
        };
        auto eval_store = [&](const NV (&buf)[B], int64_t base, auto checked) {
#pragma unroll
            for (int j = 0; j < B; ++j) {
                const int64_t v = base + j * stride;
                if (decltype(checked)::value && v >= nv) break;
                const NV cur = buf[j];
                NV out;
#pragma unroll
                for (int i = 0; i < V; ++i) out[i] = unary_one<T, OP>(cur[i], T(0), v * V + i, u, tb);
                __builtin_nontemporal_store(out, yv + v);
            }
        };
        NV ba[B] = {}, bb[B] = {};
        if (nv > 0) {
            // whole rounds (every thread's 2 B vectors below nv): no bounds
            // branches, and the barriers keep the next buffer's loads ahead of
            // this buffer's arithmetic; then one checked round
            const int64_t full = nv / (2 * B * stride);
            int64_t base = v0;
            load(ba, base);
            for (int64_t r = 0; r < full; ++r, base += 2 * B * stride) {
                load(bb, base + B * stride);
                __builtin_amdgcn_sched_barrier(0);
                eval_store(ba, base, std::false_type{});
                load(ba, base + 2 * B * stride);
                __builtin_amdgcn_sched_barrier(0);
                eval_store(bb, base + B * stride, std::false_type{});
            }
            load(bb, base + B * stride);
            eval_store(ba, base, std::true_type{});
            eval_store(bb, base + B * stride, std::true_type{});
        }
        // tail: the last n % V elements
        const int64_t t = nv * V + (int64_t)blockIdx.x * kMapThreads + threadIdx.x;
        if (t < n) y[t] = unary_one<T, OP>(reads ? x[t] : T(0), T(0), t, u, tb);
    };
    if constexpr (OP == Unary::Gelu && sizeof(T) == 4) {
        __shared__ ErfcLdsStore gtab;
        gtab.fill<kMapThreads>();
        __syncthreads();
        run(gtab.tabs());
    } else {
        run(ErfcTablesConst{});
    }
}


// ---------------------------------------------------------------- host helpers
int32_t check_input_against(const chelis_gpu_tensor *in, const chelis_gpu_tensor *out, const char *name) {
    if (int32_t s = check_tensor(in, name)) return s;
    if (in->dtype != out->dtype) return set_error(CHELIS_HIP_EDOMAIN, "%s: dtype differs from the output", name);
    if (in->rank != out->rank) return set_error(CHELIS_HIP_EDOMAIN, "%s: rank differs from the output", name);
    for (int32_t a = 0; a < in->rank; ++a)
        if (in->shape[a] != out->shape[a] && in->shape[a] != 1)
            return set_error(CHELIS_HIP_EDOMAIN, "%s: axis %d neither matches nor broadcasts", name, a);
    return CHELIS_HIP_OK;
}

template <typename T, Unary OP>
int32_t launch_unary(const chelis_gpu_tensor *x, const chelis_gpu_tensor *g, const chelis_gpu_tensor *y,
                     const UnaryArgs &u) {
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    const int64_t n = y->count;
    if (!n) return CHELIS_HIP_OK;
    constexpr int V = Vec16<T>::V;
    const int64_t nv = n / V;
    if constexpr (kStreamed<OP>) {
        // exactly the workgroups that are resident at once (a second round
        // of a few would leave most of the chip idle at the end)
        static const int per_cu = [] {
            int b = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, unary_stream_kernel<T, OP>, 256, 0) != hipSuccess ||
                b < 1)
                b = 1;
            return b;
        }();
        int64_t blocks = std::min<int64_t>((nv + 255) / 256, (int64_t)device_cus() * per_cu);
        if (blocks < 1) blocks = 1;
        unary_stream_kernel<T, OP><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
            x ? (const T *)x->data : nullptr, (T *)y->data, n, u);
        CHELIS_LAUNCH_CHECK();
        return CHELIS_HIP_OK;
    } else {
        // one 16-byte vector per thread up to 2^16 blocks (16 Mi vectors),
        // grid-stride beyond
        int64_t blocks = (nv + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        if (blocks < 1) blocks = 1;
        unary_kernel<T, OP><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
            x ? (const T *)x->data : nullptr, g ? (const T *)g->data : nullptr, (T *)y->data, n, u);
        CHELIS_LAUNCH_CHECK();
        return CHELIS_HIP_OK;
    }
}

bool vec_aligned(const chelis_gpu_tensor *t) { return (reinterpret_cast<uintptr_t>(t->data) & 15u) == 0; }

template <bool ADJ>
int32_t launch_narrow_relu(const chelis_gpu_tensor *x, const chelis_gpu_tensor *g, const chelis_gpu_tensor *y) {
    hipStream_t st = stream();
    if (!st) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    const int64_t n = y->count;
    if (!n) return CHELIS_HIP_OK;
    int64_t blocks = (n / 8 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    const uint16_t *xp = (const uint16_t *)x->data, *gp = g ? (const uint16_t *)g->data : nullptr;
    uint16_t *yp = (uint16_t *)y->data;
    if (y->dtype == CHELIS_DTYPE_BF16)
        narrow_relu_kernel<Narrow::Bf16, ADJ><<<(unsigned)blocks, 256, 0, st>>>(xp, gp, yp, n);
    else
        narrow_relu_kernel<Narrow::F16, ADJ><<<(unsigned)blocks, 256, 0, st>>>(xp, gp, yp, n);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

template <Unary OP>
int32_t unary_entry(const char *what, const chelis_gpu_tensor *x, const chelis_gpu_tensor *g,
                    const chelis_gpu_tensor *y, const UnaryArgs &u) {
    int32_t s;
    if ((s = check_tensor(y, "y"))) return s;
    const bool narrow = is_narrow16(y->dtype);
    if (narrow && OP != Unary::Relu && OP != Unary::ReluAdjoint)
        return set_error(CHELIS_HIP_EUNSUPPORTED, "%s: bf16/f16 operands are admitted for relu and its adjoint only",
                         what);
    if (!narrow && !is_float(y->dtype)) return set_error(CHELIS_HIP_EDOMAIN, "%s: dtype must be f32 or f64", what);
    for (const chelis_gpu_tensor *t : {x, g}) {
        if (!t) continue;
        if ((s = check_tensor(t, "operand"))) return s;
        if (t->dtype != y->dtype || !same_shape(t, y))
            return set_error(CHELIS_HIP_EDOMAIN, "%s: operand shape/dtype must equal the result's", what);
    }
    for (const chelis_gpu_tensor *t : {x, g, y})
        if (t && (!is_contiguous(t) || (t->count && !vec_aligned(t))))
            return set_error(CHELIS_HIP_EUNSUPPORTED, "%s: operands must be contiguous and 16-byte aligned", what);
    if (narrow) {
        if constexpr (OP == Unary::Relu || OP == Unary::ReluAdjoint)
            return launch_narrow_relu<OP == Unary::ReluAdjoint>(x, g, y);
    }
    return y->dtype == CHELIS_DTYPE_F32 ? launch_unary<float, OP>(x, g, y, u) : launch_unary<double, OP>(x, g, y, u);
}

int32_t check_rate(double rate, chelis_dtype dt) {
    // The C lane checks the dtype-rounded rate widened to f64 (emit.rs:6166).
    const double r = dt == CHELIS_DTYPE_F32 ? (double)(float)rate : rate;
    if (!(r >= 0.0 && r < 1.0))
        return set_error(CHELIS_HIP_EDOMAIN, "numeric trap: domain in dropout at %s",
                         dt == CHELIS_DTYPE_F32 ? "f32" : "f64");
    return CHELIS_HIP_OK;
}

}  // namespace

}  // namespace chelis

using namespace chelis;

namespace chelis {
namespace {

int32_t load_chain_steps(const chelis_fused_chain *chain, int32_t n_inputs, ChainDev *ch) {
    if (!chain) return set_error(CHELIS_HIP_EDOMAIN, "fused_elementwise: null chain");
    if (n_inputs < 0 || n_inputs > CHELIS_FUSED_MAX_INPUTS)
        return set_error(CHELIS_HIP_EDOMAIN, "fused_elementwise: %d inputs (max %d)", n_inputs, CHELIS_FUSED_MAX_INPUTS);
    if (chain->n_steps < 1 || chain->n_steps > CHELIS_FUSED_MAX_STEPS)
        return set_error(CHELIS_HIP_EDOMAIN, "fused_elementwise: %d steps (1..%d)", chain->n_steps, CHELIS_FUSED_MAX_STEPS);
    *ch = ChainDev{};
    ch->n_steps = chain->n_steps;
    for (int32_t i = 0; i < chain->n_steps; ++i) {
        const chelis_fused_step &st = chain->steps[i];
        if (st.op >= CHELIS_FUSED_COUNT_) return set_error(CHELIS_HIP_EDOMAIN, "fused_elementwise: step %d op %d", i, st.op);
        for (int j = 0; j < 2; ++j) {
            const int32_t a = st.args[j];
            if ((a >= 0 && a >= n_inputs) || (a < 0 && -a - 1 >= i))
                return set_error(CHELIS_HIP_EDOMAIN, "fused_elementwise: step %d arg %d out of range", i, j);
        }
        ch->op[i] = st.op;
        ch->a0[i] = (int8_t)st.args[0];
        ch->a1[i] = (int8_t)st.args[1];
        ch->imm[i] = st.imm;
    }
    return CHELIS_HIP_OK;
}

// One (inputs, output) group checked and collapsed; *flat when every
// operand streams with the output or is a single broadcast element.
int32_t prepare_group(const chelis_gpu_tensor *const *inputs, int32_t n_inputs, const chelis_gpu_tensor *out,
                      Shape *sh, int64_t (*st)[kMaxRank], bool *flat, bool allow_narrow = false) {
    int32_t s;
    if ((s = check_tensor(out, "out"))) return s;
    if (!is_float(out->dtype) && !(allow_narrow && is_narrow16(out->dtype)))
        return set_error(CHELIS_HIP_EUNSUPPORTED, "fused_elementwise: f32/f64 chains only");
    if (!is_contiguous(out)) return set_error(CHELIS_HIP_EUNSUPPORTED, "fused_elementwise: output must be contiguous");
    if (n_inputs && !inputs) return set_error(CHELIS_HIP_EDOMAIN, "fused_elementwise: null input array");
    for (int32_t k = 0; k < n_inputs; ++k)
        if ((s = check_input_against(inputs[k], out, "input"))) return s;
    if (!collapse(out, inputs, n_inputs, sh, st))
        return set_error(CHELIS_HIP_EUNSUPPORTED, "fused_elementwise: more than %d independent axes", kMaxRank);
    *flat = sh->rank <= 1;
    for (int32_t k = 0; k < n_inputs && *flat; ++k) *flat = st[k][0] == 0 || st[k][0] == 1;
    return CHELIS_HIP_OK;
}

// The vector form when every streamed pointer is 16-byte aligned and the
// chain's slots fit 64 KiB of LDS; the scalar interpreter otherwise.
template <typename T>
int32_t launch_flat(const ChainDev &ch, FlatGroups &fg, hipStream_t strm) {
    constexpr int64_t V = 16 / sizeof(T);
    const size_t lds = (size_t)(fg.n_in + ch.n_steps) * 256 * 16;
    bool vec = lds <= 65536;
    for (int32_t i = 0; vec && i < fg.n; ++i) {
        vec = (reinterpret_cast<uintptr_t>(fg.g[i].out) & 15u) == 0;
        for (int32_t k = 0; vec && k < fg.n_in; ++k)
            vec = ((fg.g[i].bcast >> k) & 1u) || (reinterpret_cast<uintptr_t>(fg.g[i].in[k]) & 15u) == 0;
    }
    if (vec) {
        int64_t blocks = 0;
        for (int32_t i = 0; i < fg.n; ++i) {
            fg.g[i].first_block = blocks;
            blocks += (fg.g[i].count + 256 * V - 1) / (256 * V);
        }
        if (blocks == 0) return CHELIS_HIP_OK;
        if (!grid_fits(blocks, 256)) return set_error(CHELIS_HIP_EUNSUPPORTED, "fused_elementwise: too many elements");
        fused_flat_vec_kernel<T><<<(unsigned)blocks, 256, lds, strm>>>(ch, fg);
        CHELIS_LAUNCH_CHECK();
        return CHELIS_HIP_OK;
    }
    int64_t blocks = 0;
    for (int32_t i = 0; i < fg.n; ++i) {
        fg.g[i].first_block = blocks;
        blocks += (fg.g[i].count + 255) / 256;
    }
    if (blocks == 0) return CHELIS_HIP_OK;
    if (!grid_fits(blocks, 256)) return set_error(CHELIS_HIP_EUNSUPPORTED, "fused_elementwise: too many elements");
    fused_flat_kernel<T><<<(unsigned)blocks, 256, 0, strm>>>(ch, fg);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

void add_group(FlatGroups &fg, const chelis_gpu_tensor *const *inputs, int32_t n_inputs, const chelis_gpu_tensor *out,
               const int64_t (*st)[kMaxRank]) {
    FlatGroup &g = fg.g[fg.n++];
    g = FlatGroup{};
    for (int32_t k = 0; k < n_inputs; ++k) {
        g.in[k] = inputs[k]->data;
        if (st[k][0] == 0) g.bcast |= 1u << k;
    }
    g.out = out->data;
    g.count = out->count;
}

}  // namespace

int32_t fused_elementwise_groups(const chelis_fused_chain *chain, int32_t n_inputs,
                                 const chelis_gpu_tensor *const *inputs, const chelis_gpu_tensor *const *outs,
                                 int32_t n_groups) {
    ChainDev ch;
    if (int32_t s = load_chain_steps(chain, n_inputs, &ch)) return s;
    if (n_groups < 1 || !outs) return set_error(CHELIS_HIP_EDOMAIN, "fused_elementwise: no groups");
    hipStream_t strm = stream();
    if (!strm) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    const chelis_dtype dt = outs[0] ? outs[0]->dtype : CHELIS_DTYPE_F32;
    FlatGroups fg{};
    fg.n_in = n_inputs;
    for (int32_t i = 0; i < n_groups; ++i) {
        const chelis_gpu_tensor *const *in = inputs + (size_t)i * n_inputs;
        Shape sh;
        int64_t st[CHELIS_FUSED_MAX_INPUTS][kMaxRank];
        bool flat = false;
        if (int32_t s = prepare_group(in, n_inputs, outs[i], &sh, st, &flat)) return s;
        if (outs[i]->dtype != dt) return set_error(CHELIS_HIP_EDOMAIN, "fused_elementwise: groups differ in dtype");
        if (!flat) {
            // a strided group runs on its own
            if (int32_t s = chelis_hip_fused_elementwise(chain, in, n_inputs, outs[i])) return s;
            continue;
        }
        if (fg.n == kMaxGroups) {
            if (int32_t s = dt == CHELIS_DTYPE_F32 ? launch_flat<float>(ch, fg, strm) : launch_flat<double>(ch, fg, strm))
                return s;
            fg.n = 0;
        }
        add_group(fg, in, n_inputs, outs[i], st);
    }
    if (fg.n == 0) return CHELIS_HIP_OK;
    return dt == CHELIS_DTYPE_F32 ? launch_flat<float>(ch, fg, strm) : launch_flat<double>(ch, fg, strm);
}

}  // namespace chelis

using namespace chelis;

extern "C" int32_t chelis_hip_fused_elementwise(const chelis_fused_chain *chain, const chelis_gpu_tensor *const *inputs,
                                                int32_t n_inputs, const chelis_gpu_tensor *out) {
    ChainDev ch;
    if (int32_t s = load_chain_steps(chain, n_inputs, &ch)) return s;
    const bool narrow = out && is_narrow16(out->dtype);
    if (narrow) {
        // 16-bit chains: sub / max_elem / min_elem steps only (emit.rs:2292-2319)
        for (int32_t i = 0; i < ch.n_steps; ++i)
            if (ch.op[i] != CHELIS_FUSED_SUB && ch.op[i] != CHELIS_FUSED_MAX_ELEM && ch.op[i] != CHELIS_FUSED_MIN_ELEM)
                return set_error(CHELIS_HIP_EUNSUPPORTED,
                                 "fused_elementwise: bf16/f16 chain step %d is outside sub/max_elem/min_elem", i);
    }
    Shape sh;
    int64_t st[CHELIS_FUSED_MAX_INPUTS][kMaxRank];
    bool flat = false;
    if (int32_t s = prepare_group(inputs, n_inputs, out, &sh, st, &flat, true)) return s;
    if (!out->count) return CHELIS_HIP_OK;
    hipStream_t strm = stream();
    if (!strm) return set_error(CHELIS_HIP_EHIP, "no HIP device");
    if (narrow) {
        Operands ops{};
        ops.n = n_inputs;
        for (int32_t k = 0; k < n_inputs; ++k) {
            ops.o[k].p = inputs[k]->data;
            for (int a = 0; a < kMaxRank; ++a) ops.o[k].st[a] = st[k][a];
        }
        int64_t blocks = (out->count + 255) / 256;
        if (blocks > 8192) blocks = 8192;
        if (out->dtype == CHELIS_DTYPE_BF16)
            narrow_chain_kernel<Narrow::Bf16><<<(unsigned)blocks, 256, 0, strm>>>(ch, ops, sh, (uint16_t *)out->data,
                                                                                 out->count);
        else
            narrow_chain_kernel<Narrow::F16><<<(unsigned)blocks, 256, 0, strm>>>(ch, ops, sh, (uint16_t *)out->data,
                                                                                out->count);
        CHELIS_LAUNCH_CHECK();
        return CHELIS_HIP_OK;
    }
    if (flat) {
        FlatGroups fg{};
        fg.n_in = n_inputs;
        add_group(fg, inputs, n_inputs, out, st);
        return out->dtype == CHELIS_DTYPE_F32 ? launch_flat<float>(ch, fg, strm) : launch_flat<double>(ch, fg, strm);
    }
    Operands ops{};
    ops.n = n_inputs;
    for (int32_t k = 0; k < n_inputs; ++k) {
        ops.o[k].p = inputs[k]->data;
        for (int a = 0; a < kMaxRank; ++a) ops.o[k].st[a] = st[k][a];
    }
    int64_t blocks = (out->count + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (out->dtype == CHELIS_DTYPE_F32)
        fused_chain_kernel<float><<<(unsigned)blocks, 256, 0, strm>>>(ch, ops, sh, (float *)out->data, out->count);
    else
        fused_chain_kernel<double><<<(unsigned)blocks, 256, 0, strm>>>(ch, ops, sh, (double *)out->data, out->count);
    CHELIS_LAUNCH_CHECK();
    return CHELIS_HIP_OK;
}

extern "C" int32_t chelis_hip_gelu(const chelis_gpu_tensor *x, const chelis_gpu_tensor *y) {
    // the exact mode: the Phi graph bit for bit; else the direct binary32
    // evaluation (binary64 is the graph either way)
    if (exact_mode() || (y && y->dtype != CHELIS_DTYPE_F32))
        return unary_entry<Unary::Gelu>("gelu", x, nullptr, y, UnaryArgs{});
    return unary_entry<Unary::GeluFast>("gelu", x, nullptr, y, UnaryArgs{});
}

extern "C" int32_t chelis_hip_relu(const chelis_gpu_tensor *x, const chelis_gpu_tensor *y) {
    return unary_entry<Unary::Relu>("relu", x, nullptr, y, UnaryArgs{});
}

extern "C" int32_t chelis_hip_relu_adjoint(const chelis_gpu_tensor *x, const chelis_gpu_tensor *g,
                                           const chelis_gpu_tensor *dx) {
    return unary_entry<Unary::ReluAdjoint>("relu_adjoint", x, g, dx, UnaryArgs{});
}

namespace chelis {
uint64_t dropout_cut(double rate, chelis_dtype dt) {
    // The unit of a word is m * 2^-53 (m = word >> 11, exact in binary64),
    // taken to the dtype (binary32: rounded to nearest, a monotone map) and
    // compared with the dtype's rate: unit < rate holds exactly for m in a
    // prefix [0, cut). cut is the least m whose unit is not below the rate,
    // found by bisection over [0, 2^53].
    const bool f32 = dt == CHELIS_DTYPE_F32;
    auto below = [&](uint64_t m) {
        const double v = (double)m * 0x1p-53;
        return f32 ? (float)v < (float)rate : v < rate;
    };
    uint64_t lo = 0, hi = uint64_t(1) << 53;  // below(hi) is false: units are < 1 <= any rate tested here
    if (!below(hi - 1)) {
        while (lo < hi) {
            const uint64_t mid = lo + (hi - lo) / 2;
            if (below(mid)) lo = mid + 1;
            else hi = mid;
        }
    } else {
        lo = hi;
    }
    return lo;
}

int32_t dropout_device_key(const uint64_t *key_dev, const chelis_gpu_tensor *x, double rate,
                           const chelis_gpu_tensor *y) {
    if (!key_dev) return set_error(CHELIS_HIP_EDOMAIN, "dropout: null key");
    if (!y || !is_float(y->dtype)) return set_error(CHELIS_HIP_EDOMAIN, "dropout: f32 or f64 result required");
    if (int32_t s = check_rate(rate, y->dtype)) return s;
    UnaryArgs u{0, rate, 0.0, key_dev};
    u.cut = dropout_cut(rate, y->dtype);
    return unary_entry<Unary::Dropout>("dropout", x, nullptr, y, u);
}
}  // namespace chelis

extern "C" uint64_t chelis_hip_dropout_cut(double rate, int32_t dtype) {
    return chelis::dropout_cut(rate, (chelis_dtype)dtype);
}

extern "C" int32_t chelis_hip_dropout(uint64_t key, const chelis_gpu_tensor *x, double rate,
                                      const chelis_gpu_tensor *y) {
    if (!y || !is_float(y->dtype)) return set_error(CHELIS_HIP_EDOMAIN, "dropout: f32 or f64 result required");
    if (int32_t s = check_rate(rate, y->dtype)) return s;
    UnaryArgs u{key, rate, 0.0, nullptr};
    u.cut = dropout_cut(rate, y->dtype);
    return unary_entry<Unary::Dropout>("dropout", x, nullptr, y, u);
}

extern "C" int32_t chelis_hip_dropout_replay(uint64_t key, const chelis_gpu_tensor *g, double rate,
                                             const chelis_gpu_tensor *dx) {
    // [05-OP-37] adjoint: the forward mask on the cotangent, kept values
    // divided by (1 - rate); the same kernel with g in place of x.
    if (!dx || !is_float(dx->dtype)) return set_error(CHELIS_HIP_EDOMAIN, "dropout_replay: f32 or f64 result required");
    if (int32_t s = check_rate(rate, dx->dtype)) return s;
    UnaryArgs u{key, rate, 0.0, nullptr};
    u.cut = dropout_cut(rate, dx->dtype);
    return unary_entry<Unary::Dropout>("dropout_replay", g, nullptr, dx, u);
}

namespace chelis {
// [05-OP-8]'s bounds at the draw's dtype: finite, ordered, a finite span.
int32_t uniform_like_run(uint64_t key, const uint64_t *key_dev, double low, double high,
                         const chelis_gpu_tensor *out) {
    if (!out || !is_float(out->dtype)) return set_error(CHELIS_HIP_EDOMAIN, "uniform_like: f32 or f64 result required");
    const bool f32 = out->dtype == CHELIS_DTYPE_F32;
    const double lo = f32 ? (double)(float)low : low, hi = f32 ? (double)(float)high : high;
    const double span = f32 ? (double)((float)hi - (float)lo) : hi - lo;
    if (!(std::isfinite(lo) && std::isfinite(hi) && lo <= hi && std::isfinite(span)))
        return set_error(CHELIS_HIP_EDOMAIN, "numeric trap: domain in uniform_like at %s", f32 ? "f32" : "f64");
    return unary_entry<Unary::Uniform>("uniform_like", nullptr, nullptr, out, UnaryArgs{key, low, high, key_dev});
}
}  // namespace chelis

extern "C" int32_t chelis_hip_uniform_like(uint64_t key, double low, double high, const chelis_gpu_tensor *out) {
    return chelis::uniform_like_run(key, nullptr, low, high, out);
}
