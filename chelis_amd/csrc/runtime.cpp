// Host tensors and checked metadata plans: the runtime C ABI subset that
// generated entries and the device owner call (include/chelis_runtime.h).
//
// Semantics follow the reference runtime: chelis_alloc zero-fills
// (crates/chelis-runtime/src/lib.rs:2155), tensors are refcounted with a
// single write lease (lib.rs:1070-1095), and metadata plans validate rank,
// extents, strides, element and byte counts with checked i64 arithmetic
// (crates/chelis-abi/src/metadata.rs:81-170, lib.rs:3022-3135). Every
// violation traps through chelis_numeric_trap with the reference's message.
#include "chelis_runtime.h"

#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <new>
#include <vector>

namespace {

[[noreturn]] void trap_domain() {
    chelis_numeric_trap("numeric trap: domain in metadata_plan at i64");
    std::abort();
}
[[noreturn]] void trap_overflow() {
    chelis_numeric_trap("numeric trap: overflow in metadata_plan at i64");
    std::abort();
}
[[noreturn]] void trap_tensor(const char *what) {
    std::fprintf(stderr, "chelis runtime: %s\n", what);
    chelis_flush_and_exit_trap();
    std::abort();
}

int64_t width_of(chelis_dtype dtype) {
    switch (dtype) {
        case CHELIS_DTYPE_F32: return 4;
        case CHELIS_DTYPE_F64: return 8;
        case CHELIS_DTYPE_I32: return 4;
        case CHELIS_DTYPE_BOOL: return 1;
        case CHELIS_DTYPE_I64: return 8;
        case CHELIS_DTYPE_BF16: return 2;
        case CHELIS_DTYPE_F16: return 2;
        case CHELIS_DTYPE_I8: return 1;
        case CHELIS_DTYPE_I16: return 2;
        case CHELIS_DTYPE_KEY: return 8;
        default: return 0;
    }
}

bool checked_mul(int64_t a, int64_t b, int64_t *out) { return !__builtin_mul_overflow(a, b, out); }
bool checked_add(int64_t a, int64_t b, int64_t *out) { return !__builtin_add_overflow(a, b, out); }

// A scalar that carries an exact i64 (the metadata carrier).
int64_t i64_of(const chelis_scalar &s) {
    if (s.dtype != CHELIS_DTYPE_I64) trap_domain();
    for (uint8_t b : s.reserved)
        if (b) trap_domain();
    return static_cast<int64_t>(s.bits);
}

int64_t element_count(const std::vector<int64_t> &shape) {
    int64_t n = 1;
    for (int64_t e : shape) {
        if (e < 0) trap_domain();
        if (!checked_mul(n, e, &n)) trap_overflow();
    }
    return n;
}

int64_t byte_count(int64_t elements, chelis_dtype dtype) {
    int64_t w = width_of(dtype);
    if (!w) trap_domain();
    int64_t b;
    if (!checked_mul(elements, w, &b)) trap_overflow();
    // Allocation bytes must be addressable on the host.
    if (static_cast<uint64_t>(b) > static_cast<uint64_t>(std::numeric_limits<ptrdiff_t>::max())) trap_overflow();
    return b;
}

std::vector<int64_t> contiguous_strides(const std::vector<int64_t> &shape) {
    std::vector<int64_t> st(shape.size());
    int64_t acc = 1;
    for (size_t i = shape.size(); i-- > 0;) {
        st[i] = acc;
        int64_t e = shape[i] > 0 ? shape[i] : 1;
        if (!checked_mul(acc, e, &acc)) trap_overflow();
    }
    return st;
}

}  // namespace

struct chelis_tensor {
    mutable std::atomic<int64_t> refs{1};
    std::atomic<int32_t> writers{0};
    int32_t rank = 0;
    std::vector<int64_t> shape;
    chelis_dtype dtype = 0;
    int64_t count = 0;
    int64_t bytes = 0;
    void *data = nullptr;
    bool owned = false;
};

struct chelis_tensor_write {
    chelis_tensor *tensor;
};

struct chelis_metadata_plan {
    int32_t rank = 0;
    std::vector<int64_t> shape;
    std::vector<int64_t> strides;
    chelis_dtype dtype = 0;
    int64_t count = 0;
    int64_t bytes = 0;          // logical bytes (count * width)
    int64_t required_span = 0;  // bytes a storage must hold
};

namespace {

chelis_tensor *make_tensor(int32_t rank, const int64_t *shape, chelis_dtype dtype) {
    if (rank < 0 || (rank > 0 && !shape)) trap_domain();
    auto *t = new (std::nothrow) chelis_tensor();
    if (!t) trap_tensor("host tensor allocation failed");
    t->rank = rank;
    t->shape.assign(shape, shape + rank);
    t->dtype = dtype;
    t->count = element_count(t->shape);
    t->bytes = byte_count(t->count, dtype);
    return t;
}

std::vector<int64_t> read_array(chelis_scalar rank, const chelis_scalar *values, int32_t *out_rank) {
    int64_t r = i64_of(rank);
    if (r < 0 || r > std::numeric_limits<int32_t>::max()) trap_domain();
    if (r > 0 && (!values || reinterpret_cast<uintptr_t>(values) % alignof(chelis_scalar))) trap_domain();
    std::vector<int64_t> out(static_cast<size_t>(r));
    for (int64_t i = 0; i < r; ++i) out[i] = i64_of(values[i]);
    *out_rank = static_cast<int32_t>(r);
    return out;
}

chelis_dtype exemplar_dtype(const chelis_scalar &exemplar) {
    if (!width_of(exemplar.dtype)) trap_domain();
    return exemplar.dtype;
}

const chelis_metadata_plan &plan_ref(const chelis_metadata_plan *p) {
    if (!p || reinterpret_cast<uintptr_t>(p) % alignof(chelis_metadata_plan)) trap_domain();
    return *p;
}

const chelis_tensor &tensor_ref(const chelis_tensor *t) {
    if (!t || reinterpret_cast<uintptr_t>(t) % alignof(chelis_tensor)) trap_tensor("null or misaligned tensor");
    return *t;
}

}  // namespace

extern "C" {

int64_t chelis_dtype_size(chelis_dtype dtype) {
    int64_t w = width_of(dtype);
    if (!w) trap_tensor("unknown dtype");
    return w;
}

chelis_scalar chelis_scalar_from_bits(chelis_dtype dtype, uint64_t bits) {
    chelis_scalar s{};
    s.dtype = dtype;
    s.bits = bits;
    return s;
}

chelis_key chelis_key_from_seed(int64_t seed) { return chelis_key{static_cast<uint64_t>(seed)}; }

chelis_tensor *chelis_alloc(int32_t rank, const int64_t *shape, chelis_dtype dtype) {
    chelis_tensor *t = make_tensor(rank, shape, dtype);
    if (t->bytes) {
        t->data = std::calloc(1, static_cast<size_t>(t->bytes));
        if (!t->data) trap_tensor("host tensor allocation failed");
    }
    t->owned = true;
    return t;
}

chelis_tensor *chelis_tensor_entry_borrow(int32_t rank, const int64_t *shape, chelis_dtype dtype, const void *data,
                                          int64_t byte_capacity) {
    chelis_tensor *t = make_tensor(rank, shape, dtype);
    if (byte_capacity < t->bytes || (t->bytes && !data)) {
        delete t;
        trap_domain();
    }
    t->data = const_cast<void *>(data);
    t->owned = false;
    return t;
}

void chelis_tensor_retain(const chelis_tensor *tensor) {
    tensor_ref(tensor).refs.fetch_add(1, std::memory_order_relaxed);
}

void chelis_tensor_release(const chelis_tensor *tensor) {
    auto *t = const_cast<chelis_tensor *>(&tensor_ref(tensor));
    if (t->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) {
        if (t->owned) std::free(t->data);
        delete t;
    }
}

chelis_read_view chelis_tensor_read_view(const chelis_tensor *tensor) {
    const chelis_tensor &t = tensor_ref(tensor);
    chelis_read_view v{};
    v.data = t.data;
    v.count = t.count;
    v.dtype = t.dtype;
    return v;
}

chelis_tensor_write *chelis_tensor_begin_write(chelis_tensor *tensor) {
    auto &t = const_cast<chelis_tensor &>(tensor_ref(tensor));
    int32_t expected = 0;
    if (!t.writers.compare_exchange_strong(expected, 1)) trap_tensor("tensor already has a write lease");
    auto *g = new (std::nothrow) chelis_tensor_write{&t};
    if (!g) trap_tensor("write guard allocation failed");
    return g;
}

chelis_write_view chelis_tensor_write_view(const chelis_tensor_write *guard) {
    if (!guard) trap_tensor("null write guard");
    chelis_write_view v{};
    v.data = guard->tensor->data;
    v.count = guard->tensor->count;
    v.dtype = guard->tensor->dtype;
    return v;
}

void chelis_tensor_end_write(chelis_tensor_write *guard) {
    if (!guard) trap_tensor("null write guard");
    guard->tensor->writers.store(0);
    delete guard;
}

int32_t chelis_tensor_rank(const chelis_tensor *tensor) { return tensor_ref(tensor).rank; }

int64_t chelis_tensor_shape(const chelis_tensor *tensor, int32_t axis) {
    const chelis_tensor &t = tensor_ref(tensor);
    if (axis < 0 || axis >= t.rank) trap_tensor("axis out of range");
    return t.shape[axis];
}

int64_t chelis_tensor_numel(const chelis_tensor *tensor) { return tensor_ref(tensor).count; }

chelis_tensor *chelis_contiguous(const chelis_tensor *tensor) {
    chelis_tensor_retain(tensor);
    return const_cast<chelis_tensor *>(tensor);
}

chelis_metadata_plan *chelis_metadata_plan_new(chelis_scalar rank, const chelis_scalar *shape, chelis_scalar exemplar) {
    auto *p = new chelis_metadata_plan();
    p->shape = read_array(rank, shape, &p->rank);
    p->dtype = exemplar_dtype(exemplar);
    p->count = element_count(p->shape);
    p->bytes = byte_count(p->count, p->dtype);
    p->strides = contiguous_strides(p->shape);
    p->required_span = p->bytes;
    return p;
}

chelis_metadata_plan *chelis_metadata_plan_view(chelis_scalar rank, const chelis_scalar *shape,
                                                const chelis_scalar *strides, chelis_scalar exemplar,
                                                chelis_scalar byte_capacity) {
    auto *p = new chelis_metadata_plan();
    int32_t stride_rank = 0;
    p->shape = read_array(rank, shape, &p->rank);
    p->strides = read_array(rank, strides, &stride_rank);
    p->dtype = exemplar_dtype(exemplar);
    int64_t capacity = i64_of(byte_capacity);
    if (capacity < 0) trap_domain();
    for (int64_t s : p->strides)
        if (s < 0) trap_domain();  // negative stride in forward view
    p->count = element_count(p->shape);
    p->bytes = byte_count(p->count, p->dtype);
    int64_t span = 0;
    if (p->count) {
        int64_t largest = 0;
        for (int32_t a = 0; a < p->rank; ++a) {
            int64_t part;
            if (!checked_mul(p->shape[a] - 1, p->strides[a], &part)) trap_overflow();
            if (!checked_add(largest, part, &largest)) trap_overflow();
        }
        if (!checked_add(largest, 1, &span)) trap_overflow();
    }
    p->required_span = byte_count(span, p->dtype);
    if (p->required_span > capacity) trap_domain();
    return p;
}

int32_t chelis_metadata_plan_rank(const chelis_metadata_plan *plan) { return plan_ref(plan).rank; }

const int64_t *chelis_metadata_plan_shape(const chelis_metadata_plan *plan) {
    const auto &p = plan_ref(plan);
    return p.shape.empty() ? nullptr : p.shape.data();
}

const int64_t *chelis_metadata_plan_strides(const chelis_metadata_plan *plan) {
    const auto &p = plan_ref(plan);
    return p.strides.empty() ? nullptr : p.strides.data();
}

int64_t chelis_metadata_plan_count(const chelis_metadata_plan *plan) { return plan_ref(plan).count; }

int64_t chelis_metadata_plan_byte_count(const chelis_metadata_plan *plan) { return plan_ref(plan).bytes; }

int64_t chelis_metadata_plan_byte_offset(const chelis_metadata_plan *plan, chelis_scalar linear_index) {
    const auto &p = plan_ref(plan);
    int64_t index = i64_of(linear_index);
    if (index < 0 || index >= p.count) trap_domain();
    int64_t offset = 0;
    for (int32_t a = p.rank; a-- > 0;) {
        int64_t coord = index % p.shape[a];
        index /= p.shape[a];
        int64_t part;
        if (!checked_mul(coord, p.strides[a], &part) || !checked_add(offset, part, &offset)) trap_overflow();
    }
    int64_t bytes;
    if (!checked_mul(offset, width_of(p.dtype), &bytes)) trap_overflow();
    return bytes;
}

chelis_dtype chelis_metadata_plan_dtype(const chelis_metadata_plan *plan) { return plan_ref(plan).dtype; }

void chelis_metadata_plan_check_capacity(const chelis_metadata_plan *plan, chelis_scalar byte_capacity) {
    const auto &p = plan_ref(plan);
    int64_t capacity = i64_of(byte_capacity);
    if (capacity < 0 || p.required_span > capacity) trap_domain();
}

void chelis_metadata_plan_release(chelis_metadata_plan *plan) {
    plan_ref(plan);
    delete plan;
}

}  // extern "C"
