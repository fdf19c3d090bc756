// Device tensor owners: the opaque-owner C ABI of include/chelis_device_owner.h.
//
// Contract (crates/chelis-backend-hip/runtime/chelis_device_owner.h:16-24,
// normative spec/11-ffi.md): an owner keeps its checked metadata plan and
// either owns zero-filled storage (alloc, clone) or borrows the caller's
// (borrow, import); observations are valid on the owner's device only;
// every invalid request ends the process through the runtime's numeric trap
// (`domain` / `overflow` in metadata_plan); a failed HIP call aborts; no C++
// exception reaches a C caller.
//
// Layout of this file:
//  * Record    - what an owner is: plan, storage, device, the packet it
//                hands out (pointing into the plan's own shape / strides).
//  * Checks    - the trap channel and the preflight of foreign arrays.
//  * Copies    - the one copy engine every data movement goes through: a
//                dense view is one hipMemcpyAsync, any other view one
//                strided-gather launch on the library stream (the reference
//                issues one blocking hipMemcpy per element,
//                chelis_device_owner.cpp:213-233,254-273). Strided host
//                copies gather into library scratch first.
//  * ABI       - the nine extern "C" entries.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <vector>

#include "chelis_device_owner.h"
#include "hip_common.h"

// ======================================================================= Record
struct chelis_device_tensor_owner {
    chelis_metadata_plan *plan;  // retained for the owner's lifetime
    void *storage;               // device pointer (null for an empty tensor)
    bool owns_storage;
    int32_t device;
    chelis_gpu_tensor packet;
};

namespace {

// ======================================================================= Checks
enum class Trap { Domain, Overflow };

[[noreturn]] void trap(Trap kind) {
    chelis_numeric_trap(kind == Trap::Domain ? "numeric trap: domain in metadata_plan at i64"
                                             : "numeric trap: overflow in metadata_plan at i64");
    std::abort();
}

void hip_must(hipError_t status, const char *what) {
    if (status == hipSuccess) return;
    std::fprintf(stderr, "HIP device owner failure: %s: %s\n", what, hipGetErrorString(status));
    std::abort();
}

int32_t device_now() {
    int device = -1;
    hip_must(hipGetDevice(&device), "hipGetDevice");
    if (device < 0) trap(Trap::Domain);
    return device;
}

// Every ABI body runs here: a C++ exception (a failed metadata allocation)
// is reported and the process aborts instead of unwinding into C.
template <class Body>
auto at_boundary(Body &&body) noexcept -> decltype(body()) {
    try {
        return body();
    } catch (const std::exception &error) {
        std::fprintf(stderr, "device metadata allocation failed: %s\n", error.what());
        std::abort();
    } catch (...) {
        std::fprintf(stderr, "device metadata allocation failed\n");
        std::abort();
    }
}

const chelis_device_tensor_owner &checked(const chelis_device_tensor_owner *owner) {
    if (owner == nullptr || reinterpret_cast<uintptr_t>(owner) % alignof(chelis_device_tensor_owner) != 0)
        trap(Trap::Domain);
    return *owner;
}

const chelis_device_tensor_owner &checked_here(const chelis_device_tensor_owner *owner) {
    const chelis_device_tensor_owner &o = checked(owner);
    if (device_now() != o.device) trap(Trap::Domain);
    return o;
}

// A foreign int64 array of `rank` entries, turned into the runtime's tagged
// i64 scalars. Both arrays of a packet are preflighted before either is read.
void preflight(int32_t rank, const int64_t *values) {
    if (rank < 0) trap(Trap::Domain);
    if (rank == 0) return;
    if (values == nullptr || reinterpret_cast<uintptr_t>(values) % alignof(int64_t) != 0) trap(Trap::Domain);
    if (static_cast<uint64_t>(rank) > static_cast<uint64_t>(PTRDIFF_MAX) / sizeof(chelis_scalar)) trap(Trap::Overflow);
}

std::vector<chelis_scalar> tagged_i64(int32_t rank, const int64_t *values) {
    std::vector<chelis_scalar> out(static_cast<size_t>(rank));
    for (int32_t a = 0; a < rank; ++a) out[a] = chelis_scalar_from_bits(CHELIS_DTYPE_I64, static_cast<uint64_t>(values[a]));
    return out;
}

chelis_scalar i64(int64_t v) { return chelis_scalar_from_bits(CHELIS_DTYPE_I64, static_cast<uint64_t>(v)); }

// The dtype request travels untyped: the plan constructor decides whether it
// names a dtype, so a bad tag traps as a metadata-plan domain error.
chelis_scalar dtype_request(chelis_dtype dtype) {
    chelis_scalar s{};
    s.dtype = dtype;
    return s;
}

// True when the plan's strides are the row-major strides of its shape (the
// runtime's convention: an extent of 0 or 1 steps like 1).
bool is_dense(const chelis_metadata_plan *plan) {
    const int32_t rank = chelis_metadata_plan_rank(plan);
    const int64_t *shape = chelis_metadata_plan_shape(plan), *strides = chelis_metadata_plan_strides(plan);
    int64_t step = 1;
    for (int32_t a = rank - 1; a >= 0; --a) {
        if (strides[a] != step) return false;
        step *= shape[a] > 1 ? shape[a] : 1;
    }
    return true;
}

// A fresh row-major plan with the source plan's shape and dtype.
chelis_metadata_plan *dense_plan_like(const chelis_metadata_plan *plan) {
    const int32_t rank = chelis_metadata_plan_rank(plan);
    const int64_t *shape = chelis_metadata_plan_shape(plan);
    preflight(rank, shape);
    std::vector<chelis_scalar> dims = tagged_i64(rank, shape);
    return chelis_metadata_plan_new(i64(rank), dims.empty() ? nullptr : dims.data(),
                                    dtype_request(chelis_metadata_plan_dtype(plan)));
}

int64_t element_width(const chelis_metadata_plan *plan) {
    const int64_t count = chelis_metadata_plan_count(plan);
    return count ? chelis_metadata_plan_byte_count(plan) / count : 0;
}

// Storage handed to borrow / import must be device memory of the current
// device, aligned to the element width.
void require_device_storage(const chelis_metadata_plan *plan, const void *data) {
    if (chelis_metadata_plan_count(plan) == 0) return;
    const int64_t width = element_width(plan);
    if (data == nullptr || reinterpret_cast<uintptr_t>(data) % static_cast<uintptr_t>(width) != 0) trap(Trap::Domain);
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, data) != hipSuccess) trap(Trap::Domain);
    if (attr.type != hipMemoryTypeDevice || attr.device != device_now()) trap(Trap::Domain);
}

template <class View>
void require_same_elements(const View &host, const chelis_gpu_tensor &dev) {
    if (host.count != dev.count || host.dtype != dev.dtype) trap(Trap::Domain);
    for (uint8_t byte : host.reserved)
        if (byte != 0) trap(Trap::Domain);
}

chelis_device_tensor_owner *make_owner(chelis_metadata_plan *plan, void *storage, bool owned, int64_t capacity,
                                       int32_t device) {
    auto *o = new chelis_device_tensor_owner{plan, storage, owned, device, {}};
    o->packet.data = storage;
    o->packet.shape = chelis_metadata_plan_shape(plan);
    o->packet.strides = chelis_metadata_plan_strides(plan);
    o->packet.count = chelis_metadata_plan_count(plan);
    o->packet.byte_capacity = capacity;
    o->packet.rank = chelis_metadata_plan_rank(plan);
    o->packet.dtype = chelis_metadata_plan_dtype(plan);
    o->packet.ownership = owned ? 1 : 0;
    return o;
}

void destroy_owner(chelis_device_tensor_owner *o) {
    if (o->owns_storage && o->storage) {
        // the free waits for the device, so no queued use outlives the block
        const int32_t here = device_now();
        if (here != o->device) hip_must(hipSetDevice(o->device), "hipSetDevice");
        hip_must(chelis::owner_block_free(o->storage, static_cast<size_t>(o->packet.byte_capacity)), "hipFree");
        if (here != o->device) hip_must(hipSetDevice(here), "hipSetDevice");
    }
    chelis_metadata_plan_release(o->plan);
    delete o;
}

hipStream_t library_stream() {
    hipStream_t s = chelis::stream();
    if (!s) {
        std::fprintf(stderr, "HIP device owner failure: no library stream\n");
        std::abort();
    }
    return s;
}

// ======================================================================= Copies
// A strided view as at most kCopyRank axes after dropping extent-1 axes and
// merging axes that step as one; element strides.
constexpr int kCopyRank = 12;
struct Strided {
    int32_t rank;
    int64_t extent[kCopyRank];
    int64_t stride[kCopyRank];
};

// The kernels below that index by thread run 256 threads per workgroup
// (their launches pass that count): the constant, not blockDim.x, which
// is a vector load from the dispatch packet at the start of each wave.
constexpr int kCopyThreads = 256;

template <typename W>
__global__ __launch_bounds__(256) void strided_to_dense_kernel(const W *__restrict__ src, W *__restrict__ dst,
                                                               Strided v, int64_t count) {
    const int64_t step = (int64_t)gridDim.x * kCopyThreads;
    for (int64_t i = (int64_t)blockIdx.x * kCopyThreads + threadIdx.x; i < count; i += step) {
        int64_t rem = i, off = 0;
        for (int a = v.rank - 1; a >= 0; --a) {
            const int64_t e = v.extent[a];
            off += (rem % e) * v.stride[a];
            rem /= e;
        }
        dst[i] = src[off];
    }
}

// Simplified axes of a view: extent-1 axes dropped, (a, a+1) merged when
// stride[a] == stride[a+1] * extent[a+1].
std::vector<std::pair<int64_t, int64_t>> simplify(int32_t rank, const int64_t *shape, const int64_t *strides) {
    std::vector<std::pair<int64_t, int64_t>> axes;  // (extent, stride)
    for (int32_t a = 0; a < rank; ++a) {
        if (shape[a] == 1) continue;
        if (!axes.empty() && axes.back().second == strides[a] * shape[a]) {
            axes.back() = {axes.back().first * shape[a], strides[a]};
        } else {
            axes.push_back({shape[a], strides[a]});
        }
    }
    return axes;
}

template <typename W>
void launch_gather(const W *src, W *dst, const std::pair<int64_t, int64_t> *axes, int32_t rank, int64_t count,
                   hipStream_t st) {
    if (rank > kCopyRank) {
        // peel the leading axis on the host until the rest fits the kernel
        const int64_t inner = count / axes[0].first;
        for (int64_t c = 0; c < axes[0].first; ++c)
            launch_gather<W>(src + c * axes[0].second, dst + c * inner, axes + 1, rank - 1, inner, st);
        return;
    }
    Strided v{};
    v.rank = rank;
    for (int32_t a = 0; a < rank; ++a) {
        v.extent[a] = axes[a].first;
        v.stride[a] = axes[a].second;
    }
    int64_t blocks = (count + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    strided_to_dense_kernel<W><<<(unsigned)blocks, 256, 0, st>>>(src, dst, v, count);
    hip_must(hipGetLastError(), "strided copy launch");
}

// dst (dense, on the device) <- the source owner's view, enqueued on `st`.
void copy_view_to_dense(const chelis_device_tensor_owner &src, void *dst, hipStream_t st) {
    const chelis_gpu_tensor &p = src.packet;
    if (p.count == 0) return;
    const int64_t width = element_width(src.plan);
    if (is_dense(src.plan)) {
        hip_must(hipMemcpyAsync(dst, p.data, static_cast<size_t>(p.count * width), hipMemcpyDeviceToDevice, st),
                 "hipMemcpyAsync");
        return;
    }
    const auto axes = simplify(p.rank, p.shape, p.strides);
    switch (width) {
        case 1: launch_gather<uint8_t>((const uint8_t *)p.data, (uint8_t *)dst, axes.data(), (int32_t)axes.size(), p.count, st); break;
        case 2: launch_gather<uint16_t>((const uint16_t *)p.data, (uint16_t *)dst, axes.data(), (int32_t)axes.size(), p.count, st); break;
        case 4: launch_gather<uint32_t>((const uint32_t *)p.data, (uint32_t *)dst, axes.data(), (int32_t)axes.size(), p.count, st); break;
        case 8: launch_gather<uint64_t>((const uint64_t *)p.data, (uint64_t *)dst, axes.data(), (int32_t)axes.size(), p.count, st); break;
        default: trap(Trap::Domain);
    }
}

// alloc's body: storage sized by the plan, zero-filled before the owner is
// handed out.
chelis_device_tensor_owner *allocate(chelis_metadata_plan *plan) {
    const int64_t bytes = chelis_metadata_plan_byte_count(plan);
    chelis_metadata_plan_check_capacity(plan, i64(bytes));
    const int32_t device = device_now();
    void *storage = nullptr;
    if (bytes > 0) {
        storage = chelis::owner_block_alloc(static_cast<size_t>(bytes));
        if (!storage) hip_must(hipErrorOutOfMemory, "hipMalloc");
        const hipStream_t st = library_stream();
        hip_must(hipMemsetAsync(storage, 0, static_cast<size_t>(bytes), st), "hipMemsetAsync");
        hip_must(hipStreamSynchronize(st), "hipStreamSynchronize");
    }
    return make_owner(plan, storage, true, bytes, device);
}

chelis_device_tensor_owner *borrow(chelis_metadata_plan *plan, void *data, chelis_scalar capacity) {
    chelis_metadata_plan_check_capacity(plan, capacity);  // traps unless capacity is an i64 >= the span
    require_device_storage(plan, data);
    return make_owner(plan, data, false, static_cast<int64_t>(capacity.bits), device_now());
}

}  // namespace

// ======================================================================= ABI
extern "C" chelis_device_tensor_owner *chelis_device_tensor_alloc(chelis_metadata_plan *plan) {
    return at_boundary([&] { return allocate(plan); });
}

extern "C" chelis_device_tensor_owner *chelis_device_tensor_borrow(chelis_metadata_plan *plan, void *data,
                                                                   chelis_scalar byte_capacity) {
    return at_boundary([&] { return borrow(plan, data, byte_capacity); });
}

extern "C" chelis_device_tensor_owner *chelis_device_tensor_import(const chelis_gpu_tensor *packet) {
    return at_boundary([&] {
        if (packet == nullptr || reinterpret_cast<uintptr_t>(packet) % alignof(chelis_gpu_tensor) != 0)
            trap(Trap::Domain);
        const chelis_gpu_tensor p = *packet;
        if (p.ownership != 0 || p.reserved[0] != 0 || p.reserved[1] != 0) trap(Trap::Domain);
        preflight(p.rank, p.shape);
        preflight(p.rank, p.strides);
        std::vector<chelis_scalar> dims = tagged_i64(p.rank, p.shape), steps = tagged_i64(p.rank, p.strides);
        chelis_metadata_plan *plan =
            chelis_metadata_plan_view(i64(p.rank), dims.empty() ? nullptr : dims.data(),
                                      steps.empty() ? nullptr : steps.data(), dtype_request(p.dtype), i64(p.byte_capacity));
        if (chelis_metadata_plan_count(plan) != p.count) trap(Trap::Domain);
        return borrow(plan, p.data, i64(p.byte_capacity));
    });
}

extern "C" const chelis_gpu_tensor *chelis_device_tensor_view(const chelis_device_tensor_owner *owner) {
    return &checked_here(owner).packet;
}

extern "C" int32_t chelis_device_tensor_device(const chelis_device_tensor_owner *owner) {
    return checked(owner).device;
}

extern "C" chelis_device_tensor_owner *chelis_device_tensor_clone(const chelis_device_tensor_owner *source) {
    return at_boundary([&] {
        const chelis_device_tensor_owner &src = checked_here(source);
        // the dense result plan is checked (and its storage zero-filled)
        // before any byte moves, also for an empty source view
        chelis_device_tensor_owner *copy = allocate(dense_plan_like(src.plan));
        if (src.packet.count != 0) {
            const hipStream_t st = library_stream();
            copy_view_to_dense(src, copy->storage, st);
            hip_must(hipStreamSynchronize(st), "hipStreamSynchronize");
        }
        return copy;
    });
}

extern "C" void chelis_device_tensor_release(chelis_device_tensor_owner *owner) {
    at_boundary([&] {
        checked(owner);
        destroy_owner(owner);
        return 0;
    });
}

extern "C" void chelis_device_tensor_copy_from_host(chelis_device_tensor_owner *destination,
                                                    const chelis_tensor *source) {
    at_boundary([&] {
        const chelis_device_tensor_owner &dst = checked_here(destination);
        const chelis_read_view host = chelis_tensor_read_view(source);
        require_same_elements(host, dst.packet);
        // only owned dense storage takes host bytes
        if (!dst.owns_storage || !is_dense(dst.plan)) trap(Trap::Domain);
        const int64_t bytes = chelis_metadata_plan_byte_count(dst.plan);
        if (bytes > 0) {
            const hipStream_t st = library_stream();
            hip_must(hipMemcpyAsync(dst.storage, host.data, static_cast<size_t>(bytes), hipMemcpyHostToDevice, st),
                     "hipMemcpyAsync");
            hip_must(hipStreamSynchronize(st), "hipStreamSynchronize");
        }
        return 0;
    });
}

extern "C" void chelis_device_tensor_copy_to_host(chelis_tensor_write *destination,
                                                  const chelis_device_tensor_owner *source) {
    at_boundary([&] {
        const chelis_device_tensor_owner &src = checked_here(source);
        const chelis_write_view host = chelis_tensor_write_view(destination);
        require_same_elements(host, src.packet);
        if (src.packet.count == 0) return 0;
        const int64_t bytes = chelis_metadata_plan_byte_count(src.plan);
        const hipStream_t st = library_stream();
        if (is_dense(src.plan)) {
            hip_must(hipMemcpyAsync(host.data, src.storage, static_cast<size_t>(bytes), hipMemcpyDeviceToHost, st),
                     "hipMemcpyAsync");
        } else {
            void *staging = chelis::scratch_alloc(static_cast<size_t>(bytes));
            if (!staging) hip_must(hipErrorOutOfMemory, "staging for a strided copy");
            copy_view_to_dense(src, staging, st);
            hip_must(hipMemcpyAsync(host.data, staging, static_cast<size_t>(bytes), hipMemcpyDeviceToHost, st),
                     "hipMemcpyAsync");
            chelis::scratch_free(staging, static_cast<size_t>(bytes));
        }
        hip_must(hipStreamSynchronize(st), "hipStreamSynchronize");
        return 0;
    });
}
