// Opaque device tensor owner (include/chelis_device_owner.h).
//
// Same contract as crates/chelis-backend-hip/runtime/chelis_device_owner.cpp:
// the owner retains its metadata plan, owns or borrows the storage, checks
// the current device on every observation, never lets a C++ exception cross
// the ABI, and traps `domain` / `overflow` on invalid input. The MI355X
// differences are inside: clone and strided copies are one gather kernel on
// the library stream (the reference issues one hipMemcpy per element,
// chelis_device_owner.cpp:213-233,254-273), contiguous copies are one
// hipMemcpyAsync, and allocation zero-fills with hipMemsetAsync on the
// library stream followed by one stream synchronize.
#include "chelis_device_owner.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <exception>
#include <memory>
#include <new>
#include <utility>
#include <vector>

#include "hip_common.h"

namespace {

[[noreturn]] void domain() {
    chelis_numeric_trap("numeric trap: domain in metadata_plan at i64");
    std::abort();
}
void hip_checked(hipError_t status) {
    if (status != hipSuccess) {
        std::fprintf(stderr, "HIP device owner failure: %s\n", hipGetErrorString(status));
        std::abort();
    }
}
void chelis_checked(int32_t status) {
    if (status != CHELIS_HIP_OK) {
        std::fprintf(stderr, "HIP device owner failure: %s\n", chelis_hip_last_error());
        std::abort();
    }
}
int32_t current_device() {
    int device = -1;
    hip_checked(hipGetDevice(&device));
    if (device < 0) domain();
    return device;
}
hipStream_t lib_stream() {
    hipStream_t s = chelis::stream();
    if (!s) {
        std::fprintf(stderr, "HIP device owner failure: no stream\n");
        std::abort();
    }
    return s;
}

class DeviceScope final {
public:
    explicit DeviceScope(int32_t device) : previous_(current_device()) {
        if (previous_ != device) hip_checked(hipSetDevice(device));
    }
    ~DeviceScope() {
        if (current_device() != previous_) hip_checked(hipSetDevice(previous_));
    }
    DeviceScope(const DeviceScope &) = delete;
    DeviceScope &operator=(const DeviceScope &) = delete;

private:
    const int32_t previous_;
};

struct PlanRelease {
    void operator()(chelis_metadata_plan *plan) const {
        if (plan) chelis_metadata_plan_release(plan);
    }
};
using Plan = std::unique_ptr<chelis_metadata_plan, PlanRelease>;

struct DeviceRelease {
    int32_t device = 0;
    void operator()(void *data) const {
        if (data) {
            DeviceScope scope(device);
            hip_checked(hipFree(data));
        }
    }
};
using Allocation = std::unique_ptr<void, DeviceRelease>;

chelis_scalar integer(int64_t value) { return chelis_scalar_from_bits(CHELIS_DTYPE_I64, static_cast<uint64_t>(value)); }
chelis_scalar exemplar(chelis_dtype dtype) { return chelis_scalar{dtype, {0, 0, 0, 0, 0, 0, 0}, 0}; }

std::vector<chelis_scalar> tagged(int32_t rank, const int64_t *values) {
    if (rank < 0) domain();
    if (rank > 0 && (!values || reinterpret_cast<uintptr_t>(values) % alignof(int64_t))) domain();
    std::vector<chelis_scalar> out;
    out.reserve(static_cast<size_t>(rank));
    for (int32_t a = 0; a < rank; ++a) out.push_back(integer(values[a]));
    return out;
}

Plan canonical_plan(const chelis_metadata_plan *source) {
    auto rank = chelis_metadata_plan_rank(source);
    auto shape = tagged(rank, chelis_metadata_plan_shape(source));
    return Plan(chelis_metadata_plan_new(integer(rank), shape.data(), exemplar(chelis_metadata_plan_dtype(source))));
}

bool canonical_strides(const chelis_metadata_plan *plan) {
    auto canon = canonical_plan(plan);
    auto rank = chelis_metadata_plan_rank(plan);
    auto l = chelis_metadata_plan_strides(plan);
    auto r = chelis_metadata_plan_strides(canon.get());
    for (int32_t a = 0; a < rank; ++a)
        if (l[a] != r[a]) return false;
    return true;
}

void validate_data(const chelis_metadata_plan *plan, const void *data) {
    auto count = chelis_metadata_plan_count(plan);
    if (!count) return;
    auto width = chelis_metadata_plan_byte_count(plan) / count;
    if (!data || reinterpret_cast<uintptr_t>(data) % static_cast<uintptr_t>(width)) domain();
    hipPointerAttribute_t attributes{};
    if (hipPointerGetAttributes(&attributes, data) != hipSuccess || attributes.type != hipMemoryTypeDevice ||
        attributes.device != current_device())
        domain();
}

template <class Operation>
auto guarded(Operation operation) -> decltype(operation()) {
    try {
        return operation();
    } catch (const std::exception &error) {
        std::fprintf(stderr, "device metadata allocation failed: %s\n", error.what());
        std::abort();
    }
}

}  // namespace

struct chelis_device_tensor_owner final {
    chelis_device_tensor_owner(Plan plan, Allocation allocation, bool borrowed, void *data, int64_t capacity,
                               int32_t device)
        : plan_(std::move(plan)),
          allocation_(std::move(allocation)),
          borrowed_(borrowed),
          device_(device),
          packet_{data,
                  chelis_metadata_plan_shape(plan_.get()),
                  chelis_metadata_plan_strides(plan_.get()),
                  chelis_metadata_plan_count(plan_.get()),
                  capacity,
                  chelis_metadata_plan_rank(plan_.get()),
                  chelis_metadata_plan_dtype(plan_.get()),
                  static_cast<uint8_t>(borrowed ? 0 : 1),
                  {0, 0}} {}
    chelis_device_tensor_owner(const chelis_device_tensor_owner &) = delete;
    chelis_device_tensor_owner &operator=(const chelis_device_tensor_owner &) = delete;
    const chelis_gpu_tensor *view() const { return &packet_; }
    const chelis_metadata_plan *plan() const { return plan_.get(); }
    bool owns_storage() const { return !borrowed_; }
    int32_t device() const { return device_; }
    void require_current() const {
        if (current_device() != device_) domain();
    }

private:
    Plan plan_;
    Allocation allocation_;
    const bool borrowed_;
    const int32_t device_;
    const chelis_gpu_tensor packet_;
};

namespace {

const chelis_device_tensor_owner &owner(const chelis_device_tensor_owner *value) {
    if (!value || reinterpret_cast<uintptr_t>(value) % alignof(chelis_device_tensor_owner)) domain();
    return *value;
}

chelis_device_tensor_owner *borrow_plan(Plan plan, void *data, chelis_scalar capacity) {
    chelis_metadata_plan_check_capacity(plan.get(), capacity);
    validate_data(plan.get(), data);
    auto bytes = static_cast<int64_t>(capacity.bits);
    return new chelis_device_tensor_owner(std::move(plan), Allocation{}, true, data, bytes, current_device());
}

chelis_device_tensor_owner *allocate_plan(Plan plan) {
    auto bytes = chelis_metadata_plan_byte_count(plan.get());
    chelis_metadata_plan_check_capacity(plan.get(), integer(bytes));
    auto device = current_device();
    void *data = nullptr;
    if (bytes) hip_checked(hipMalloc(&data, static_cast<size_t>(bytes)));
    Allocation allocation(data, DeviceRelease{device});
    if (bytes) {
        hipStream_t st = lib_stream();
        hip_checked(hipMemsetAsync(data, 0, static_cast<size_t>(bytes), st));
        hip_checked(hipStreamSynchronize(st));
    }
    return new chelis_device_tensor_owner(std::move(plan), std::move(allocation), false, data, bytes, device);
}

void require_matching(const chelis_read_view &host, const chelis_gpu_tensor &device) {
    if (host.count != device.count || host.dtype != device.dtype) domain();
    for (auto byte : host.reserved)
        if (byte) domain();
}
void require_matching(const chelis_write_view &host, const chelis_gpu_tensor &device) {
    if (host.count != device.count || host.dtype != device.dtype) domain();
    for (auto byte : host.reserved)
        if (byte) domain();
}

}  // namespace

extern "C" chelis_device_tensor_owner *chelis_device_tensor_alloc(chelis_metadata_plan *plan) {
    return guarded([&] { return allocate_plan(Plan(plan)); });
}

extern "C" chelis_device_tensor_owner *chelis_device_tensor_borrow(chelis_metadata_plan *plan, void *data,
                                                                   chelis_scalar byte_capacity) {
    return guarded([&] { return borrow_plan(Plan(plan), data, byte_capacity); });
}

extern "C" chelis_device_tensor_owner *chelis_device_tensor_import(const chelis_gpu_tensor *packet) {
    return guarded([&] {
        if (!packet || reinterpret_cast<uintptr_t>(packet) % alignof(chelis_gpu_tensor)) domain();
        if (packet->ownership != 0 || packet->reserved[0] || packet->reserved[1]) domain();
        auto shape = tagged(packet->rank, packet->shape);
        auto strides = tagged(packet->rank, packet->strides);
        Plan plan(chelis_metadata_plan_view(integer(packet->rank), shape.data(), strides.data(),
                                            exemplar(packet->dtype), integer(packet->byte_capacity)));
        if (packet->count != chelis_metadata_plan_count(plan.get())) domain();
        return borrow_plan(std::move(plan), packet->data, integer(packet->byte_capacity));
    });
}

extern "C" const chelis_gpu_tensor *chelis_device_tensor_view(const chelis_device_tensor_owner *value) {
    owner(value).require_current();
    return owner(value).view();
}

extern "C" int32_t chelis_device_tensor_device(const chelis_device_tensor_owner *value) { return owner(value).device(); }

extern "C" chelis_device_tensor_owner *chelis_device_tensor_clone(const chelis_device_tensor_owner *source) {
    return guarded([&] {
        auto &input = owner(source);
        input.require_current();
        std::unique_ptr<chelis_device_tensor_owner> result(allocate_plan(canonical_plan(input.plan())));
        const chelis_gpu_tensor *v = input.view();
        if (v->count) {
            hipStream_t st = lib_stream();
            const int64_t width = chelis_metadata_plan_byte_count(input.plan()) / v->count;
            if (canonical_strides(input.plan())) {
                hip_checked(hipMemcpyAsync(result->view()->data, v->data,
                                           static_cast<size_t>(chelis_metadata_plan_byte_count(input.plan())),
                                           hipMemcpyDeviceToDevice, st));
            } else {
                chelis_checked(chelis::gather_contiguous(v->data, result->view()->data, v->rank, v->shape, v->strides,
                                                         width, v->count, st));
            }
            hip_checked(hipStreamSynchronize(st));
        }
        return result.release();
    });
}

extern "C" void chelis_device_tensor_release(chelis_device_tensor_owner *value) {
    owner(value);
    delete value;
}

extern "C" void chelis_device_tensor_copy_from_host(chelis_device_tensor_owner *destination,
                                                    const chelis_tensor *source) {
    guarded([&] {
        auto &output = owner(destination);
        output.require_current();
        auto input = chelis_tensor_read_view(source);
        require_matching(input, *output.view());
        if (!output.owns_storage() || !canonical_strides(output.plan())) domain();
        auto bytes = chelis_metadata_plan_byte_count(output.plan());
        if (bytes) {
            hipStream_t st = lib_stream();
            hip_checked(hipMemcpyAsync(output.view()->data, input.data, static_cast<size_t>(bytes),
                                       hipMemcpyHostToDevice, st));
            hip_checked(hipStreamSynchronize(st));
        }
        return 0;
    });
}

extern "C" void chelis_device_tensor_copy_to_host(chelis_tensor_write *destination,
                                                  const chelis_device_tensor_owner *source) {
    guarded([&] {
        auto &input = owner(source);
        input.require_current();
        auto output = chelis_tensor_write_view(destination);
        require_matching(output, *input.view());
        const chelis_gpu_tensor *v = input.view();
        if (!v->count) return 0;
        hipStream_t st = lib_stream();
        const int64_t bytes = chelis_metadata_plan_byte_count(input.plan());
        if (canonical_strides(input.plan())) {
            hip_checked(hipMemcpyAsync(output.data, v->data, static_cast<size_t>(bytes), hipMemcpyDeviceToHost, st));
        } else {
            void *staging = nullptr;
            hip_checked(hipMallocAsync(&staging, static_cast<size_t>(bytes), st));
            chelis_checked(chelis::gather_contiguous(v->data, staging, v->rank, v->shape, v->strides, bytes / v->count,
                                                     v->count, st));
            hip_checked(hipMemcpyAsync(output.data, staging, static_cast<size_t>(bytes), hipMemcpyDeviceToHost, st));
            hip_checked(hipFreeAsync(staging, st));
        }
        hip_checked(hipStreamSynchronize(st));
        return 0;
    });
}
