// Library context: one HIP stream per device, the last error of the calling
// thread, and packet validation shared by every launcher.
//
// The reference launches on stream 0 and looks up device properties and
// kernel functions on every launch (runtime/chelis_hip_runtime.h:455-485);
// here the stream is created once per device (default priority, non-blocking)
// and kernels are compiled into this library, so a launch is one
// hipLaunchKernel on that stream.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "hip_common.h"

namespace chelis {

namespace {
thread_local char g_error[512] = "";
std::mutex g_stream_mutex;
constexpr int kMaxDevices = 64;
hipStream_t g_streams[kMaxDevices] = {};
int g_cus[kMaxDevices] = {};
}  // namespace

int32_t set_error(int32_t status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_error, sizeof g_error, fmt, ap);
    va_end(ap);
    return status;
}

hipStream_t stream() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_stream_mutex);
    if (!g_streams[device]) {
        hipStream_t s = nullptr;
        if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
        g_streams[device] = s;
    }
    return g_streams[device];
}

// ---- stream-ordered scratch ---------------------------------------------
// Every launcher of a device enqueues on that device's one library stream,
// so a block handed back by scratch_free() may be handed out again at once:
// whoever gets it next enqueues its kernels on the same stream, after the
// kernels that used the block before. Blocks are cached per device in
// power-of-two size classes (at least 256 B) and kept until the process
// ends; only a cache miss allocates (hipMalloc).
namespace {
std::mutex g_scratch_mutex;
constexpr int kClasses = 48;
std::vector<void *> g_free[kMaxDevices][kClasses];

int size_class(size_t bytes) {
    int c = 8;  // 256 B
    while (c < kClasses - 1 && (size_t(1) << c) < bytes) ++c;
    return c;
}
}  // namespace

namespace {
std::atomic<int64_t> g_scratch_requests{0}, g_device_allocations{0};
}  // namespace

hipError_t device_malloc(void **p, size_t bytes) {
    g_device_allocations.fetch_add(1, std::memory_order_relaxed);
    return hipMalloc(p, bytes);
}

void *scratch_alloc(size_t bytes) {
    if (!bytes) return nullptr;
    g_scratch_requests.fetch_add(1, std::memory_order_relaxed);
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return nullptr;
    const int c = size_class(bytes);
    if ((size_t(1) << c) < bytes) return nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        std::vector<void *> &fl = g_free[device][c];
        if (!fl.empty()) {
            void *p = fl.back();
            fl.pop_back();
            return p;
        }
    }
    void *p = nullptr;
    if (device_malloc(&p, size_t(1) << c) != hipSuccess) return nullptr;
    return p;
}

void scratch_free(void *p, size_t bytes) {
    if (!p) return;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    g_free[device][size_class(bytes)].push_back(p);
}

// ---- owner storage ---------------------------------------------------------
// chelis_device_tensor_alloc's blocks come from the same per-device size
// classes, up to kOwnerCacheMax bytes (larger ones are allocated and freed
// directly), so an entry that allocates its outputs on every call reuses
// the blocks earlier calls released instead of paying hipMalloc and hipFree
// (hipFree waits for the whole device). A released block waits for the
// device before it returns to the cache, as hipFree would, so no queued use
// on any stream outlives it.
namespace {
constexpr size_t kOwnerCacheMax = size_t(1) << 28;
}  // namespace

void *owner_block_alloc(size_t bytes) {
    if (!bytes) return nullptr;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return nullptr;
    void *p = nullptr;
    if (bytes > kOwnerCacheMax) return device_malloc(&p, bytes) == hipSuccess ? p : nullptr;
    const int c = size_class(bytes);
    {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        std::vector<void *> &fl = g_free[device][c];
        if (!fl.empty()) {
            p = fl.back();
            fl.pop_back();
            return p;
        }
    }
    return device_malloc(&p, size_t(1) << c) == hipSuccess ? p : nullptr;
}

hipError_t owner_block_free(void *p, size_t bytes) {
    if (!p) return hipSuccess;
    if (bytes > kOwnerCacheMax) return hipFree(p);
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    g_free[device][size_class(bytes)].push_back(p);
    return hipSuccess;
}

// ---- status words ---------------------------------------------------------
// Two int32 words per device, allocated and cleared once, kept until the
// process ends: word 0 carries the error code of a launcher that returns it
// synchronously, word 1 is the trap channel that launchers enqueued without
// waiting record into (OR of codes) until chelis_hip_trap_status reads and
// clears it. The host side of both reads is one pinned word per device.
namespace {
std::mutex g_status_mutex;
int32_t *g_status[kMaxDevices] = {};
int32_t *g_status_host[kMaxDevices] = {};
}  // namespace

int32_t *status_words(int32_t **host) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_status_mutex);
    if (!g_status[device]) {
        int32_t *d = nullptr, *h = nullptr;
        if (device_malloc(reinterpret_cast<void **>(&d), 256) != hipSuccess) return nullptr;
        if (hipMemset(d, 0, 256) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
            hipHostMalloc(&h, sizeof(int32_t), hipHostMallocDefault) != hipSuccess) {
            (void)hipFree(d);
            return nullptr;
        }
        g_status[device] = d;
        g_status_host[device] = h;
    }
    if (host) *host = g_status_host[device];
    return g_status[device];
}

int device_cus() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return 0;
    std::lock_guard<std::mutex> lock(g_stream_mutex);
    if (!g_cus[device]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
        g_cus[device] = n;
    }
    return g_cus[device];
}

int32_t check_tensor(const chelis_gpu_tensor *t, const char *name) {
    if (!t) return set_error(CHELIS_HIP_EDOMAIN, "%s: null tensor packet", name);
    if (t->rank < 0 || t->rank > 8) return set_error(CHELIS_HIP_EDOMAIN, "%s: rank %d outside 0..8", name, t->rank);
    if (t->rank > 0 && (!t->shape || !t->strides))
        return set_error(CHELIS_HIP_EDOMAIN, "%s: null shape or strides", name);
    if (t->reserved[0] || t->reserved[1]) return set_error(CHELIS_HIP_EDOMAIN, "%s: reserved bytes set", name);
    int64_t width = dtype_width(t->dtype);
    if (!width) return set_error(CHELIS_HIP_EDOMAIN, "%s: unknown dtype %d", name, (int)t->dtype);
    int64_t count = 1, span = 0;
    for (int32_t a = 0; a < t->rank; ++a) {
        if (t->shape[a] < 0 || t->strides[a] < 0)
            return set_error(CHELIS_HIP_EDOMAIN, "%s: negative extent or stride on axis %d", name, a);
        if (__builtin_mul_overflow(count, t->shape[a], &count))
            return set_error(CHELIS_HIP_EDOMAIN, "%s: element count overflows i64", name);
    }
    if (count != t->count) return set_error(CHELIS_HIP_EDOMAIN, "%s: count %lld != product of shape %lld", name,
                                            (long long)t->count, (long long)count);
    if (count) {
        for (int32_t a = 0; a < t->rank; ++a) {
            int64_t part;
            if (__builtin_mul_overflow(t->shape[a] - 1, t->strides[a], &part) ||
                __builtin_add_overflow(span, part, &span))
                return set_error(CHELIS_HIP_EDOMAIN, "%s: view span overflows i64", name);
        }
        int64_t bytes;
        if (__builtin_add_overflow(span, 1, &span) || __builtin_mul_overflow(span, width, &bytes) ||
            bytes > t->byte_capacity)
            return set_error(CHELIS_HIP_EDOMAIN, "%s: view reaches past byte_capacity %lld", name,
                             (long long)t->byte_capacity);
        if (!t->data) return set_error(CHELIS_HIP_EDOMAIN, "%s: null data", name);
        if (reinterpret_cast<uintptr_t>(t->data) % (uintptr_t)width)
            return set_error(CHELIS_HIP_EDOMAIN, "%s: data not aligned to its dtype", name);
    }
    return CHELIS_HIP_OK;
}

bool is_contiguous(const chelis_gpu_tensor *t) {
    for (int32_t a = 0; a < t->rank; ++a)
        if (t->shape[a] == 0) return true;  // no element: any strides hold it
    int64_t expect = 1;
    for (int32_t a = t->rank; a-- > 0;) {
        if (t->shape[a] != 1 && t->strides[a] != expect) return false;
        expect *= t->shape[a];
    }
    return true;
}

bool same_shape(const chelis_gpu_tensor *a, const chelis_gpu_tensor *b) {
    if (a->rank != b->rank) return false;
    for (int32_t i = 0; i < a->rank; ++i)
        if (a->shape[i] != b->shape[i]) return false;
    return true;
}

bool row_view(const chelis_gpu_tensor *t, RowView *v) {
    if (t->rank == 0) {
        v->rows = 1;
        v->n = 1;
        v->ld = 1;
        return true;
    }
    v->n = t->shape[t->rank - 1];
    if (v->n > 1 && t->strides[t->rank - 1] != 1) return false;
    v->rows = 1;
    for (int32_t a = 0; a < t->rank - 1; ++a) v->rows *= t->shape[a];
    // Leading axes must collapse to one uniform row stride.
    int64_t ld = -1, expect = -1;
    for (int32_t a = t->rank - 1; a-- > 0;) {
        if (t->shape[a] == 1) continue;
        if (ld < 0) {
            ld = t->strides[a];
            expect = ld * t->shape[a];
        } else {
            if (t->strides[a] != expect) return false;
            expect *= t->shape[a];
        }
    }
    v->ld = ld < 0 ? v->n : ld;
    return true;
}

namespace {
std::atomic<int32_t> g_exact_mode{0};
thread_local int32_t t_pinned = -1;  // the mode a scope pinned for this thread, -1 none
}  // namespace

bool exact_mode() {
    return t_pinned >= 0 ? t_pinned != 0 : g_exact_mode.load(std::memory_order_relaxed) != 0;
}

ModeScope::ModeScope(int32_t mode) : prev_(t_pinned) {
    if (mode >= 0) t_pinned = mode != 0;
    else if (t_pinned < 0) t_pinned = g_exact_mode.load(std::memory_order_relaxed) != 0;
}

ModeScope::~ModeScope() { t_pinned = prev_; }

}  // namespace chelis

extern "C" {

const char *chelis_hip_last_error(void) { return chelis::g_error; }

int32_t chelis_hip_set_exact(int32_t on) { return chelis::g_exact_mode.exchange(on ? 1 : 0); }

int32_t chelis_hip_set_exact_matmul(int32_t on) { return chelis_hip_set_exact(on); }

void *chelis_hip_stream(void) { return (void *)chelis::stream(); }

int32_t chelis_hip_synchronize(void) {
    hipStream_t s = chelis::stream();
    if (!s) return chelis::set_error(CHELIS_HIP_EHIP, "no HIP device");
    CHELIS_HIP_TRY(hipStreamSynchronize(s));
    return CHELIS_HIP_OK;
}

const char *chelis_hip_build_info(void) {
#ifdef CHELIS_BUILD_ID
    return "gfx950 " CHELIS_BUILD_ID;
#else
    return "gfx950";
#endif
}

}  // extern "C"

extern "C" void chelis_hip_allocation_counts(int64_t *scratch_requests, int64_t *device_allocations) {
    if (scratch_requests) *scratch_requests = chelis::g_scratch_requests.load(std::memory_order_relaxed);
    if (device_allocations) *device_allocations = chelis::g_device_allocations.load(std::memory_order_relaxed);
}
