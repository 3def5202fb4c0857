// Host runtime of the KunlunK200 surface over HIP: device selection, the
// process-wide lock, fail-fast checks, copies, allocation accounting, the
// rowwise INT8 weight upload and statistics.
//
// Reference behaviour restated here: src/k200.cpp:25-123 and :633-634.
// Differences of substance:
//   * a device is one HIP device, valid ids [0, min(hipGetDeviceCount, 8));
//   * each device has one library-owned HIP stream (default flags and
//     priority); matmul submits to it and wait() synchronizes it;
//   * copies that touch host memory complete before copy() returns.
#include "runtime_internal.h"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace kunlun {
namespace detail {
namespace {

std::recursive_mutex global_mutex;
std::atomic<size_t> allocated[max_devices];
std::atomic<size_t> matmuls[max_devices];
std::atomic<size_t> peer_copies{0}, peer_bytes{0};
DeviceContext contexts[max_devices];

thread_local int diagnostic_device = -1;
thread_local const char * diagnostic_name = nullptr;
thread_local int64_t diagnostic_shape[4] = {};

void diagnostic_print() {
    std::fprintf(stderr, "Kunlun context: device=%d tensor=%s shape=[%lld,%lld,%lld,%lld]\n", diagnostic_device,
                 diagnostic_name ? diagnostic_name : "<outside graph>", (long long)diagnostic_shape[0],
                 (long long)diagnostic_shape[1], (long long)diagnostic_shape[2], (long long)diagnostic_shape[3]);
    std::fflush(stderr);
}

int visible_devices() {
    static int count = -1;
    if (count < 0) {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void)hipGetLastError();
            n = 0;
        }
        count = std::min(n, max_devices);
    }
    return count;
}

} // namespace

std::recursive_mutex & mutex() { return global_mutex; }

[[noreturn]] void fail(const char * message) {
    diagnostic_print();
    std::fprintf(stderr, "Kunlun %s\n", message);
    std::fflush(stderr);
    std::abort();
}

void check_hip(hipError_t status, const char * what) {
    if (status != hipSuccess) {
        std::fprintf(stderr, "Kunlun failure: api=%s status=%d (%s)\n", what, (int)status, hipGetErrorString(status));
        kunlun::check((int)status);
    }
}

int current_device() {
    int device = 0;
    check_hip(hipGetDevice(&device), "hipGetDevice");
    return device;
}

DeviceContext & context(int device) {
    std::lock_guard<std::recursive_mutex> lock(global_mutex);
    select(device);
    DeviceContext & ctx = contexts[device];
    if (!ctx.ready) {
        check_hip(hipStreamCreate(&ctx.stream), "hipStreamCreate");
        void * word = nullptr;
        check_hip(hipMalloc(&word, 256), "hipMalloc(status)");
        const int zero = 0;
        check_hip(hipMemcpy(word, &zero, sizeof(zero), hipMemcpyHostToDevice), "hipMemcpy(status)");
        ctx.status = static_cast<int *>(word);
        check_hip(hipDeviceGetAttribute(&ctx.cus, hipDeviceAttributeMultiprocessorCount, device),
                  "hipDeviceGetAttribute(multiprocessors)");
        ctx.ready = true;
    }
    return ctx;
}

void count_matmul(int device) { ++matmuls[device]; }
size_t matmul_count(int device) {
    kunlun::require(device >= 0 && device < max_devices);
    return matmuls[device].load();
}

} // namespace detail

std::recursive_mutex & runtime_mutex() { return detail::global_mutex; }

void diagnostic_tensor(const char * name, const int64_t * dimensions) {
    detail::diagnostic_name = name;
    for (int i = 0; i < 4; ++i) detail::diagnostic_shape[i] = dimensions ? dimensions[i] : 0;
}

void check(int status) {
    if (status) {
        detail::diagnostic_print();
        std::fprintf(stderr, "Kunlun runtime error %d\n", status);
        std::fflush(stderr);
        std::abort();
    }
}

void require(bool condition) {
    if (!condition) detail::fail("invalid argument or unavailable resource");
}

int device_count(int * count) {
    std::lock_guard<std::recursive_mutex> lock(detail::global_mutex);
    require(count != nullptr);
    const hipError_t status = hipGetDeviceCount(count);
    if (status == hipSuccess) *count = std::min(*count, max_devices);
    return (int)status;
}

void select(int device) {
    detail::diagnostic_device = device;
    require(device >= 0 && device < detail::visible_devices());
    detail::check_hip(hipSetDevice(device), "hipSetDevice");
}

int wait() {
    std::lock_guard<std::recursive_mutex> lock(detail::global_mutex);
    int device = 0;
    hipError_t status = hipGetDevice(&device);
    if (status != hipSuccess) return (int)status;
    detail::DeviceContext & ctx = detail::contexts[device];
    // Every stream of the device, as the reference's xpu_wait() (reference
    // src/k200.cpp:68): the library's own stream and the caller's HIP work.
    status = hipDeviceSynchronize();
    if (status != hipSuccess || !ctx.ready) return (int)status;
    if (ctx.status_pending) {
        int word = 0;
        status = hipMemcpy(&word, ctx.status, sizeof(word), hipMemcpyDeviceToHost);
        if (status != hipSuccess) return (int)status;
        ctx.status_pending = false;
        if (word != 0) {
            const int zero = 0;
            (void)hipMemcpy(ctx.status, &zero, sizeof(zero), hipMemcpyHostToDevice);
            // The reference rejects non-finite rowwise_i8 activations with
            // require() (reference src/k200.cpp:213); the device reports them here.
            detail::fail("invalid argument or unavailable resource (non-finite rowwise_i8 activation)");
        }
    }
    return (int)hipSuccess;
}

int copy(void * dst, const void * src, size_t bytes, CopyKind kind) {
    require(kind == host_to_device || kind == device_to_host || kind == device_to_device);
    std::lock_guard<std::recursive_mutex> lock(detail::global_mutex);
    const int device = detail::current_device();
    detail::DeviceContext & ctx = detail::context(device);
    const hipMemcpyKind direction = kind == host_to_device   ? hipMemcpyHostToDevice
                                    : kind == device_to_host ? hipMemcpyDeviceToHost
                                                             : hipMemcpyDeviceToDevice;
    // Ordered after the library's submitted work on this device and complete
    // on return in every direction, as the reference's synchronous
    // xpu_memcpy (reference src/k200.cpp:69-75).
    hipError_t status = hipMemcpyAsync(dst, src, bytes, direction, ctx.stream);
    if (status == hipSuccess) status = hipStreamSynchronize(ctx.stream);
    return (int)status;
}

void * allocate(int device, size_t bytes) {
    std::lock_guard<std::recursive_mutex> lock(detail::global_mutex);
    select(device);
    const size_t size = std::max<size_t>(bytes, 256);
    void * ptr = nullptr;
    if (hipMalloc(&ptr, size) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    detail::allocated[device] += size;
    return ptr;
}

void release(int device, void * ptr, size_t bytes) {
    std::lock_guard<std::recursive_mutex> lock(detail::global_mutex);
    if (!ptr) return;
    select(device);
    detail::check_hip(hipFree(ptr), "hipFree");
    detail::allocated[device] -= std::max<size_t>(bytes, 256);
}

size_t allocated_bytes(int device) {
    require(device >= 0 && device < max_devices);
    return detail::allocated[device].load();
}

void peer(int dst_device, void * dst, int src_device, const void * src, size_t bytes) {
    std::lock_guard<std::recursive_mutex> lock(detail::global_mutex);
    select(src_device);
    check(wait());
    detail::DeviceContext & ctx = detail::context(dst_device);
    detail::check_hip(hipMemcpyPeerAsync(dst, dst_device, src, src_device, bytes, ctx.stream), "hipMemcpyPeerAsync");
    check(wait());
    ++detail::peer_copies;
    detail::peer_bytes += bytes;
}

Buffer::Buffer(int device, size_t bytes) : device_(device), bytes_(bytes), ptr_(allocate(device, bytes)) {
    require(ptr_ != nullptr);
}
Buffer::~Buffer() { release(device_, ptr_, bytes_); }

size_t aligned(size_t bytes) {
    require(bytes <= SIZE_MAX - 255);
    return (bytes + 255) & ~size_t(255);
}
size_t packed_i8_size(int k, int rows) {
    require(k > 0 && rows >= 0);
    return aligned((size_t)k * rows) + aligned((size_t)rows * 4) + 256;
}
float * packed_i8_scales(void * weights, int k, int rows) {
    return (float *)((char *)weights + aligned((size_t)k * rows));
}
float * packed_i8_maxima(void * weights, int k, int rows) {
    return (float *)((char *)packed_i8_scales(weights, k, rows) + aligned((size_t)rows * 4));
}

// Host quantizer of the reference (reference src/k200.cpp:102-123): per row
// max|v| (finite required), scale = max/127 (1 for a zero row),
// q = clamp((int)(v*inv +/- 0.5f), -127, 127) with inv = 127/max (0 for a
// zero row); codes, scales and maxima[6] = 127 are copied to the device.
void upload_i8_rows(int device, void * weights, int k, int rows, int first_row, int count, const float * input) {
    std::lock_guard<std::recursive_mutex> lock(detail::global_mutex);
    require(weights && input && k > 0 && rows > 0 && first_row >= 0 && count >= 0 && first_row <= rows &&
            count <= rows - first_row);
    std::vector<int8_t> codes((size_t)count * k);
    std::vector<float> scales(count);
    for (int r = 0; r < count; ++r) {
        const float * row = input + (size_t)r * k;
        float maximum = 0.0f;
        for (int j = 0; j < k; ++j) {
            require(std::isfinite(row[j]));
            maximum = std::max(maximum, std::fabs(row[j]));
        }
        scales[r] = maximum > 0 ? maximum / 127 : 1;
        const float inv = maximum > 0 ? 127 / maximum : 0;
        for (int j = 0; j < k; ++j) {
            const float value = row[j] * inv;
            codes[(size_t)r * k + j] = (int8_t)std::max(-127, std::min(127, (int)(value + (value >= 0 ? .5f : -.5f))));
        }
    }
    const float maxima[6] = {127, 127, 127, 127, 127, 127};
    select(device);
    check(copy((char *)weights + (size_t)first_row * k, codes.data(), codes.size(), host_to_device));
    check(copy(packed_i8_scales(weights, k, rows) + first_row, scales.data(), scales.size() * 4, host_to_device));
    check(copy(packed_i8_maxima(weights, k, rows), maxima, sizeof(maxima), host_to_device));
    check(wait());
}

Statistics statistics() {
    Statistics s{};
    s.matmuls[0] = detail::matmuls[0].load();
    s.matmuls[1] = detail::matmuls[1].load();
    s.peer_copies = detail::peer_copies.load();
    s.peer_bytes = detail::peer_bytes.load();
    return s;
}

const char * version() { return "0.7.12-gfx950"; }

} // namespace kunlun
