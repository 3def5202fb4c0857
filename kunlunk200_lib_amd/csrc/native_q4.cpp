// Native Q4 layout and API (reference src/q4-layout.cpp:7-45,
// src/k200.cpp:546-617): layout size and host repack, the reference's
// argument rules and accelerated-route predicate, and the exact GEMV over the
// layout (kk_native_q4_gemv). Every call completes before returning.
#include "launch.h"
#include "runtime_internal.h"

#include <climits>
#include <cstdint>
#include <cstring>
#include <vector>

namespace kunlun {

bool native_q4_layout_supported(int k, int n) {
    return k > 0 && k <= 16384 && k % 32 == 0 && n > 0 && n <= 90000000 / k;
}

size_t native_q4_size(int k, int n) {
    if (!native_q4_layout_supported(k, n)) return 0;
    const size_t rows = ((size_t)n + 31) & ~(size_t)31;
    return aligned(rows * k / 2) + aligned(rows * (k / 32) * 2);
}

bool pack_native_q4(void * destination, size_t bytes, const void * q4, int k, int n) {
    const size_t need = native_q4_size(k, n);
    if (!need || bytes < need || !destination || !q4) return false;
    const uintptr_t dst = (uintptr_t)destination, src = (uintptr_t)q4;
    const int blocks = k / 32;
    const size_t source_bytes = (size_t)n * blocks * 18;
    if (dst + need < dst || src + source_bytes < src) return false;
    if (!(dst + need <= src || src + source_bytes <= dst)) return false;
    uint8_t * out = static_cast<uint8_t *>(destination);
    const uint8_t * in = static_cast<const uint8_t *>(q4);
    const size_t rows = ((size_t)n + 31) & ~(size_t)31;
    uint8_t * scales = out + aligned(rows * k / 2);
    std::memset(out, 0, need);
    for (int row = 0; row < n; ++row) {
        const int lane = row % 32;
        for (int b = 0; b < blocks; ++b) {
            const uint8_t * block = in + ((size_t)row * blocks + b) * 18;
            const size_t tile_block = (size_t)(row / 32) * blocks + b;
            std::memcpy(scales + (tile_block * 32 + lane) * 2, block, 2);
            // Q4_0 byte i holds K i (low nibble) and K 16+i (high), offset by
            // 8; pair byte j holds K 2j (low) and 2j+1 (high) as signed nibbles.
            uint8_t * tile = out + tile_block * 512 + lane;
            for (int j = 0; j < 8; ++j) {
                const uint32_t lo = block[2 + 2 * j] & 15u, hi = block[3 + 2 * j] & 15u;
                tile[j * 32] = (uint8_t)((lo ^ 8u) | ((hi ^ 8u) << 4));
            }
            for (int j = 8; j < 16; ++j) {
                const uint32_t lo = block[2 + 2 * j - 16] >> 4, hi = block[3 + 2 * j - 16] >> 4;
                tile[j * 32] = (uint8_t)((lo ^ 8u) | ((hi ^ 8u) << 4));
            }
        }
    }
    return true;
}

void upload_native_q4(int device, void * weights, const void * q4, int k, int n) {
    std::lock_guard<std::recursive_mutex> lock(runtime_mutex());
    std::vector<uint8_t> packed(native_q4_size(k, n));
    require(pack_native_q4(packed.data(), packed.size(), q4, k, n));
    select(device);
    check(copy(weights, packed.data(), packed.size(), host_to_device));
    check(wait());
}

const char * native_q4_reason(int k, int n, int batch, InputType type) {
    if (!native_q4_layout_supported(k, n)) return "K/N/layout capacity";
    if (type != InputType::f32 && type != InputType::f16) return "input type";
    if (batch != 1) return "batch != 1";
    if (n % 128) return "rows not divisible by 128 (N64 requires 256)";
    if ((size_t)n * (k / 32) * 4 > 16 * 1024 * 1024) return "partial capacity";
    return "";
}

struct NativeQ4Workspace::Impl {
    int id = -1;
    size_t accelerated = 0, fallback = 0;
};

NativeQ4Workspace::NativeQ4Workspace() : impl_(new Impl{}) {}

NativeQ4Workspace::~NativeQ4Workspace() {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    delete impl_;
}

NativeQ4Statistics NativeQ4Workspace::statistics() const {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    return {impl_->accelerated, impl_->fallback, 0, 0};
}

bool native_q4_matmul(NativeQ4Workspace & workspace, int id, void * y, const void * weights, const void * input,
                      int k, int n, int batch, InputType type) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    require(id >= 0 && id < max_devices && native_q4_layout_supported(k, n));
    require(type == InputType::f32 || type == InputType::f16);
    require(batch > 0 && (size_t)n * batch <= INT_MAX / 4 && (size_t)k * batch <= INT_MAX / 4);
    require(y && weights && input);
    const int x_bytes = type == InputType::f16 ? 2 : 4;
    const uintptr_t yp = (uintptr_t)y, wp = (uintptr_t)weights, xp = (uintptr_t)input;
    const size_t ys = (size_t)n * batch * 4, ws = native_q4_size(k, n), xs = (size_t)k * batch * x_bytes;
    require(yp % 4 == 0 && wp % 256 == 0 && xp % x_bytes == 0);
    require(yp + ys >= yp && wp + ws >= wp && xp + xs >= xp);
    require((yp + ys <= wp || wp + ws <= yp) && (yp + ys <= xp || xp + xs <= yp) && (wp + ws <= xp || xp + xs <= wp));
    NativeQ4Workspace::Impl & s = *workspace.impl_;
    require(s.id == -1 || s.id == id);
    detail::DeviceContext & ctx = detail::context(id);
    s.id = id;
    const bool accelerated = !*native_q4_reason(k, n, batch, type) && ((yp | xp) & 63) == 0;
    detail::check_hip((hipError_t)kk_native_q4_gemv(weights, input, type == InputType::f16 ? 1 : 0,
                                                    static_cast<float *>(y), k, n, batch, ctx.stream),
                      "kk_native_q4_gemv");
    detail::check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    if (accelerated) ++s.accelerated;
    else ++s.fallback;
    detail::count_matmul(id);
    detail::note_route("native_q4_gemv");
    return accelerated;
}

} // namespace kunlun
