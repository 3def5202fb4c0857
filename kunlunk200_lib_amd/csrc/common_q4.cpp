// Common Q4 ABI v1 host side (reference src/q4-common.inc, src/q4-common-pack.h,
// src/q4-activation.inc, src/q4-pair.inc): the persistent layout and its host
// packer, the weight handle, the workspace with its activation storage and
// leases, the reference's argument rules and route choice, and submission of
// the kernels in common_q4.hip. Every call completes before returning.
#include "launch.h"
#include "runtime_internal.h"

#include <algorithm>
#include <chrono>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <vector>

namespace kunlun {

namespace {

constexpr size_t kLeaseLimit = 16u * 1024 * 1024;      // reference q4-activation.inc:50
constexpr size_t kExactRoute = size_t(1) << 27;        // Np * Kp above which M = 1 runs exact

int round_up(int v, int a) { return (v + a - 1) / a * a; }

CommonQ4Info describe(int k, int n, int device) {
    CommonQ4Info a{};
    a.abi_version = 1;
    a.quant_type = 2;
    a.layout = 1;
    a.scale_order = 1;
    a.k = k;
    a.n = n;
    a.kp = round_up(k, k < 512 ? 512 : 256);
    a.np = round_up(n, 256);
    a.device = device;
    a.scale_offset = (size_t)a.kp * a.np / 2;
    a.payload_bytes = a.scale_offset + (size_t)a.kp * a.np / 16;
    return a;
}

bool abi_ok(const CommonQ4Info & a) {
    if (!common_q4_supported(a.k, a.n)) return false;
    const CommonQ4Info e = describe(a.k, a.n, a.device);
    return a.abi_version == 1 && a.quant_type == 2 && a.layout == 1 && a.scale_order == 1 && a.kp == e.kp &&
           a.np == e.np && a.scale_offset == e.scale_offset && a.payload_bytes == e.payload_bytes;
}

// Byte of column c's pair p (K 2p, 2p+1) in layout 1, and its scale in order 1.
size_t weight_byte(const CommonQ4Info & a, int c, int pair) {
    const int kb = pair / 16, p = pair % 16;
    const size_t tile = (size_t)(c / 32) * (a.kp / 32);
    return (tile + kb) * 512 + (size_t)(c % 16) * 32 + (size_t)((c % 32) / 16) * 16 + p;
}
size_t scale_byte(const CommonQ4Info & a, int c, int kb) { return a.scale_offset + ((size_t)kb * a.np + c) * 2; }

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch()).count();
}

bool overlaps(uintptr_t a, size_t a_bytes, uintptr_t b, size_t b_bytes) { return a < b + b_bytes && b < a + a_bytes; }

// Device storage of quantized activations, shared by a workspace and the
// leases it issued; a lease is live while its epoch equals the storage's.
struct ActivationStorage {
    int device = -1;
    void * quant = nullptr;
    size_t quant_bytes = 0;
    void * scale = nullptr;
    size_t scale_bytes = 0;
    void * tiled = nullptr;             // M > 1 codes in the GEMM's operand order
    size_t tiled_bytes = 0;
    uint64_t epoch = 0;
    bool valid = false;
    bool profile = false;
    CommonQ4ActivationStatistics stats{};
    ActivationStorage() {
        const char * p = std::getenv("KUNLUN_Q4_ACT_PROFILE");
        profile = p && !std::strcmp(p, "1");
    }
    ~ActivationStorage() {
        std::lock_guard<std::recursive_mutex> lock(detail::mutex());
        if (device >= 0) {
            select(device);
            check(wait());
            release(device, quant, quant_bytes);
            release(device, scale, scale_bytes);
            release(device, tiled, tiled_bytes);
        }
    }
};

void invalidate(ActivationStorage & s) {
    if (s.valid) ++s.stats.invalidations;
    s.valid = false;
    require(++s.epoch != 0);
}

// Grow a device buffer of the storage; waits for submitted work first.
void reserve(ActivationStorage & s, int id, void *& ptr, size_t & bytes, size_t need) {
    if (bytes >= need) return;
    detail::DeviceContext & ctx = detail::context(id);
    detail::check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    release(id, ptr, bytes);
    ptr = allocate(id, need);
    require(ptr != nullptr);
    bytes = need;
    s.device = id;
}

} // namespace

bool common_q4_supported(int k, int n) { return k > 0 && k <= 16384 && n > 0 && n <= 32000; }

size_t common_q4_size(int k, int n) { return common_q4_supported(k, n) ? describe(k, n, 0).payload_bytes : 0; }

// ---------------------------------------------------------------------------
struct CommonQ4Weight::Impl {
    CommonQ4Info info{};
    void * owned = nullptr;
    void * storage = nullptr;
    bool ready = false;
    CommonQ4WeightStatistics stats{};
};

CommonQ4Weight::CommonQ4Weight(int id, int k, int n, void * storage, size_t bytes) : impl_(new Impl{}) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    int count = 0;
    require(id >= 0 && id < max_devices && common_q4_supported(k, n));
    require(device_count(&count) == 0 && id < count);
    impl_->info = describe(k, n, id);
    const size_t need = impl_->info.payload_bytes;
    if (!storage) {
        impl_->owned = allocate(id, need);
        require(impl_->owned != nullptr);
        storage = impl_->owned;
        bytes = need;
    }
    require((uintptr_t)storage % 256 == 0 && bytes >= need);
    impl_->storage = storage;
}

CommonQ4Weight::~CommonQ4Weight() {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    if (impl_->owned) {
        select(impl_->info.device);
        check(wait());
        release(impl_->info.device, impl_->owned, impl_->info.payload_bytes);
    }
    delete impl_;
}

CommonQ4Info CommonQ4Weight::info() const { return impl_->info; }
void * CommonQ4Weight::data() const { return impl_->storage; }
CommonQ4WeightStatistics CommonQ4Weight::statistics() const {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    return impl_->stats;
}

void CommonQ4Weight::upload(const void * q4, size_t bytes) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    Impl & s = *impl_;
    const CommonQ4Info a = s.info;
    const int blocks = (a.k + 31) / 32;
    require(q4 && bytes == (size_t)a.n * blocks * 18);
    const auto t0 = std::chrono::steady_clock::now();
    // Q4_0 byte i of a block holds K i (low nibble) and 16 + i (high), offset
    // by 8; layout byte of pair p holds K 2p (low) and 2p + 1 (high) signed.
    std::vector<uint8_t> packed(a.payload_bytes, 0);
    const uint8_t * raw = static_cast<const uint8_t *>(q4);
    for (int c = 0; c < a.n; ++c) {
        for (int b = 0; b < blocks; ++b) {
            const uint8_t * src = raw + ((size_t)c * blocks + b) * 18;
            const size_t sb = scale_byte(a, c, b);
            packed[sb] = src[0];
            packed[sb + 1] = src[1];
            uint8_t * dst = packed.data() + weight_byte(a, c, b * 16);
            for (int p = 0; p < 8; ++p)
                dst[p] = (uint8_t)(((src[2 + 2 * p] & 15u) ^ 8u) | (((src[3 + 2 * p] & 15u) ^ 8u) << 4));
            for (int p = 8; p < 16; ++p)
                dst[p] = (uint8_t)(((src[2 + 2 * p - 16] >> 4) ^ 8u) | (((src[3 + 2 * p - 16] >> 4) ^ 8u) << 4));
        }
    }
    const auto t1 = std::chrono::steady_clock::now();
    select(a.device);
    check(wait());
    check(copy(s.storage, packed.data(), a.payload_bytes, host_to_device));
    check(wait());
    const auto t2 = std::chrono::steady_clock::now();
    s.stats.pack_ms += std::chrono::duration<double, std::milli>(t1 - t0).count();
    s.stats.upload_ms += std::chrono::duration<double, std::milli>(t2 - t1).count();
    ++s.stats.uploads;
    s.stats.upload_bytes += a.payload_bytes;
    s.ready = true;
}

// ---------------------------------------------------------------------------
struct CommonQ4ActivationLease::Impl {
    std::shared_ptr<ActivationStorage> storage;
    uint64_t epoch = 0, generation = 0;
    int id = -1, k = 0, m = 0;
    InputType type = InputType::f32;
    const void * input = nullptr;
    size_t input_bytes = 0;
    std::vector<CommonQ4ActivationChunk> chunks;
    std::vector<const void *> tiled;       // per chunk: M > 1 codes in the GEMM's operand order
};

struct CommonQ4Workspace::Impl {
    int id = -1;
    std::shared_ptr<ActivationStorage> activation = std::make_shared<ActivationStorage>();
    CommonQ4Statistics stats{};
    CommonQ4PairStatistics pair_stats{};
    CommonQ4PairStatus pair_status = CommonQ4PairStatus::NotAttempted;
    const void * last_values = nullptr;
    const void * last_scales = nullptr;
    int last_rows = 0, last_kp = 0, last_components = 0;
};

CommonQ4Workspace::CommonQ4Workspace() : impl_(new Impl{}) {}
CommonQ4Workspace::~CommonQ4Workspace() {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    invalidate(*impl_->activation);
    delete impl_;
}

CommonQ4Statistics CommonQ4Workspace::statistics() const {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    CommonQ4Statistics a = impl_->stats;
    const ActivationStorage & st = *impl_->activation;
    a.hbm_workspace_bytes = 0;
    for (size_t b : {st.quant_bytes, st.scale_bytes, st.tiled_bytes})
        if (b) a.hbm_workspace_bytes += std::max<size_t>(b, 256);
    a.l3_workspace_bytes = 0;
    a.slice_bytes = 0;
    return a;
}

CommonQ4ActivationStatistics CommonQ4Workspace::activation_statistics() const {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    const ActivationStorage & st = *impl_->activation;
    CommonQ4ActivationStatistics a = st.stats;
    a.hbm_activation_bytes = 0;
    for (size_t b : {st.quant_bytes, st.scale_bytes, st.tiled_bytes})
        if (b) a.hbm_activation_bytes += std::max<size_t>(b, 256);
    return a;
}

CommonQ4MacStatistics CommonQ4Workspace::mac_statistics() const { return CommonQ4MacStatistics{}; }

CommonQ4Quantization CommonQ4Workspace::quantization() const {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    const Impl & s = *impl_;
    return {s.last_components ? s.last_values : nullptr, s.last_components ? s.last_scales : nullptr, s.last_rows,
            s.last_kp, s.last_components};
}

CommonQ4ActivationLease::CommonQ4ActivationLease() : impl_(new Impl{}) {}
CommonQ4ActivationLease::~CommonQ4ActivationLease() {
    reset();
    delete impl_;
}
void CommonQ4ActivationLease::reset() {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    Impl & a = *impl_;
    if (a.storage && a.storage->valid && a.epoch == a.storage->epoch) invalidate(*a.storage);
    a.storage.reset();
    a.chunks.clear();
    a.tiled.clear();
    a.epoch = a.generation = 0;
}
bool CommonQ4ActivationLease::matches(int id, int k, int m, InputType type, uint64_t generation) const {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    const Impl & a = *impl_;
    return generation && a.storage && a.storage->valid && a.epoch == a.storage->epoch && a.generation == generation &&
           a.id == id && a.k == k && a.m == m && a.type == type;
}
size_t CommonQ4ActivationLease::chunks() const {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    const Impl & a = *impl_;
    return a.storage && a.storage->valid && a.epoch == a.storage->epoch ? a.chunks.size() : 0;
}
CommonQ4ActivationChunk CommonQ4ActivationLease::chunk(size_t index) const {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    return index < chunks() ? impl_->chunks[index] : CommonQ4ActivationChunk{};
}

// ---------------------------------------------------------------------------
namespace {

int padded_rows(int m, int rows) { return m == 1 ? 1 : rows <= 8 ? 8 : rows <= 32 ? 32 : rows <= 64 ? 64 : 128; }

// Route index of CommonQ4Statistics::paths for an M > 1 chunk.
int gemm_path(int padded, int kp) {
    if (padded == 8) return 1;
    if (padded == 32) return 2;
    if (padded == 64) return kp > 8192 ? 5 : 3;
    return kp > 4096 ? 6 : 4;
}

bool exact_route(const CommonQ4Info & a) { return (size_t)a.np * a.kp > kExactRoute; }

// Quantizes one chunk of rows into (values, scales); returns launches made.
void quantize_chunk(CommonQ4Workspace::Impl & s, hipStream_t stream, const void * x, int x_f16, const CommonQ4Info & a,
                    int m, int rows, int padded, void * values, void * scales, void * tiled) {
    ActivationStorage & st = *s.activation;
    const uint64_t t0 = st.profile ? now_ns() : 0;
    if (m == 1)
        detail::check_hip((hipError_t)kk_common_quant_pair(x, x_f16, a.k, a.kp, values, scales, stream),
                          "kk_common_quant_pair");
    else
        detail::check_hip((hipError_t)kk_common_quant_rows(x, x_f16, a.k, a.kp, rows, round_up(padded, 32), values,
                                                           scales, tiled, stream),
                          "kk_common_quant_rows");
    if (st.profile) {
        detail::check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
        st.stats.quantization_ns += now_ns() - t0;
    }
    ++st.stats.quantized_chunks;
    ++st.stats.quant_kernel_launches;
}

// Runs every chunk of Y = X W^T. `prepared` supplies quantized chunks (or
// null: quantize here into the workspace). False: a prepared M = 1 lease met
// the exact route, which needs the raw activations (nothing written).
bool execute(CommonQ4Workspace::Impl & s, int id, void * y, const CommonQ4Info & a, const void * w,
             const void * input, int m, InputType type, const CommonQ4ActivationLease::Impl * prepared) {
    const int bytes = type == InputType::f16 ? 2 : 4, x_f16 = bytes == 2;
    detail::DeviceContext & ctx = detail::context(id);
    ActivationStorage & st = *s.activation;
    if (m == 1 && exact_route(a) && prepared) return false;
    size_t index = 0;
    for (int first = 0; first < m;) {
        const int rows = std::min(128, m - first), padded = padded_rows(m, rows);
        const void * x = static_cast<const char *>(input) + (size_t)first * a.k * bytes;
        float * out = static_cast<float *>(y) + (size_t)first * a.n;
        const CommonQ4ActivationChunk * chunk = prepared ? &prepared->chunks[index++] : nullptr;
        if (m == 1 && exact_route(a)) {
            detail::check_hip((hipError_t)kk_common_gemv(w, out, nullptr, nullptr, x, 2, x_f16, nullptr, nullptr, a.k,
                                                         a.kp, a.n, a.np, ctx.stream),
                              "kk_common_gemv");
            s.last_components = 0;
            ++s.stats.paths[7];
        } else {
            const void * values;
            const void * scales;
            const void * tiled = nullptr;
            if (chunk) {
                values = chunk->values;
                scales = chunk->scales;
                tiled = prepared->tiled[index - 1];
            } else {
                reserve(st, id, st.quant, st.quant_bytes, m == 1 ? (size_t)4 * a.kp + 1024 : (size_t)128 * a.kp + 1024);
                reserve(st, id, st.scale, st.scale_bytes, m == 1 ? 64 : 128 * 64);
                if (m != 1) reserve(st, id, st.tiled, st.tiled_bytes, (size_t)128 * a.kp);
                // M = 1 quantizes inside the GEMV (every workgroup for itself,
                // workgroup 0 writes the view); M > 1 runs the row kernel first
                if (m != 1) quantize_chunk(s, ctx.stream, x, x_f16, a, m, rows, padded, st.quant, st.scale, st.tiled);
                else ++st.stats.quantized_chunks;
                values = st.quant;
                scales = st.scale;
                tiled = st.tiled;
            }
            if (m == 1) {
                const bool fused = chunk == nullptr;
                detail::check_hip((hipError_t)kk_common_gemv(w, out, nullptr, nullptr, fused ? x : values, fused ? 1 : 0,
                                                             x_f16, const_cast<void *>(scales),
                                                             const_cast<void *>(values), a.k, a.kp, a.n, a.np,
                                                             ctx.stream),
                                  "kk_common_gemv");
                s.last_components = 2;
                ++s.stats.paths[0];
            } else {
                detail::check_hip((hipError_t)kk_common_gemm(w, tiled, scales, out, rows, round_up(padded, 32), a.kp,
                                                             a.n, a.np, ctx.stream),
                                  "kk_common_gemm");
                s.last_components = 1;
                ++s.stats.paths[gemm_path(padded, a.kp)];
            }
            s.last_values = values;
            s.last_scales = scales;
        }
        s.last_rows = rows;
        s.last_kp = a.kp;
        first += rows;
        ++s.stats.chunks;
    }
    detail::check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    ++s.stats.calls;
    detail::count_matmul(id);
    detail::note_route(m == 1 ? (exact_route(a) ? "common_gemv_exact" : "common_gemv_a8") : "common_gemm_a8");
    return true;
}

} // namespace

void common_q4_matmul(CommonQ4Workspace & workspace, int id, void * y, const CommonQ4Weight & weight,
                      const void * input, int m, InputType type) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    const CommonQ4Weight::Impl & w = *weight.impl_;
    const CommonQ4Info a = w.info;
    CommonQ4Workspace::Impl & s = *workspace.impl_;
    require(w.ready && id == a.device && abi_ok(a));
    require(m > 0 && (size_t)m * a.k <= INT_MAX / 4 && (size_t)m * a.n <= INT_MAX / 4 && input && y &&
            (type == InputType::f32 || type == InputType::f16));
    const int bytes = type == InputType::f16 ? 2 : 4;
    const uintptr_t yp = (uintptr_t)y, xp = (uintptr_t)input, wp = (uintptr_t)w.storage;
    const size_t ys = (size_t)m * a.n * 4, xs = (size_t)m * a.k * bytes, ws = a.payload_bytes;
    require(yp % 4 == 0 && xp % bytes == 0 && wp % 256 == 0 && yp + ys >= yp && xp + xs >= xp && wp + ws >= wp);
    require(!overlaps(yp, ys, xp, xs) && !overlaps(yp, ys, wp, ws) && !overlaps(xp, xs, wp, ws));
    require(s.id == -1 || s.id == id);
    s.id = id;
    invalidate(*s.activation);
    s.last_components = 0;
    require(execute(s, id, y, a, w.storage, input, m, type, nullptr));
}

bool common_q4_prepare(CommonQ4Workspace & work, int id, const void * input, int k, int m, InputType type,
                       uint64_t generation, CommonQ4ActivationLease & lease) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    CommonQ4Workspace::Impl & s = *work.impl_;
    ActivationStorage & st = *s.activation;
    auto reject = [&]() {
        ++st.stats.rejected_calls;
        return false;
    };
    int count = 0;
    if (id < 0 || id >= max_devices || device_count(&count) != 0 || id >= count || !input || !generation ||
        !common_q4_supported(k, 1) || m <= 0 || (size_t)m * k > INT_MAX / 4 ||
        (type != InputType::f32 && type != InputType::f16) || (s.id != -1 && s.id != id))
        return reject();
    const int bytes = type == InputType::f16 ? 2 : 4;
    const uintptr_t xp = (uintptr_t)input;
    const size_t input_bytes = (size_t)m * k * bytes;
    if (xp % bytes || xp + input_bytes < xp) return reject();
    // The quantized view of an earlier call is not a valid source for the
    // buffer about to be overwritten.
    if ((st.quant && overlaps(xp, input_bytes, (uintptr_t)st.quant, st.quant_bytes)) ||
        (st.scale && overlaps(xp, input_bytes, (uintptr_t)st.scale, st.scale_bytes)))
        return reject();
    const CommonQ4Info a = describe(k, 1, id);
    const size_t chunks = ((size_t)m + 127) / 128;
    const size_t qstride = m == 1 ? (size_t)4 * a.kp + 1024 : (size_t)128 * a.kp + 1024;
    const size_t sstride = m == 1 ? 64 : 128 * 64;
    if (chunks * qstride > kLeaseLimit) return reject();
    const uint64_t t0 = st.profile ? now_ns() : 0;
    lease.reset();
    invalidate(st);
    s.last_components = 0;
    s.id = id;
    detail::DeviceContext & ctx = detail::context(id);
    reserve(st, id, st.quant, st.quant_bytes, chunks * qstride);
    reserve(st, id, st.scale, st.scale_bytes, chunks * sstride);
    if (m != 1) reserve(st, id, st.tiled, st.tiled_bytes, chunks * 128 * (size_t)a.kp);
    CommonQ4ActivationLease::Impl & l = *lease.impl_;
    l.storage = s.activation;
    l.epoch = st.epoch;
    l.generation = generation;
    l.id = id;
    l.k = k;
    l.m = m;
    l.type = type;
    l.input = input;
    l.input_bytes = input_bytes;
    size_t index = 0;
    for (int first = 0; first < m; ++index) {
        const int rows = std::min(128, m - first), padded = padded_rows(m, rows);
        const void * x = static_cast<const char *>(input) + (size_t)first * k * bytes;
        void * q = static_cast<char *>(st.quant) + index * qstride;
        void * sc = static_cast<char *>(st.scale) + index * sstride;
        void * tl = m == 1 ? nullptr : static_cast<char *>(st.tiled) + index * 128 * (size_t)a.kp;
        quantize_chunk(s, ctx.stream, x, bytes == 2, a, m, rows, padded, q, sc, tl);
        l.tiled.push_back(tl);
        const int defined = m == 1 ? 1 : round_up(padded, 32);
        l.chunks.push_back({q, sc, first, rows, padded, a.kp, m == 1 ? 2 : 1,
                            m == 1 ? qstride : (size_t)defined * a.kp, m == 1 ? sstride : (size_t)defined * 64});
        s.last_values = q;
        s.last_scales = sc;
        s.last_rows = rows;
        s.last_kp = a.kp;
        s.last_components = m == 1 ? 2 : 1;
        first += rows;
    }
    detail::check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    st.valid = true;
    ++st.stats.prepare_calls;
    if (st.profile) st.stats.preparation_ns += now_ns() - t0;
    return true;
}

bool common_q4_matmul_shared(CommonQ4Workspace & work, int id, void * y, const CommonQ4Weight & weight,
                             const CommonQ4ActivationLease & lease, uint64_t generation) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    CommonQ4Workspace::Impl & s = *work.impl_;
    const CommonQ4ActivationLease::Impl & l = *lease.impl_;
    const CommonQ4Weight::Impl & w = *weight.impl_;
    const CommonQ4Info a = w.info;
    ActivationStorage & st = *s.activation;
    auto reject = [&]() {
        ++st.stats.rejected_calls;
        return false;
    };
    if (l.storage != s.activation || !lease.matches(id, a.k, l.m, l.type, generation) || !w.ready || id != a.device ||
        s.id != id || !y)
        return reject();
    if (!abi_ok(a) || (size_t)l.m * a.n > INT_MAX / 4) return reject();
    const uintptr_t yp = (uintptr_t)y, wp = (uintptr_t)w.storage;
    const size_t ys = (size_t)l.m * a.n * 4;
    if (yp % 4 || yp + ys < yp || wp % 256 || wp + a.payload_bytes < wp ||
        overlaps(yp, ys, (uintptr_t)l.input, l.input_bytes) || overlaps(yp, ys, wp, a.payload_bytes) ||
        overlaps((uintptr_t)l.input, l.input_bytes, wp, a.payload_bytes) ||
        overlaps(yp, ys, (uintptr_t)st.quant, st.quant_bytes) || overlaps(yp, ys, (uintptr_t)st.scale, st.scale_bytes))
        return reject();
    if (!execute(s, id, y, a, w.storage, l.input, l.m, l.type, &l)) return reject();
    ++st.stats.prepared_matmuls;
    st.stats.prepared_chunks += l.chunks.size();
    return true;
}

bool common_q4_matmul_pair(CommonQ4Workspace & work, int id, void * y0, void * y1, const CommonQ4Weight & weight0,
                           const CommonQ4Weight & weight1, const CommonQ4ActivationLease & lease, uint64_t generation) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    CommonQ4Workspace::Impl & s = *work.impl_;
    const CommonQ4ActivationLease::Impl & l = *lease.impl_;
    const CommonQ4Weight::Impl & w0 = *weight0.impl_;
    const CommonQ4Weight::Impl & w1 = *weight1.impl_;
    const CommonQ4Info a = w0.info, b = w1.info;
    ActivationStorage & st = *s.activation;
    auto reject = [&](CommonQ4PairStatus reason) {
        ++s.pair_stats.declined;
        s.pair_status = reason;
        return false;
    };
    const char * flag = std::getenv("GGML_KUNLUN_Q4_GATE_UP_PAIR");
    if (flag && std::strcmp(flag, "auto") && std::strcmp(flag, "1")) return reject(CommonQ4PairStatus::Disabled);
    if (id < 0 || id >= max_devices || s.id != id || !y0 || !y1 || !w0.ready || !w1.ready || a.device != id ||
        b.device != id || a.k != b.k || a.n != b.n || !((a.k == 4096 && a.n == 11008) || (a.k == 2048 && a.n == 5632)))
        return reject(CommonQ4PairStatus::InvalidInput);
    if (l.storage != s.activation || l.m != 1 || l.type != InputType::f32 ||
        !lease.matches(id, a.k, 1, InputType::f32, generation) || l.chunks.size() != 1)
        return reject(CommonQ4PairStatus::Lease);
    for (const CommonQ4Info & v : {a, b})
        if (!abi_ok(v) || v.k != v.kp || v.n != v.np) return reject(CommonQ4PairStatus::WeightAbi);
    struct Range {
        uintptr_t p;
        size_t bytes;
    };
    const Range outputs[] = {{(uintptr_t)y0, (size_t)a.n * 4}, {(uintptr_t)y1, (size_t)a.n * 4}};
    const Range inputs[] = {{(uintptr_t)w0.storage, a.payload_bytes},
                            {(uintptr_t)w1.storage, b.payload_bytes},
                            {(uintptr_t)l.input, l.input_bytes},
                            {(uintptr_t)st.quant, st.quant_bytes},
                            {(uintptr_t)st.scale, st.scale_bytes}};
    auto overlap = [](const Range & x, const Range & z) { return x.p < z.p + z.bytes && z.p < x.p + x.bytes; };
    for (const Range & x : outputs)
        if (x.p % 64 || x.bytes > UINTPTR_MAX - x.p) return reject(CommonQ4PairStatus::Alias);
    for (const Range & x : inputs)
        if (!x.p || x.bytes > UINTPTR_MAX - x.p) return reject(CommonQ4PairStatus::Alias);
    if (overlap(outputs[0], outputs[1]) || w0.storage == w1.storage || overlap(inputs[0], inputs[2]) ||
        overlap(inputs[1], inputs[2]))
        return reject(CommonQ4PairStatus::Alias);
    for (const Range & x : outputs)
        for (const Range & z : inputs)
            if (overlap(x, z)) return reject(CommonQ4PairStatus::Alias);
    const CommonQ4ActivationChunk & chunk = l.chunks[0];
    if (chunk.kp != a.k || chunk.rows != 1 || chunk.padded_rows != 1 || chunk.components != 2)
        return reject(CommonQ4PairStatus::Lease);
    if ((size_t)a.n * (a.k / 32) * 4 > 8u * 1024 * 1024) return reject(CommonQ4PairStatus::Workspace);
    detail::DeviceContext & ctx = detail::context(id);
    detail::check_hip((hipError_t)kk_common_gemv(w0.storage, static_cast<float *>(y0), w1.storage,
                                                 static_cast<float *>(y1), chunk.values, 0, 0,
                                                 const_cast<void *>(chunk.scales), nullptr, a.k, a.kp, a.n, a.np,
                                                 ctx.stream),
                      "kk_common_gemv");
    detail::check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    s.last_values = chunk.values;
    s.last_scales = chunk.scales;
    s.last_components = 2;
    s.last_rows = 1;
    s.last_kp = a.k;
    s.stats.paths[0] += 2;
    s.stats.calls += 2;
    s.stats.chunks += 2;
    detail::count_matmul(id);
    detail::count_matmul(id);
    st.stats.prepared_matmuls += 2;
    st.stats.prepared_chunks += 2;
    s.pair_status = CommonQ4PairStatus::Success;
    ++s.pair_stats.calls;
    detail::note_route("common_gemv_a8_pair");
    return true;
}

CommonQ4PairStatus common_q4_pair_last_status(const CommonQ4Workspace & work) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    return work.impl_->pair_status;
}

CommonQ4PairStatistics common_q4_pair_statistics(const CommonQ4Workspace & work) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    return work.impl_->pair_stats;
}

} // namespace kunlun
