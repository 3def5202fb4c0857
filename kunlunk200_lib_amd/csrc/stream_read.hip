// Read-only streaming kernels: the measured HBM read ceiling the matmul
// GEMVs are compared against (bench.py --only read). Built into its own
// library (libkunlunk200_stream.so), not into libkunlunk200.so.0.
//
// Each kernel reads every byte of a buffer exactly once with 16-byte vector
// loads and folds the data into one XOR word per lane, stored only when it
// equals a sentinel, so no output traffic competes with the reads.
//   variant 0  grid-stride loop, one 16-byte load per lane per iteration.
//   variant 1  "all issued": each wave owns a contiguous range of R KiB and
//              issues all R of its 1 KiB load instructions (lane i at
//              16 * i of each KiB) before the first use.
//   variant 2  as 1 with non-temporal loads (no reuse: stream past the caches).
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace {

constexpr int kThreads = 512;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void read_grid_stride(const u32x4 *__restrict__ p, size_t n16,
                                                             unsigned *out) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    unsigned acc = 0;
    for (size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) out[0] = acc;
}

// R loads of 1 KiB per wave (clamped to the buffer, so the tail wave re-reads
// the last chunk instead of running past it).
template <int R, bool NT>
__global__ __launch_bounds__(kThreads) void read_all_issued(const u32x4 *__restrict__ p, size_t n16,
                                                            size_t per_wave16, unsigned *out) {
    const int lane = threadIdx.x & 63;
    const size_t wave = blockIdx.x * static_cast<size_t>(kThreads / 64) + (threadIdx.x >> 6);
    const size_t base = wave * per_wave16;
    u32x4 v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        size_t idx = base + static_cast<size_t>(i) * 64 + lane;
        idx = idx < n16 ? idx : n16 - 1;
        v[i] = NT ? __builtin_nontemporal_load(p + idx) : p[idx];
    }
    unsigned acc = 0;
#pragma unroll
    for (int i = 0; i < R; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (acc == 0x9e3779b9u) out[0] = acc;
}

template <bool NT>
hipError_t launch_all_issued(const u32x4 *p, size_t n16, int waves, unsigned *out, hipStream_t stream) {
    const size_t per_wave16 = ((n16 + waves - 1) / waves + 63) / 64 * 64;   // whole KiB per wave
    const size_t r = per_wave16 / 64;
    const dim3 grid(waves / (kThreads / 64)), block(kThreads);
#define KK_READ_CASE(RR)                                                                                 \
    if (r <= RR) {                                                                                       \
        hipLaunchKernelGGL((read_all_issued<RR, NT>), grid, block, 0, stream, p, n16, per_wave16, out); \
        return hipGetLastError();                                                                        \
    }
    KK_READ_CASE(4)
    KK_READ_CASE(8)
    KK_READ_CASE(13)
    KK_READ_CASE(18)
    KK_READ_CASE(24)
    KK_READ_CASE(36)
    KK_READ_CASE(48)
    KK_READ_CASE(64)
#undef KK_READ_CASE
    return hipErrorInvalidValue;
}

} // namespace

extern "C" {

// Reads `bytes` (a multiple of 16, 16-byte aligned) at `p` once. `variant`
// as above; `waves` (a multiple of 8) sizes the grid: the number of waves for
// variants 1 and 2 (at most 64 KiB per wave), the number of waves of the
// grid-stride loop for variant 0. `out` is one device word (written only on
// a sentinel match). Returns 0 or a hipError_t.
int kk_stream_read(const void *p, size_t bytes, int variant, int waves, void *out, void *stream) {
    if (!p || !out || bytes < 16 || (bytes & 15) || (reinterpret_cast<uintptr_t>(p) & 15) || waves <= 0 ||
        (waves & 7))
        return hipErrorInvalidValue;
    const u32x4 *v = static_cast<const u32x4 *>(p);
    const size_t n16 = bytes / 16;
    unsigned *o = static_cast<unsigned *>(out);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (variant == 0) {
        hipLaunchKernelGGL(read_grid_stride, dim3(waves / 8), dim3(kThreads), 0, s, v, n16, o);
        return hipGetLastError();
    }
    if (variant == 1) return launch_all_issued<false>(v, n16, waves, o, s);
    if (variant == 2) return launch_all_issued<true>(v, n16, waves, o, s);
    return hipErrorInvalidValue;
}

} // extern "C"
