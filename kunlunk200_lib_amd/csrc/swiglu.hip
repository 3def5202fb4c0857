// SiLU(gate) * up over rows of contiguous F32 or F16 values on gfx950
// (reference src/k200.cpp:324-368, kernels/kunlun-swiglu.xpu). F32
// intermediates, one final rounding for F16 output. HBM-bound: 3 x bytes per
// element (two reads, one write).
#include "device_common.h"
#include "launch.h"

namespace {

constexpr int kThreads = 256;

template <int BYTES>
__device__ __forceinline__ float load_value(const uint8_t *p) {
    if constexpr (BYTES == 4) {
        return *reinterpret_cast<const float *>(p);
    } else {
        return static_cast<float>(*reinterpret_cast<const _Float16 *>(p));
    }
}

template <int BYTES>
__device__ __forceinline__ void store_value(uint8_t *p, float v) {
    if constexpr (BYTES == 4) {
        *reinterpret_cast<float *>(p) = v;
    } else {
        *reinterpret_cast<_Float16 *>(p) = static_cast<_Float16>(v);   // round to nearest even
    }
}

// Element e of the rows x width grid is row e / width, column e % width.
// Each element is read and written by one thread only, so an output that
// aliases an input element for element (equal strides) is safe.
template <int BYTES>
__global__ __launch_bounds__(kThreads) void swiglu_rows(uint8_t *y, const uint8_t *gate, const uint8_t *up,
                                                       int width, int rows, int gate_stride, int up_stride,
                                                       int output_stride) {
    const long long total = static_cast<long long>(width) * rows;
    const long long step = static_cast<long long>(gridDim.x) * kThreads;
    for (long long e = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; e < total; e += step) {
        const int row = static_cast<int>(e / width);
        const int col = static_cast<int>(e - static_cast<long long>(row) * width);
        const size_t column_bytes = static_cast<size_t>(col) * BYTES;
        const float g = load_value<BYTES>(gate + static_cast<size_t>(row) * gate_stride + column_bytes);
        const float u = load_value<BYTES>(up + static_cast<size_t>(row) * up_stride + column_bytes);
        store_value<BYTES>(y + static_cast<size_t>(row) * output_stride + column_bytes, kk::swiglu_value(g, u));
    }
}

} // namespace

extern "C" int kk_swiglu(void *y, const void *gate, const void *up, int width, int rows, int gate_stride,
                         int up_stride, int output_stride, int bytes, hipStream_t stream) {
    if (!y || !gate || !up || width <= 0 || rows <= 0 || (bytes != 2 && bytes != 4)) return hipErrorInvalidValue;
    const long long total = static_cast<long long>(width) * rows;
    const long long wanted = (total + kThreads - 1) / kThreads;
    const int groups = static_cast<int>(wanted < 4096 ? wanted : 4096);
    if (bytes == 4)
        hipLaunchKernelGGL(swiglu_rows<4>, dim3(groups), dim3(kThreads), 0, stream, static_cast<uint8_t *>(y),
                           static_cast<const uint8_t *>(gate), static_cast<const uint8_t *>(up), width, rows,
                           gate_stride, up_stride, output_stride);
    else
        hipLaunchKernelGGL(swiglu_rows<2>, dim3(groups), dim3(kThreads), 0, stream, static_cast<uint8_t *>(y),
                           static_cast<const uint8_t *>(gate), static_cast<const uint8_t *>(up), width, rows,
                           gate_stride, up_stride, output_stride);
    return hipGetLastError();
}
