// Elementwise operations of the reference's k200-bench surface on gfx950
// (reference src/k200.cpp:280-323, kernels/kunlun-elementwise.xpu): y = a + b,
// a * b (b of n values, or of `width` values repeated every row), SiLU(a),
// a * parameter, and RMS normalisation of each `width` row with eps =
// parameter. F32 throughout. HBM-bound: 8 or 12 bytes per element.
#include "device_common.h"
#include "launch.h"

#include <algorithm>

namespace {

constexpr int kThreads = 256;

// op: 0 add, 1 multiply, 2 silu, 4 scale (element e of b is b[e % b_count]).
// y may alias a or b: element e is read before it is written, by the same lane.
__global__ __launch_bounds__(kThreads) void elementwise_flat(float *y, const float *a,
                                                            const float *b, int count, int b_count, int op,
                                                            float parameter) {
    const int step = gridDim.x * kThreads;
    for (int e = blockIdx.x * kThreads + threadIdx.x; e < count; e += step) {
        const float v = a[e];
        float out;
        if (op == 0) {
            out = v + b[b_count == count ? e : e % b_count];
        } else if (op == 1) {
            out = v * b[b_count == count ? e : e % b_count];
        } else if (op == 2) {
            out = v / (1.0f + expf(-v));
        } else {
            out = v * parameter;
        }
        y[e] = out;
    }
}

// One workgroup per row: sum of squares (F32), then y = a / sqrt(mean + eps)
// computed as a * (1 / sqrt(sum / width + eps)), the reference's expression.
// Every element is read before the workgroup writes it, so y may equal a.
__global__ __launch_bounds__(kThreads) void rms_norm_rows(float *y, const float *a, int width, float eps) {
    __shared__ float partial[kThreads / kk::kWave];
    const float *row = a + static_cast<size_t>(blockIdx.x) * width;
    float *out = y + static_cast<size_t>(blockIdx.x) * width;
    float sum = 0.0f;
    for (int j = threadIdx.x; j < width; j += kThreads) sum = fmaf(row[j], row[j], sum);
    sum = kk::wave_sum(sum);
    if ((threadIdx.x & (kk::kWave - 1)) == 0) partial[threadIdx.x / kk::kWave] = sum;
    __syncthreads();
    sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kThreads / kk::kWave; ++i) sum += partial[i];
    const float scale = 1.0f / sqrtf(sum / static_cast<float>(width) + eps);
    for (int j = threadIdx.x; j < width; j += kThreads) out[j] = row[j] * scale;
}

} // namespace

extern "C" int kk_elementwise(float *y, const float *a, const float *b, int count, int width, int b_count, int op,
                              float parameter, hipStream_t stream) {
    if (!y || !a || count <= 0 || width <= 0 || count % width != 0 || op < 0 || op > 4) return hipErrorInvalidValue;
    if (op == 3) {
        hipLaunchKernelGGL(rms_norm_rows, dim3(count / width), dim3(kThreads), 0, stream, y, a, width, parameter);
    } else {
        if ((op == 0 || op == 1) && (!b || b_count <= 0)) return hipErrorInvalidValue;
        const int groups = std::max(1, std::min((count + kThreads - 1) / kThreads, 8192));
        hipLaunchKernelGGL(elementwise_flat, dim3(groups), dim3(kThreads), 0, stream, y, a, b, count, b_count, op,
                           parameter);
    }
    return hipGetLastError();
}
