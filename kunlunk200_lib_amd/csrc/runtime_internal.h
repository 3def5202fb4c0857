// Host runtime state shared by the C++ surface, the matmul dispatcher and the
// C ABI. Not installed.
#pragma once

#include <kunlun/k200.h>
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>

namespace kunlun {
namespace detail {

// Per-device submission state, created on first use of a device.
struct DeviceContext {
    bool ready = false;
    hipStream_t stream = nullptr;
    int *status = nullptr;          // device word written by kernels on bad input
    bool status_pending = false;    // a submitted kernel may have written it
    int cus = 0;                    // compute units of the device
};

std::recursive_mutex & mutex();
// Selects `device` and returns its context, creating stream and status word.
DeviceContext & context(int device);
int current_device();
void count_matmul(int device);
size_t matmul_count(int device);
// Abort with the diagnostic context and a message (the require() text).
[[noreturn]] void fail(const char * message);
// Abort when a HIP call fails, naming the call.
void check_hip(hipError_t status, const char * what);
// Kernel route taken by the calling thread's last matmul or swiglu (static string).
const char * route_of_last_matmul();
void note_route(const char * route);

} // namespace detail

} // namespace kunlun

namespace kk {
// matmul's route predicates (matmul.cpp): the smallest batch on the fp16-MFMA
// GEMM, and the batch ranges of the Q4_0 (streamed: K % 256 == 0 and 16-byte
// aligned weights) and the F32/F16 single-pass MFMA GEMVs.
int gemm_min_batch();
bool q4_mfma_batch(int batch, bool streamed);
bool q4_bdiag_batch(int batch);
bool q4_stream_batch(int batch);
bool dense_mfma_batch(int batch);
} // namespace kk

namespace kunlun {

struct Kernel::Impl {
    int id = -1;
    void * i8_workspace = nullptr;      // rowwise_i8 activation codes and maxima
    size_t i8_workspace_size = 0;
    void * gemm_workspace = nullptr;    // fp16 activations of the prefill GEMM
    size_t gemm_workspace_size = 0;
    void * pair_workspace = nullptr;    // gate/up GEMV outputs of matmul_swiglu; elementwise copy of b
    size_t pair_workspace_size = 0;
    const char * route = nullptr;
};

} // namespace kunlun
