// extern "C" entry points declared in include/kunlun/k200_c.h. Each forwards
// to the C++ surface and keeps its argument meaning and fail-fast behaviour.
#include <kunlun/k200_c.h>

#include "runtime_internal.h"

struct kunlun_kernel {
    kunlun::Kernel kernel;
    const char * route = nullptr;
};

struct kunlun_native_q4_workspace {
    kunlun::NativeQ4Workspace workspace;
};

namespace {
kunlun::InputType input_type(int type) {
    kunlun::require(type == KUNLUN_INPUT_F32 || type == KUNLUN_INPUT_F16);
    return type == KUNLUN_INPUT_F16 ? kunlun::InputType::f16 : kunlun::InputType::f32;
}
} // namespace

extern "C" {

void kunlun_lock(void) { kunlun::runtime_mutex().lock(); }
void kunlun_unlock(void) { kunlun::runtime_mutex().unlock(); }
void kunlun_check(int status) { kunlun::check(status); }
void kunlun_require(int condition) { kunlun::require(condition != 0); }
void kunlun_diagnostic_tensor(const char * name, const int64_t * dimensions) {
    kunlun::diagnostic_tensor(name, dimensions);
}
int kunlun_device_count(int * count) { return kunlun::device_count(count); }
void kunlun_select(int device) { kunlun::select(device); }
int kunlun_wait(void) { return kunlun::wait(); }
int kunlun_copy(void * dst, const void * src, size_t bytes, int kind) {
    kunlun::require(kind >= KUNLUN_HOST_TO_DEVICE && kind <= KUNLUN_DEVICE_TO_DEVICE);
    return kunlun::copy(dst, src, bytes, static_cast<kunlun::CopyKind>(kind));
}
void kunlun_peer(int dst_device, void * dst, int src_device, const void * src, size_t bytes) {
    kunlun::peer(dst_device, dst, src_device, src, bytes);
}
void * kunlun_allocate(int device, size_t bytes) { return kunlun::allocate(device, bytes); }
void kunlun_release(int device, void * ptr, size_t bytes) { kunlun::release(device, ptr, bytes); }
size_t kunlun_allocated_bytes(int device) { return kunlun::allocated_bytes(device); }

kunlun_kernel * kunlun_kernel_create(void) { return new kunlun_kernel(); }
void kunlun_kernel_destroy(kunlun_kernel * kernel) { delete kernel; }

size_t kunlun_aligned(size_t bytes) { return kunlun::aligned(bytes); }
size_t kunlun_packed_i8_size(int k, int rows) { return kunlun::packed_i8_size(k, rows); }
float * kunlun_packed_i8_scales(void * weights, int k, int rows) { return kunlun::packed_i8_scales(weights, k, rows); }
float * kunlun_packed_i8_maxima(void * weights, int k, int rows) { return kunlun::packed_i8_maxima(weights, k, rows); }
void kunlun_upload_i8_rows(int device, void * weights, int k, int rows, int first_row, int count,
                           const float * input) {
    kunlun::upload_i8_rows(device, weights, k, rows, first_row, count, input);
}

void kunlun_matmul(kunlun_kernel * kernel, int device, void * y, const void * w, const void * x, int k, int n,
                   int batch, int type, const float * scales, const float * maxima, int tile) {
    kunlun::require(kernel != nullptr);
    kunlun::require(type >= KUNLUN_F32 && type <= KUNLUN_Q6_K);
    kunlun::matmul(kernel->kernel, device, y, w, x, k, n, batch, static_cast<kunlun::WeightType>(type), scales,
                   maxima, tile);
    kernel->route = kunlun::detail::route_of_last_matmul();
}

int kunlun_native_q4_layout_supported(int k, int n) { return kunlun::native_q4_layout_supported(k, n) ? 1 : 0; }
size_t kunlun_native_q4_size(int k, int n) { return kunlun::native_q4_size(k, n); }
int kunlun_pack_native_q4(void * destination, size_t bytes, const void * q4, int k, int n) {
    return kunlun::pack_native_q4(destination, bytes, q4, k, n) ? 1 : 0;
}
void kunlun_upload_native_q4(int device, void * weights, const void * q4, int k, int n) {
    kunlun::upload_native_q4(device, weights, q4, k, n);
}
const char * kunlun_native_q4_reason(int k, int n, int batch, int type) {
    if (type != KUNLUN_INPUT_F32 && type != KUNLUN_INPUT_F16) {
        if (!kunlun::native_q4_layout_supported(k, n)) return "K/N/layout capacity";
        return "input type";
    }
    return kunlun::native_q4_reason(k, n, batch, input_type(type));
}
kunlun_native_q4_workspace * kunlun_native_q4_workspace_create(void) { return new kunlun_native_q4_workspace(); }
void kunlun_native_q4_workspace_destroy(kunlun_native_q4_workspace * workspace) { delete workspace; }
void kunlun_native_q4_statistics(const kunlun_native_q4_workspace * workspace, size_t out[4]) {
    kunlun::require(workspace != nullptr && out != nullptr);
    const kunlun::NativeQ4Statistics s = workspace->workspace.statistics();
    out[0] = s.accelerated;
    out[1] = s.fallback;
    out[2] = s.hbm_workspace_bytes;
    out[3] = s.l3_workspace_bytes;
}
int kunlun_native_q4_matmul(kunlun_native_q4_workspace * workspace, int device, void * y, const void * weights,
                            const void * input, int k, int n, int batch, int type) {
    kunlun::require(workspace != nullptr);
    return kunlun::native_q4_matmul(workspace->workspace, device, y, weights, input, k, n, batch,
                                    input_type(type)) ? 1 : 0;
}

void kunlun_statistics(size_t out[4]) {
    kunlun::require(out != nullptr);
    const kunlun::Statistics s = kunlun::statistics();
    out[0] = s.matmuls[0];
    out[1] = s.matmuls[1];
    out[2] = s.peer_copies;
    out[3] = s.peer_bytes;
}
const char * kunlun_version(void) { return kunlun::version(); }

void kunlun_elementwise(kunlun_kernel * kernel, int device, void * y, const void * a, const void * b, int count,
                        int width, int b_count, int op, float parameter) {
    kunlun::require(kernel != nullptr);
    kunlun::elementwise(kernel->kernel, device, y, a, b, count, width, b_count, static_cast<kunlun::ElementwiseOp>(op),
                        parameter);
    kernel->route = kunlun::detail::route_of_last_matmul();
}

const char * kunlun_swiglu_reason(int width, int rows, int gate_stride, int up_stride, int output_stride, int type) {
    const kunlun::SwiGLULayout layout{width, rows, gate_stride, up_stride, output_stride,
                                      static_cast<kunlun::InputType>(type)};
    return kunlun::swiglu_reason(layout);
}

int kunlun_swiglu(kunlun_kernel * kernel, int device, void * y, size_t y_bytes, const void * gate, size_t gate_bytes,
                  const void * up, size_t up_bytes, int width, int rows, int gate_stride, int up_stride,
                  int output_stride, int type) {
    if (!kernel) return 0;
    const kunlun::SwiGLULayout layout{width, rows, gate_stride, up_stride, output_stride,
                                      static_cast<kunlun::InputType>(type)};
    const bool done = kunlun::swiglu(kernel->kernel, device, y, y_bytes, gate, gate_bytes, up, up_bytes, layout);
    if (done) kernel->route = kunlun::detail::route_of_last_matmul();
    return done ? 1 : 0;
}

void kunlun_matmul_swiglu(kunlun_kernel * kernel, int device, void * y, const void * w_gate, const void * w_up,
                          const void * x, int k, int n, int batch, int type) {
    kunlun::require(kernel != nullptr);
    kunlun::require(type >= KUNLUN_F32 && type <= KUNLUN_Q6_K);
    kunlun::matmul_swiglu(kernel->kernel, device, y, w_gate, w_up, x, k, n, batch,
                          static_cast<kunlun::WeightType>(type));
    kernel->route = kunlun::detail::route_of_last_matmul();
}

size_t kunlun_matmul_count(int device) { return kunlun::detail::matmul_count(device); }
void * kunlun_stream(int device) { return static_cast<void *>(kunlun::detail::context(device).stream); }
const char * kunlun_kernel_route(const kunlun_kernel * kernel) { return kernel ? kernel->route : nullptr; }

}
