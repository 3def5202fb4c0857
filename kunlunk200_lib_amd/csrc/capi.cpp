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

struct kunlun_common_q4_weight {
    kunlun::CommonQ4Weight weight;
    kunlun_common_q4_weight(int device, int k, int n, void * storage, size_t bytes)
        : weight(device, k, n, storage, bytes) {}
};
struct kunlun_common_q4_workspace {
    kunlun::CommonQ4Workspace workspace;
};
struct kunlun_common_q4_lease {
    kunlun::CommonQ4ActivationLease lease;
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

int kunlun_common_q4_supported(int k, int n) { return kunlun::common_q4_supported(k, n) ? 1 : 0; }
size_t kunlun_common_q4_size(int k, int n) { return kunlun::common_q4_size(k, n); }
kunlun_common_q4_weight * kunlun_common_q4_weight_create(int device, int k, int n, void * storage, size_t bytes) {
    return new kunlun_common_q4_weight(device, k, n, storage, bytes);
}
void kunlun_common_q4_weight_destroy(kunlun_common_q4_weight * weight) { delete weight; }
void kunlun_common_q4_weight_info(const kunlun_common_q4_weight * weight, kunlun_common_q4_info * out) {
    kunlun::require(weight && out);
    const kunlun::CommonQ4Info a = weight->weight.info();
    *out = {a.abi_version, a.quant_type, a.layout, a.scale_order, a.k, a.n, a.kp, a.np, a.device, a.scale_offset,
            a.payload_bytes};
}
void * kunlun_common_q4_weight_data(const kunlun_common_q4_weight * weight) {
    kunlun::require(weight != nullptr);
    return weight->weight.data();
}
void kunlun_common_q4_weight_upload(kunlun_common_q4_weight * weight, const void * q4, size_t bytes) {
    kunlun::require(weight != nullptr);
    weight->weight.upload(q4, bytes);
}
void kunlun_common_q4_weight_statistics(const kunlun_common_q4_weight * weight, size_t counts[2], double ms[2]) {
    kunlun::require(weight && counts && ms);
    const kunlun::CommonQ4WeightStatistics s = weight->weight.statistics();
    counts[0] = s.uploads;
    counts[1] = s.upload_bytes;
    ms[0] = s.pack_ms;
    ms[1] = s.upload_ms;
}
kunlun_common_q4_workspace * kunlun_common_q4_workspace_create(void) { return new kunlun_common_q4_workspace(); }
void kunlun_common_q4_workspace_destroy(kunlun_common_q4_workspace * workspace) { delete workspace; }
void kunlun_common_q4_workspace_statistics(const kunlun_common_q4_workspace * workspace, size_t out[13]) {
    kunlun::require(workspace && out);
    const kunlun::CommonQ4Statistics s = workspace->workspace.statistics();
    for (int i = 0; i < 8; ++i) out[i] = s.paths[i];
    out[8] = s.calls;
    out[9] = s.chunks;
    out[10] = s.hbm_workspace_bytes;
    out[11] = s.l3_workspace_bytes;
    out[12] = s.slice_bytes;
}
void kunlun_common_q4_activation_statistics(const kunlun_common_q4_workspace * workspace, uint64_t out[10]) {
    kunlun::require(workspace && out);
    const kunlun::CommonQ4ActivationStatistics s = workspace->workspace.activation_statistics();
    const uint64_t v[10] = {s.prepare_calls, s.quantized_chunks, s.quant_kernel_launches, s.prepared_matmuls,
                            s.prepared_chunks, s.invalidations, s.rejected_calls, s.hbm_activation_bytes,
                            s.quantization_ns, s.preparation_ns};
    for (int i = 0; i < 10; ++i) out[i] = v[i];
}
void kunlun_common_q4_mac_statistics(const kunlun_common_q4_workspace * workspace, size_t out[4]) {
    kunlun::require(workspace && out);
    const kunlun::CommonQ4MacStatistics s = workspace->workspace.mac_statistics();
    out[0] = s.baseline_sd_calls;
    out[1] = s.stream_sd_calls;
    out[2] = s.shape_fallbacks;
    out[3] = s.resident_l1d_bytes;
}
void kunlun_common_q4_quantization(const kunlun_common_q4_workspace * workspace, const void ** values,
                                   const void ** scales, int out[3]) {
    kunlun::require(workspace && values && scales && out);
    const kunlun::CommonQ4Quantization q = workspace->workspace.quantization();
    *values = q.values;
    *scales = q.scales;
    out[0] = q.rows;
    out[1] = q.kp;
    out[2] = q.components;
}
void kunlun_common_q4_matmul(kunlun_common_q4_workspace * workspace, int device, void * y,
                             const kunlun_common_q4_weight * weight, const void * input, int m, int type) {
    kunlun::require(workspace && weight);
    kunlun::common_q4_matmul(workspace->workspace, device, y, weight->weight, input, m, input_type(type));
}
kunlun_common_q4_lease * kunlun_common_q4_lease_create(void) { return new kunlun_common_q4_lease(); }
void kunlun_common_q4_lease_destroy(kunlun_common_q4_lease * lease) { delete lease; }
void kunlun_common_q4_lease_reset(kunlun_common_q4_lease * lease) {
    kunlun::require(lease != nullptr);
    lease->lease.reset();
}
int kunlun_common_q4_lease_matches(const kunlun_common_q4_lease * lease, int device, int k, int rows, int type,
                                   uint64_t generation) {
    kunlun::require(lease != nullptr);
    if (type != KUNLUN_INPUT_F32 && type != KUNLUN_INPUT_F16) return 0;
    return lease->lease.matches(device, k, rows, input_type(type), generation) ? 1 : 0;
}
size_t kunlun_common_q4_lease_chunks(const kunlun_common_q4_lease * lease) {
    kunlun::require(lease != nullptr);
    return lease->lease.chunks();
}
void kunlun_common_q4_lease_chunk(const kunlun_common_q4_lease * lease, size_t index, const void ** values,
                                  const void ** scales, int ints[5], size_t bytes[2]) {
    kunlun::require(lease && values && scales && ints && bytes);
    const kunlun::CommonQ4ActivationChunk c = lease->lease.chunk(index);
    *values = c.values;
    *scales = c.scales;
    ints[0] = c.first;
    ints[1] = c.rows;
    ints[2] = c.padded_rows;
    ints[3] = c.kp;
    ints[4] = c.components;
    bytes[0] = c.values_bytes;
    bytes[1] = c.scales_bytes;
}
int kunlun_common_q4_prepare(kunlun_common_q4_workspace * workspace, int device, const void * input, int k,
                             int rows, int type, uint64_t generation, kunlun_common_q4_lease * lease) {
    kunlun::require(workspace && lease);
    const kunlun::InputType t = type == KUNLUN_INPUT_F16 ? kunlun::InputType::f16
                                : type == KUNLUN_INPUT_F32 ? kunlun::InputType::f32
                                                           : static_cast<kunlun::InputType>(type);
    return kunlun::common_q4_prepare(workspace->workspace, device, input, k, rows, t, generation, lease->lease) ? 1
                                                                                                                 : 0;
}
int kunlun_common_q4_matmul_shared(kunlun_common_q4_workspace * workspace, int device, void * y,
                                   const kunlun_common_q4_weight * weight, const kunlun_common_q4_lease * lease,
                                   uint64_t generation) {
    kunlun::require(workspace && weight && lease);
    return kunlun::common_q4_matmul_shared(workspace->workspace, device, y, weight->weight, lease->lease,
                                           generation) ? 1 : 0;
}
int kunlun_common_q4_matmul_pair(kunlun_common_q4_workspace * workspace, int device, void * y0, void * y1,
                                 const kunlun_common_q4_weight * w0, const kunlun_common_q4_weight * w1,
                                 const kunlun_common_q4_lease * lease, uint64_t generation) {
    kunlun::require(workspace && w0 && w1 && lease);
    return kunlun::common_q4_matmul_pair(workspace->workspace, device, y0, y1, w0->weight, w1->weight, lease->lease,
                                         generation) ? 1 : 0;
}
void kunlun_common_q4_pair_statistics(const kunlun_common_q4_workspace * workspace, size_t out[3]) {
    kunlun::require(workspace && out);
    const kunlun::CommonQ4PairStatistics s = kunlun::common_q4_pair_statistics(workspace->workspace);
    out[0] = s.calls;
    out[1] = s.declined;
    out[2] = s.l3_partial_bytes;
}
int kunlun_common_q4_pair_last_status(const kunlun_common_q4_workspace * workspace) {
    kunlun::require(workspace != nullptr);
    return static_cast<int>(kunlun::common_q4_pair_last_status(workspace->workspace));
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
