// kunlun::swiglu_reason / kunlun::swiglu: the reference's layout and pointer
// contract (reference src/k200.cpp:324-368), then the HIP SwiGLU kernel. The
// call completes before returning, as the reference's does.
#include "launch.h"
#include "runtime_internal.h"

#include <climits>
#include <cstdint>

namespace kunlun {

namespace {

int element_bytes(InputType type) { return type == InputType::f32 ? 4 : 2; }

// Bytes from the first element of row 0 to the end of the last row.
size_t span_bytes(const SwiGLULayout & p, int stride) {
    return (size_t)(p.rows - 1) * (size_t)stride + (size_t)p.width * element_bytes(p.type);
}

bool overlaps(uintptr_t a, size_t a_bytes, uintptr_t b, size_t b_bytes) { return a < b + b_bytes && b < a + a_bytes; }

} // namespace

const char * swiglu_reason(const SwiGLULayout & p) {
    if (p.type != InputType::f32 && p.type != InputType::f16) return "type";
    const int bytes = element_bytes(p.type);
    if (p.width <= 0 || p.width > 65536 || p.rows <= 0 || p.rows > INT_MAX / p.width / bytes) return "shape";
    for (const int stride : {p.gate_stride, p.up_stride, p.output_stride}) {
        if (stride < p.width * bytes || stride % bytes != 0) return "stride";
        if (span_bytes(p, stride) > (size_t)INT_MAX) return "byte extent";
    }
    return "";
}

bool swiglu(Kernel & kernel, int id, void * y, size_t y_bytes, const void * gate, size_t gate_bytes, const void * up,
            size_t up_bytes, const SwiGLULayout & p) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    if (*swiglu_reason(p) || id < 0 || id >= max_devices || !y || !gate || !up) return false;
    const int bytes = element_bytes(p.type);
    const uintptr_t yp = (uintptr_t)y, gp = (uintptr_t)gate, upp = (uintptr_t)up;
    const size_t ys = span_bytes(p, p.output_stride), gs = span_bytes(p, p.gate_stride),
                 us = span_bytes(p, p.up_stride);
    if (ys > y_bytes || gs > gate_bytes || us > up_bytes) return false;
    if (yp % bytes || gp % bytes || upp % bytes) return false;
    if (yp + ys < yp || gp + gs < gp || upp + us < upp) return false;
    // The output may equal an input element for element, or (packed gate/up
    // rows) sit in the same rows as an input without sharing elements.
    const bool same_as_gate = yp == gp && p.output_stride == p.gate_stride;
    const bool same_as_up = yp == upp && p.output_stride == p.up_stride;
    const size_t row_values = (size_t)p.width * bytes;
    auto disjoint_in_rows = [&](uintptr_t input, int stride) {
        const size_t delta = yp > input ? yp - input : input - yp;
        return (same_as_gate || same_as_up) && stride == p.output_stride && delta >= row_values &&
               delta <= (size_t)stride - row_values;
    };
    if (!same_as_gate && overlaps(yp, ys, gp, gs) && !disjoint_in_rows(gp, p.gate_stride)) return false;
    if (!same_as_up && overlaps(yp, ys, upp, us) && !disjoint_in_rows(upp, p.up_stride)) return false;
    if (kernel.impl_->id != -1 && kernel.impl_->id != id) return false;
    int count = 0;
    if (device_count(&count) != 0 || id >= count) return false;

    kernel.impl_->id = id;
    detail::DeviceContext & ctx = detail::context(id);
    detail::check_hip((hipError_t)kk_swiglu(y, gate, up, p.width, p.rows, p.gate_stride, p.up_stride,
                                            p.output_stride, bytes, ctx.stream),
                      "kk_swiglu");
    detail::check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    kernel.impl_->route = bytes == 4 ? "swiglu_f32" : "swiglu_f16";
    detail::note_route(kernel.impl_->route);
    return true;
}

} // namespace kunlun
