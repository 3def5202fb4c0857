// kunlun::elementwise: the reference's argument rules and alias handling
// (reference src/k200.cpp:280-323), then the HIP kernels. Completes before
// returning, as the reference's does.
#include "launch.h"
#include "runtime_internal.h"

#include <climits>
#include <cmath>
#include <cstdint>

namespace kunlun {

void elementwise(Kernel & kernel, int id, void * y, const void * a, const void * b, int count, int width,
                 int b_count, ElementwiseOp operation, float parameter) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    const int op = (int)operation;
    require(y && a && b && count > 0 && count <= INT_MAX / 4 && width > 0 && width <= 16384 &&
            count % width == 0);
    require(op >= 0 && op <= 4 && (b_count == count || b_count == width));
    if (operation == ElementwiseOp::rms_norm) require(std::isfinite(parameter) && parameter > 0);
    require(kernel.impl_->id == -1 || kernel.impl_->id == id);
    require(((uintptr_t)y & 3) == 0 && ((uintptr_t)a & 3) == 0 && ((uintptr_t)b & 3) == 0);
    detail::DeviceContext & ctx = detail::context(id);
    Kernel::Impl & impl = *kernel.impl_;
    impl.id = id;
    // y == a, and y == b with b_count == count, touch each element in one
    // thread only. A repeated b that y overwrites is copied aside first.
    const float * bp = static_cast<const float *>(b);
    if ((op == 0 || op == 1) && y == b && b_count != count) {
        const size_t bytes = (size_t)b_count * 4;
        if (impl.pair_workspace_size < bytes) {
            detail::check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
            release(id, impl.pair_workspace, impl.pair_workspace_size);
            impl.pair_workspace = allocate(id, bytes);
            require(impl.pair_workspace != nullptr);
            impl.pair_workspace_size = bytes;
        }
        detail::check_hip(hipMemcpyAsync(impl.pair_workspace, b, bytes, hipMemcpyDeviceToDevice, ctx.stream),
                          "hipMemcpyAsync");
        bp = static_cast<const float *>(impl.pair_workspace);
    }
    detail::check_hip((hipError_t)kk_elementwise(static_cast<float *>(y), static_cast<const float *>(a), bp, count,
                                                 width, b_count, op, parameter, ctx.stream),
                      "kk_elementwise");
    detail::check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
    static const char * const routes[] = {"elementwise_add", "elementwise_multiply", "elementwise_silu",
                                          "elementwise_rms_norm", "elementwise_scale"};
    impl.route = routes[op];
    detail::note_route(impl.route);
}

} // namespace kunlun
