// kunlun::Kernel and kunlun::matmul: argument validation exactly as the
// reference (reference src/k200.cpp:268-279), then submission of the HIP
// kernels for the weight format (reference dispatch src/k200.cpp:187-247).
#include "launch.h"
#include "runtime_internal.h"
#include "tuning.h"

#include <algorithm>
#include <climits>
#include <cstdint>

namespace kunlun {
namespace detail {
thread_local const char * last_route = nullptr;
const char * route_of_last_matmul() { return last_route; }
void note_route(const char * route) { last_route = route; }
} // namespace detail

namespace {

// Grows a Kernel-owned device workspace; waits for work that may still use
// the old one before releasing it.
void * grow(int id, detail::DeviceContext & ctx, void *& ptr, size_t & size, size_t need) {
    if (size < need) {
        if (ptr) {
            detail::check_hip(hipStreamSynchronize(ctx.stream), "hipStreamSynchronize");
            release(id, ptr, size);
            ptr = nullptr;
            size = 0;
        }
        ptr = allocate(id, need);
        require(ptr != nullptr);
        size = need;
    }
    return ptr;
}

} // namespace
} // namespace kunlun

namespace kk {

// Route predicates, shared with the allocation-free entry point (noalloc.hip).
//
// Smallest batch that uses the fp16-MFMA prefill GEMM (F16 and Q4_0 weights);
// smaller batches keep the F32-accumulate GEMV kernels.
int gemm_min_batch() {
    const int v = kk::tuning(kk::kGemmMinBatch);
    return v > 0 ? v : 64;
}

// Batch range of the single-pass Q4_0 MFMA GEMV (within 1..16). Below the
// minimum the batch-1 kernel's passes (two columns each) are faster: the
// streamed kernel (K % 256 == 0, 16-byte aligned weights) wins from 3
// columns, the register-staged one from 5.
bool q4_mfma_batch(int batch, bool streamed) {
    const int min_b = std::max(1, kk::tuning_or(kk::kQ4MfmaMin, streamed ? 3 : 5));
    const int max_b = std::min(16, kk::tuning_or(kk::kQ4MfmaMax, 16));
    return batch >= min_b && batch <= max_b;
}

// Batch range of the block-diagonal Q4_0 MFMA GEMV (the single-pass kernel's
// range, unless KUNLUN_Q4_BDIAG=0 leaves it to the LDS-staged kernels).
bool q4_bdiag_batch(int batch) {
    return kk::tuning_or(kk::kQ4Bdiag, 1) != 0 && q4_mfma_batch(batch, true);
}

// Batch range of the streamed Q4_0 GEMV at K = 4096: KUNLUN_Q4_STREAM_MIN
// (default 5) to 8; a minimum above 8 turns it off.
bool q4_stream_batch(int batch) {
    const int min_b = kk::tuning_or(kk::kQ4StreamMin, 5);
    return batch >= std::max(1, min_b) && batch <= 8;
}

// Batch range of the single-pass F32/F16 MFMA GEMV (within 1..16).
bool dense_mfma_batch(int batch) {
    const int min_b = std::max(1, kk::tuning_or(kk::kDenseMfmaMin, 2));
    const int max_b = std::min(16, kk::tuning_or(kk::kDenseMfmaMax, 16));
    return batch >= min_b && batch <= max_b;
}

} // namespace kk

namespace kunlun {
using kk::dense_mfma_batch;
using kk::gemm_min_batch;
using kk::q4_mfma_batch;

namespace {

// The reference's matmul argument rules (reference src/k200.cpp:271-275):
// supported type, K % 32 == 0, K <= 16384, products that fit int, and a
// weight matrix of at most INT_MAX bytes.
void validate_shape(const void * y, const void * w, const void * x, int k, int n, int batch, WeightType type,
                    int tile) {
    require(type == WeightType::f32 || type == WeightType::f16 || type == WeightType::q4_0 ||
            type == WeightType::rowwise_i8);
    require(k > 0 && k <= 16384 && k % 32 == 0 && n > 0 && batch > 0 && n <= INT_MAX / batch &&
            k <= INT_MAX / batch);
    require((size_t)n * batch <= INT_MAX / 4 && (size_t)k * batch <= INT_MAX / 4);
    const size_t row_bytes = type == WeightType::f32   ? (size_t)k * 4
                             : type == WeightType::f16 ? (size_t)k * 2
                             : type == WeightType::q4_0 ? (size_t)k / 32 * 18
                                                        : (size_t)k;
    require(y && w && x && (size_t)n <= INT_MAX / row_bytes && (tile == 1 || tile == 16));
}

} // namespace

Kernel::Kernel() : impl_(new Impl{}) {}

Kernel::~Kernel() {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    if (impl_->id >= 0) {
        select(impl_->id);
        check(wait());
        release(impl_->id, impl_->i8_workspace, impl_->i8_workspace_size);
        release(impl_->id, impl_->gemm_workspace, impl_->gemm_workspace_size);
        release(impl_->id, impl_->pair_workspace, impl_->pair_workspace_size);
    }
    delete impl_;
}

// The F32/F16/Q4_0 product's route for one matrix (matmul's, and each half of
// an unfused gate/up pair): the prefill GEMM, the small-batch MFMA GEMVs,
// else the single-pass GEMVs.
static void dispatch_dense(Kernel::Impl & impl, detail::DeviceContext & ctx, int id, void * y, const void * w,
                    const void * x, int k, int n, int batch, WeightType type) {
    const bool gemm = (type == WeightType::q4_0 || (type == WeightType::f16 && ((uintptr_t)w & 15) == 0)) &&
                      batch >= gemm_min_batch() && ((uintptr_t)x & 15) == 0;
    if (!gemm && batch > 16) {
        // batches between the small-batch kernels and the GEMM: chunks of 16
        // columns, each on the route a 16-column call takes (one pass over
        // the weights per chunk, against one per 2-4 columns on the general
        // GEMV). X and Y chunks keep their alignment (K % 32 == 0).
        const char * first = nullptr;
        for (int b0 = 0; b0 < batch; b0 += 16) {
            dispatch_dense(impl, ctx, id, static_cast<char *>(y) + (size_t)b0 * n * 4, w,
                           static_cast<const char *>(x) + (size_t)b0 * k * 4, k, n, std::min(16, batch - b0), type);
            if (!first) first = impl.route;
        }
        impl.route = first;
        return;
    }
    if (gemm) {
        grow(id, ctx, impl.gemm_workspace, impl.gemm_workspace_size, kk_gemm_workspace_bytes(k, n, batch));
        detail::check_hip((hipError_t)kk_gemm((int)type, w, static_cast<const float *>(x), static_cast<float *>(y), k,
                                              n, batch, impl.gemm_workspace, ctx.stream, &impl.route),
                          "kk_gemm");
    } else if ((type == WeightType::f32 || type == WeightType::f16) && dense_mfma_batch(batch) &&
               ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0) {
        detail::check_hip((hipError_t)kk_dense_mfma_gemv((int)type, w, static_cast<const float *>(x),
                                                         static_cast<float *>(y), k, n, batch, ctx.stream),
                          "kk_dense_mfma_gemv");
        impl.route = type == WeightType::f16 ? "f16_mfma_gemv" : "f32_mfma_gemv";
    } else if (type == WeightType::q4_0 && kk::q4_stream_batch(batch) &&
               kk_q4_stream_gemv_supported(w, static_cast<const float *>(x), k, n, batch)) {
        detail::check_hip((hipError_t)kk_q4_stream_gemv(w, static_cast<const float *>(x), static_cast<float *>(y), k, n,
                                                        batch, ctx.cus, ctx.stream),
                          "kk_q4_stream_gemv");
        impl.route = "q4_stream_gemv";
    } else if (type == WeightType::q4_0 && kk::q4_bdiag_batch(batch) &&
               kk_q4_bdiag_gemv_supported(w, static_cast<const float *>(x), k, n, batch)) {
        detail::check_hip((hipError_t)kk_q4_bdiag_gemv(w, static_cast<const float *>(x), static_cast<float *>(y), k, n,
                                                       batch, ctx.cus, ctx.stream),
                          "kk_q4_bdiag_gemv");
        impl.route = "q4_bdiag_gemv";
    } else if (type == WeightType::q4_0 && q4_mfma_batch(batch, k % 256 == 0 && ((uintptr_t)w & 15) == 0) &&
               k % 64 == 0 && ((uintptr_t)w & 3) == 0) {
        grow(id, ctx, impl.gemm_workspace, impl.gemm_workspace_size, kk_q4_mfma_gemv_workspace_bytes(k));
        detail::check_hip((hipError_t)kk_q4_mfma_gemv(w, static_cast<const float *>(x), static_cast<float *>(y), k, n,
                                                      batch, impl.gemm_workspace, ctx.cus, ctx.stream),
                          "kk_q4_mfma_gemv");
        impl.route = "q4_mfma_gemv";
    } else {
        detail::check_hip((hipError_t)kk_dense_matmul((int)type, w, static_cast<const float *>(x),
                                                      static_cast<float *>(y), k, n, batch, ctx.stream,
                                                      &impl.route),
                          "kk_dense_matmul");
    }
}

void matmul(Kernel & kernel, int id, void * y, const void * w, const void * x, int k, int n, int batch,
            WeightType type, const float * scales, const float * maximum, int tile) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    validate_shape(y, w, x, k, n, batch, type, tile);
    require(kernel.impl_->id == -1 || kernel.impl_->id == id);
    require(type != WeightType::rowwise_i8 || (scales && maximum));
    // F32 activations and outputs must be element aligned (an F32 array always is).
    require(((uintptr_t)x & 3) == 0 && ((uintptr_t)y & 3) == 0);

    detail::DeviceContext & ctx = detail::context(id);
    Kernel::Impl & impl = *kernel.impl_;
    impl.id = id;
    if (type == WeightType::rowwise_i8) {
        require(((uintptr_t)w & 3) == 0 && ((uintptr_t)scales & 3) == 0 && ((uintptr_t)maximum & 3) == 0);
        if (kk_i8_gemv_rows_supported(k, batch)) {
            detail::check_hip((hipError_t)kk_i8_gemv_rows(static_cast<const float *>(x), static_cast<const int8_t *>(w),
                                                          scales, maximum, static_cast<float *>(y), k, n, ctx.cus,
                                                          ctx.status, ctx.stream),
                              "kk_i8_gemv_rows");
            ctx.status_pending = true;
            impl.route = "i8_rows_gemv";
            detail::last_route = impl.route;
            detail::count_matmul(id);
            return;
        }
        if (kk_i8_gemv_fused_supported(k, batch)) {
            detail::check_hip((hipError_t)kk_i8_gemv_fused(static_cast<const float *>(x),
                                                           static_cast<const int8_t *>(w), scales, maximum,
                                                           static_cast<float *>(y), k, n, batch, ctx.status,
                                                           ctx.stream),
                              "kk_i8_gemv_fused");
            ctx.status_pending = true;
            impl.route = "i8_fused_gemv";
            detail::last_route = impl.route;
            detail::count_matmul(id);
            return;
        }
        grow(id, ctx, impl.i8_workspace, impl.i8_workspace_size, kk_i8_workspace_bytes(k, batch));
        detail::check_hip((hipError_t)kk_i8_quantize(static_cast<const float *>(x), k, batch, impl.i8_workspace,
                                                     ctx.status, ctx.stream),
                          "kk_i8_quantize");
        ctx.status_pending = true;
        detail::check_hip((hipError_t)kk_i8_matmul(impl.i8_workspace, static_cast<const int8_t *>(w), scales,
                                                   maximum, static_cast<float *>(y), k, n, batch, ctx.stream,
                                                   &impl.route),
                          "kk_i8_matmul");
    } else {
        dispatch_dense(impl, ctx, id, y, w, x, k, n, batch, type);
    }
    detail::last_route = impl.route;
    detail::count_matmul(id);
}

// Q4_0 gate/up pair of `batch` columns in one launch (both products and
// SwiGLU), batch 1..16: the batch-1/2 GEMV's, the streamed, block-diagonal or
// LDS-staged GEMV's pair form, whichever takes the shape; none: two GEMVs and
// SwiGLU instead.
enum class Q4PairRoute { none, dot8, stream, bdiag, mfma };

static Q4PairRoute q4_pair_route(const void * w_gate, const void * w_up, const float * x, int k, int n, int batch) {
    if (kk_q4_gemv_pair_swiglu_supported(w_gate, w_up, x, k, n, batch)) return Q4PairRoute::dot8;
    if (kk::q4_stream_batch(batch) && kk_q4_stream_gemv_supported(w_gate, x, k, n, batch) &&
        kk_q4_stream_gemv_supported(w_up, x, k, n, batch))
        return Q4PairRoute::stream;
    if (kk::q4_bdiag_batch(batch) && kk_q4_bdiag_gemv_supported(w_gate, x, k, n, batch) &&
        kk_q4_bdiag_gemv_supported(w_up, x, k, n, batch))
        return Q4PairRoute::bdiag;
    if (q4_mfma_batch(batch, true) && kk_q4_mfma_pair_swiglu_supported(w_gate, w_up, x, k, n, batch))
        return Q4PairRoute::mfma;
    return Q4PairRoute::none;
}

static void run_q4_pair(Q4PairRoute route, Kernel::Impl & impl, detail::DeviceContext & ctx, int id, float * y,
                        const void * w_gate, const void * w_up, const float * x, int k, int n, int batch) {
    switch (route) {
    case Q4PairRoute::dot8:
        // decode: both matrices in one GEMV pass, SwiGLU in its epilogue
        detail::check_hip((hipError_t)kk_q4_gemv_pair_swiglu(w_gate, w_up, x, y, k, n, batch, ctx.stream),
                          "kk_q4_gemv_pair_swiglu");
        impl.route = "q4_gemv_fused_pair_swiglu";
        break;
    case Q4PairRoute::stream:
        detail::check_hip((hipError_t)kk_q4_stream_gemv_pair_swiglu(w_gate, w_up, x, y, k, n, batch, ctx.cus, ctx.stream),
                          "kk_q4_stream_gemv_pair_swiglu");
        impl.route = "q4_stream_pair_swiglu";
        break;
    case Q4PairRoute::bdiag:
        detail::check_hip((hipError_t)kk_q4_bdiag_gemv_pair_swiglu(w_gate, w_up, x, y, k, n, batch, ctx.cus, ctx.stream),
                          "kk_q4_bdiag_gemv_pair_swiglu");
        impl.route = "q4_bdiag_pair_swiglu";
        break;
    case Q4PairRoute::mfma:
        // the LDS-staged MFMA GEMV: one activation prepass, both products and
        // SwiGLU in one launch
        grow(id, ctx, impl.gemm_workspace, impl.gemm_workspace_size, kk_q4_mfma_gemv_workspace_bytes(k));
        detail::check_hip((hipError_t)kk_q4_mfma_gemv_pair_swiglu(w_gate, w_up, x, y, k, n, batch, impl.gemm_workspace,
                                                                  ctx.stream),
                          "kk_q4_mfma_gemv_pair_swiglu");
        impl.route = "q4_mfma_pair_swiglu";
        break;
    case Q4PairRoute::none:
        break;
    }
}

void matmul_swiglu(Kernel & kernel, int id, void * y, const void * w_gate, const void * w_up, const void * x,
                   int k, int n, int batch, WeightType type) {
    std::lock_guard<std::recursive_mutex> lock(detail::mutex());
    require(type == WeightType::f32 || type == WeightType::f16 || type == WeightType::q4_0);
    validate_shape(y, w_gate, x, k, n, batch, type, 16);
    require(w_up != nullptr);
    require(kernel.impl_->id == -1 || kernel.impl_->id == id);
    require(((uintptr_t)x & 3) == 0 && ((uintptr_t)y & 3) == 0);

    detail::DeviceContext & ctx = detail::context(id);
    Kernel::Impl & impl = *kernel.impl_;
    impl.id = id;
    const bool f16_aligned = ((uintptr_t)w_gate & 15) == 0 && ((uintptr_t)w_up & 15) == 0;
    if ((type == WeightType::q4_0 || (type == WeightType::f16 && f16_aligned)) && batch >= gemm_min_batch() &&
        ((uintptr_t)x & 15) == 0) {
        grow(id, ctx, impl.gemm_workspace, impl.gemm_workspace_size, kk_gemm_workspace_bytes(k, n, batch));
        detail::check_hip((hipError_t)kk_gemm_swiglu((int)type, w_gate, w_up, static_cast<const float *>(x),
                                                     static_cast<float *>(y), k, n, batch, impl.gemm_workspace,
                                                     ctx.stream, &impl.route),
                          "kk_gemm_swiglu");
    } else if (type == WeightType::q4_0 &&
               q4_pair_route(w_gate, w_up, static_cast<const float *>(x), k, n, batch) != Q4PairRoute::none) {
        // decode and small batch: both products and SwiGLU in one launch
        run_q4_pair(q4_pair_route(w_gate, w_up, static_cast<const float *>(x), k, n, batch), impl, ctx, id,
                    static_cast<float *>(y), w_gate, w_up, static_cast<const float *>(x), k, n, batch);
    } else if (type == WeightType::q4_0 && batch > 16 &&
               q4_pair_route(w_gate, w_up, static_cast<const float *>(x), k, n, 16) != Q4PairRoute::none &&
               (batch % 16 == 0 || q4_pair_route(w_gate, w_up, static_cast<const float *>(x), k, n, batch % 16) !=
                                       Q4PairRoute::none)) {
        // batches between the small-batch kernels and the GEMM: chunks of 16
        // columns, each in one pair launch (X and Y chunks keep their
        // alignment: K % 32 == 0)
        const char * first = nullptr;
        for (int b0 = 0; b0 < batch; b0 += 16) {
            const int cols = std::min(16, batch - b0);
            const float * xc = reinterpret_cast<const float *>(static_cast<const char *>(x) + (size_t)b0 * k * 4);
            run_q4_pair(q4_pair_route(w_gate, w_up, xc, k, n, cols), impl, ctx, id,
                        reinterpret_cast<float *>(static_cast<char *>(y) + (size_t)b0 * n * 4), w_gate, w_up, xc, k, n,
                        cols);
            if (!first) first = impl.route;
        }
        impl.route = first;
    } else {
        // gate and up rows side by side in the workspace: [batch][2n] F32
        const size_t half = (size_t)batch * n * 4;
        grow(id, ctx, impl.pair_workspace, impl.pair_workspace_size, 2 * half);
        float * gate = static_cast<float *>(impl.pair_workspace);
        float * up = reinterpret_cast<float *>(static_cast<char *>(impl.pair_workspace) + half);
        // each product on matmul's own route for its shape
        dispatch_dense(impl, ctx, id, gate, w_gate, x, k, n, batch, type);
        dispatch_dense(impl, ctx, id, up, w_up, x, k, n, batch, type);
        detail::check_hip((hipError_t)kk_swiglu(y, gate, up, n, batch, n * 4, n * 4, n * 4, 4, ctx.stream),
                          "kk_swiglu");
        impl.route = type == WeightType::q4_0 ? "q4_gemv_pair_swiglu"
                     : type == WeightType::f16 ? "f16_gemv_pair_swiglu"
                                               : "f32_gemv_pair_swiglu";
    }
    detail::last_route = impl.route;
    detail::count_matmul(id);
    detail::count_matmul(id);
}

} // namespace kunlun
