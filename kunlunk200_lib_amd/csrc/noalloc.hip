// kunlun_matmul_noalloc: kunlun_matmul for F32, F16 and Q4_0 weights without
// any device allocation, for callers that cannot allocate (code under HIP
// graph capture, tight serving loops). It takes the routes and kernels of
// kunlun::matmul (matmul.cpp); the routes that need device memory beyond the
// inputs and outputs -- the fp16-MFMA prefill GEMM (fp16 activations and row
// scales, kk_gemm_workspace_bytes) and the LDS-staged Q4_0 MFMA GEMV
// (activation fragments, kk_q4_mfma_gemv_workspace_bytes) -- take it from `scratch`, a
// file-scope device array of kScratchBytes, instead of a Kernel's workspace.
//
// Every GPU the library runs on holds its own copy of the array until the
// process ends. Host code reaches it only through the per-device address
// hipGetSymbolAddress returns (taken once per device, with that device
// current, on the entry point's first call there); the array's name in host
// code is a host-side stand-in, not a device address. The kernels write every
// scratch byte they read in the same call, so nothing needs clearing, but
// calls that overlap on one GPU share the array and race.
#include "launch.h"
#include "runtime_internal.h"

#include <kunlun/k200_c.h>

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <mutex>

namespace {

constexpr size_t kScratchBytes = size_t(16) << 20;   // 16 MiB: batch * K_pad <= 8M activations on the GEMM

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct DeviceScratch {
    std::once_flag once;
    hipError_t status = hipErrorNotInitialized;
    void *ptr = nullptr;   // this device's copy of `scratch`
    int cus = 0;
};
DeviceScratch g_scratch[kunlun::max_devices];

// Called once per device, with the device current.
void set_up(DeviceScratch &d) {
    void *ptr = nullptr;
    hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    int cus = 0;
    if (rc == hipSuccess) {
        int device = 0;
        rc = hipGetDevice(&device);
        if (rc == hipSuccess) rc = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    }
    if (rc == hipSuccess && (ptr == nullptr || (reinterpret_cast<uintptr_t>(ptr) & 255) || cus <= 0))
        rc = hipErrorInvalidSymbol;
    d.ptr = ptr;
    d.cus = cus;
    d.status = rc;
}

int too_large(size_t need) {
    std::fprintf(stderr,
                 "kunlun_matmul_noalloc: this call needs %zu bytes of scratch, above the fixed %zu "
                 "(KUNLUN_NOALLOC_SCRATCH_BYTES); use kunlun_matmul\n",
                 need, kScratchBytes);
    return KUNLUN_NOALLOC_TOO_LARGE;
}

// kunlun_matmul's route for at most 16 columns (X 16-byte aligned or not),
// with its scratch in the device's array
hipError_t small_batch(DeviceScratch &d, int type, const void *w, const float *xf, float *yf, int k, int n, int batch,
                       uintptr_t wa, hipStream_t s, const char **taken) {
    const uintptr_t xa = reinterpret_cast<uintptr_t>(xf);
    if ((type == 0 || type == 1) && kk::dense_mfma_batch(batch) && (wa & 15) == 0 && (xa & 15) == 0) {
        *taken = type == 1 ? "f16_mfma_gemv" : "f32_mfma_gemv";
        return static_cast<hipError_t>(kk_dense_mfma_gemv(type, w, xf, yf, k, n, batch, s));
    }
    if (type == 2 && kk::q4_stream_batch(batch) && kk_q4_stream_gemv_supported(w, xf, k, n, batch)) {
        *taken = "q4_stream_gemv";
        return static_cast<hipError_t>(kk_q4_stream_gemv(w, xf, yf, k, n, batch, d.cus, s));
    }
    if (type == 2 && kk::q4_bdiag_batch(batch) && kk_q4_bdiag_gemv_supported(w, xf, k, n, batch)) {
        *taken = "q4_bdiag_gemv";
        return static_cast<hipError_t>(kk_q4_bdiag_gemv(w, xf, yf, k, n, batch, d.cus, s));
    }
    if (type == 2 && kk::q4_mfma_batch(batch, k % 256 == 0 && (wa & 15) == 0) && k % 64 == 0 && (wa & 3) == 0) {
        const size_t need = kk_q4_mfma_gemv_workspace_bytes(k);
        if (need > kScratchBytes) return static_cast<hipError_t>(too_large(need));
        *taken = "q4_mfma_gemv";
        return static_cast<hipError_t>(kk_q4_mfma_gemv(w, xf, yf, k, n, batch, d.ptr, d.cus, s));
    }
    return static_cast<hipError_t>(kk_dense_matmul(type, w, xf, yf, k, n, batch, s, taken));
}

} // namespace

extern "C" int kunlun_matmul_noalloc(int device, void *y, const void *w, const void *x, int k, int n, int batch,
                                     int type, void *stream, const char **route) {
    static_assert(kScratchBytes == KUNLUN_NOALLOC_SCRATCH_BYTES, "header and array agree");
    if (route) *route = nullptr;
    // kunlun::matmul's argument rules (reference src/k200.cpp:271-275) for the
    // types this entry point takes, as a status instead of an abort
    if (type != 0 && type != 1 && type != 2) return KUNLUN_NOALLOC_INVALID;
    if (device < 0 || device >= kunlun::max_devices || !y || !w || !x || k <= 0 || k > 16384 || k % 32 ||
        n <= 0 || batch <= 0 || n > INT32_MAX / batch || k > INT32_MAX / batch ||
        static_cast<size_t>(n) * batch > INT32_MAX / 4 || static_cast<size_t>(k) * batch > INT32_MAX / 4)
        return KUNLUN_NOALLOC_INVALID;
    const size_t row_bytes = type == 0 ? static_cast<size_t>(k) * 4
                             : type == 1 ? static_cast<size_t>(k) * 2 : static_cast<size_t>(k) / 32 * 18;
    if (static_cast<size_t>(n) > INT32_MAX / row_bytes) return KUNLUN_NOALLOC_INVALID;
    if ((reinterpret_cast<uintptr_t>(x) & 3) || (reinterpret_cast<uintptr_t>(y) & 3)) return KUNLUN_NOALLOC_INVALID;

    hipError_t rc = hipSetDevice(device);
    if (rc != hipSuccess) return rc;
    DeviceScratch &d = g_scratch[device];
    std::call_once(d.once, set_up, std::ref(d));
    if (d.status != hipSuccess) return d.status;

    const hipStream_t s = static_cast<hipStream_t>(stream);
    const float *xf = static_cast<const float *>(x);
    float *yf = static_cast<float *>(y);
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w), xa = reinterpret_cast<uintptr_t>(x);
    const char *taken = nullptr;
    const bool gemm = (type == 2 || (type == 1 && (wa & 15) == 0)) && batch >= kk::gemm_min_batch() && (xa & 15) == 0;
    if (gemm) {
        const size_t need = kk_gemm_workspace_bytes(k, n, batch);
        if (need > kScratchBytes) return too_large(need);
        rc = static_cast<hipError_t>(kk_gemm(type, w, xf, yf, k, n, batch, d.ptr, s, &taken));
    } else {
        // kunlun_matmul's small-batch routes; above 16 columns, chunks of 16
        // (as kunlun_matmul runs them), in stream order on the one array
        for (int b0 = 0; b0 < batch && rc == hipSuccess; b0 += 16) {
            const int bc = std::min(16, batch - b0);
            const char *chunk_route = nullptr;
            rc = small_batch(d, type, w, xf + static_cast<size_t>(b0) * k, yf + static_cast<size_t>(b0) * n, k, n, bc,
                             wa, s, &chunk_route);
            if (!taken) taken = chunk_route;
        }
        if (rc == static_cast<hipError_t>(KUNLUN_NOALLOC_TOO_LARGE)) return rc;
    }
    if (route) *route = taken;
    return rc;
}
