/* C ABI of the KunlunK200 matmul path for MI355X (gfx950).
 *
 * Plain pointers and sizes, no C++ or HIP types in the signatures, so that
 * ctypes, cgo, JNI or any C caller binds the library directly. Each function
 * forwards to the C++ drop-in surface in <kunlun/k200.h> and keeps its
 * argument meaning and fail-fast error behaviour: invalid arguments and device
 * errors print a diagnostic and abort(), as the reference does
 * (reference src/k200.cpp:53-62). Functions that only exist in this library
 * say so.
 *
 * All device pointers are HIP device addresses. Work is submitted to one HIP
 * stream per device, owned by the library (kunlun_stream()).
 */
#ifndef KUNLUN_K200_C_H
#define KUNLUN_K200_C_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque handle that owns one kunlun::Kernel (reference include/kunlun/k200.h:62-88). */
typedef struct kunlun_kernel kunlun_kernel;
/* Opaque handle that owns one kunlun::NativeQ4Workspace (reference include/kunlun/k200.h:208-219). */
typedef struct kunlun_native_q4_workspace kunlun_native_q4_workspace;
/* Opaque handles owning kunlun::CommonQ4Weight, CommonQ4Workspace and
 * CommonQ4ActivationLease (reference include/kunlun/k200.h:249-326). */
typedef struct kunlun_common_q4_weight kunlun_common_q4_weight;
typedef struct kunlun_common_q4_workspace kunlun_common_q4_workspace;
typedef struct kunlun_common_q4_lease kunlun_common_q4_lease;
/* kunlun::CommonQ4Info, same fields and types (reference include/kunlun/k200.h:227-231). */
typedef struct {
    uint32_t abi_version, quant_type, layout, scale_order;
    int k, n, kp, np, device;
    size_t scale_offset, payload_bytes;
} kunlun_common_q4_info;

/* Copy directions, same values as kunlun::CopyKind (reference include/kunlun/k200.h:18). */
enum { KUNLUN_HOST_TO_DEVICE = 0, KUNLUN_DEVICE_TO_HOST = 1, KUNLUN_DEVICE_TO_DEVICE = 2 };
/* Weight formats, same values as kunlun::WeightType (reference include/kunlun/k200.h:40). */
enum { KUNLUN_F32 = 0, KUNLUN_F16 = 1, KUNLUN_Q4_0 = 2, KUNLUN_ROWWISE_I8 = 3, KUNLUN_Q6_K = 4 };

/* runtime_mutex() lock/unlock (reference include/kunlun/k200.h:10). Recursive. */
void kunlun_lock(void);
void kunlun_unlock(void);
/* check() / require() (reference include/kunlun/k200.h:11,14): abort on failure. */
void kunlun_check(int status);
void kunlun_require(int condition);
/* diagnostic_tensor() (reference include/kunlun/k200.h:13); dimensions may be NULL. */
void kunlun_diagnostic_tensor(const char *name, const int64_t *dimensions);
/* device_count() (reference include/kunlun/k200.h:15); returns a HIP status. */
int kunlun_device_count(int *count);
/* select() (reference include/kunlun/k200.h:16). */
void kunlun_select(int device);
/* wait() (reference include/kunlun/k200.h:17): completes all work on the
 * selected device (hipDeviceSynchronize); returns a HIP status. */
int kunlun_wait(void);
/* copy() (reference include/kunlun/k200.h:19); kind is a KUNLUN_*_TO_* value.
 * Runs after the library's submitted work and completes before returning. */
int kunlun_copy(void *dst, const void *src, size_t bytes, int kind);
/* peer() (reference include/kunlun/k200.h:20). */
void kunlun_peer(int dst_device, void *dst, int src_device, const void *src, size_t bytes);
/* allocate() / release() / allocated_bytes() (reference include/kunlun/k200.h:21-23). */
void *kunlun_allocate(int device, size_t bytes);
void kunlun_release(int device, void *ptr, size_t bytes);
size_t kunlun_allocated_bytes(int device);

/* Kernel::Kernel() / Kernel::~Kernel() (reference include/kunlun/k200.h:62-66). */
kunlun_kernel *kunlun_kernel_create(void);
void kunlun_kernel_destroy(kunlun_kernel *kernel);

/* aligned() / packed_i8_size() / packed_i8_scales() / packed_i8_maxima()
 * (reference include/kunlun/k200.h:90-93). */
size_t kunlun_aligned(size_t bytes);
size_t kunlun_packed_i8_size(int k, int rows);
float *kunlun_packed_i8_scales(void *weights, int k, int rows);
float *kunlun_packed_i8_maxima(void *weights, int k, int rows);
/* upload_i8_rows() (reference include/kunlun/k200.h:95-96); input is host memory. */
void kunlun_upload_i8_rows(int device, void *weights, int k, int rows,
                           int first_row, int count, const float *input);

/* matmul() (reference include/kunlun/k200.h:103-105). Submits Y[batch,n] =
 * X[batch,k] * W[n,k]^T; kunlun_select(device) + kunlun_wait() completes it.
 * scales/maxima are required for KUNLUN_ROWWISE_I8 and ignored otherwise;
 * tile must be 1 or 16 (accepted for compatibility, no effect on results). */
void kunlun_matmul(kunlun_kernel *kernel, int device, void *y, const void *w, const void *x,
                   int k, int n, int batch, int type,
                   const float *scales, const float *maxima, int tile);

/* Elementwise ops, same values as kunlun::ElementwiseOp (reference include/kunlun/k200.h:41). */
enum { KUNLUN_EW_ADD = 0, KUNLUN_EW_MULTIPLY = 1, KUNLUN_EW_SILU = 2, KUNLUN_EW_RMS_NORM = 3, KUNLUN_EW_SCALE = 4 };
/* elementwise() (reference include/kunlun/k200.h:106-107): F32 op over count
 * values, completed before returning; invalid arguments abort. */
void kunlun_elementwise(kunlun_kernel *kernel, int device, void *y, const void *a, const void *b, int count,
                        int width, int b_count, int op, float parameter);

/* Element types of SwiGLU, same values as kunlun::InputType (reference include/kunlun/k200.h:132). */
enum { KUNLUN_INPUT_F32 = 0, KUNLUN_INPUT_F16 = 1 };
/* swiglu_reason() (reference include/kunlun/k200.h:192) on the SwiGLULayout
 * {width, rows, gate_stride, up_stride, output_stride, type}: "" when
 * supported, else the first rule broken ("type", "shape", "stride",
 * "byte extent"). */
const char *kunlun_swiglu_reason(int width, int rows, int gate_stride, int up_stride, int output_stride, int type);
/* swiglu() (reference include/kunlun/k200.h:197-199): y = SiLU(gate) * up
 * with F32 intermediates, completed before returning. Returns 1, or 0 when
 * the layout or pointer contract is not met (nothing submitted). */
int kunlun_swiglu(kunlun_kernel *kernel, int device, void *y, size_t y_bytes, const void *gate,
                  size_t gate_bytes, const void *up, size_t up_bytes, int width, int rows,
                  int gate_stride, int up_stride, int output_stride, int type);

/* Native Q4 layout (reference include/kunlun/k200.h:127-131): 1/0 for
 * native_q4_layout_supported, bytes of the layout (0 when unsupported), host
 * repack (1 on success, 0 for a bad shape, short buffer or overlap), and
 * pack + upload completed before returning (invalid arguments abort). */
int kunlun_native_q4_layout_supported(int k, int n);
size_t kunlun_native_q4_size(int k, int n);
int kunlun_pack_native_q4(void *destination, size_t bytes, const void *q4, int k, int n);
void kunlun_upload_native_q4(int device, void *weights, const void *q4, int k, int n);
/* native_q4_reason() (reference include/kunlun/k200.h:203); type is a KUNLUN_INPUT_* value. */
const char *kunlun_native_q4_reason(int k, int n, int batch, int type);
kunlun_native_q4_workspace *kunlun_native_q4_workspace_create(void);
void kunlun_native_q4_workspace_destroy(kunlun_native_q4_workspace *workspace);
/* NativeQ4Workspace::statistics(): out = {accelerated, fallback,
 * hbm_workspace_bytes, l3_workspace_bytes}. */
void kunlun_native_q4_statistics(const kunlun_native_q4_workspace *workspace, size_t out[4]);
/* native_q4_matmul() (reference include/kunlun/k200.h:223-224): completes
 * before returning; 1 where the reference takes its accelerated route, else 0. */
int kunlun_native_q4_matmul(kunlun_native_q4_workspace *workspace, int device, void *y, const void *weights,
                            const void *input, int k, int n, int batch, int type);

/* Common Q4 ABI v1 (reference include/kunlun/k200.h:226-335, 381-383). Each
 * function forwards to the C++ entry of the same name; type is a
 * KUNLUN_INPUT_* value. */
int kunlun_common_q4_supported(int k, int n);
size_t kunlun_common_q4_size(int k, int n);
/* CommonQ4Weight(device, k, n, storage, bytes); storage NULL allocates. */
kunlun_common_q4_weight *kunlun_common_q4_weight_create(int device, int k, int n, void *storage, size_t bytes);
void kunlun_common_q4_weight_destroy(kunlun_common_q4_weight *weight);
void kunlun_common_q4_weight_info(const kunlun_common_q4_weight *weight, kunlun_common_q4_info *out);
void *kunlun_common_q4_weight_data(const kunlun_common_q4_weight *weight);
void kunlun_common_q4_weight_upload(kunlun_common_q4_weight *weight, const void *q4, size_t bytes);
/* counts = {uploads, upload_bytes}, ms = {pack_ms, upload_ms}. */
void kunlun_common_q4_weight_statistics(const kunlun_common_q4_weight *weight, size_t counts[2], double ms[2]);
kunlun_common_q4_workspace *kunlun_common_q4_workspace_create(void);
void kunlun_common_q4_workspace_destroy(kunlun_common_q4_workspace *workspace);
/* out = {paths[0..7], calls, chunks, hbm_workspace_bytes, l3_workspace_bytes, slice_bytes}. */
void kunlun_common_q4_workspace_statistics(const kunlun_common_q4_workspace *workspace, size_t out[13]);
/* out = {prepare_calls, quantized_chunks, quant_kernel_launches, prepared_matmuls,
 * prepared_chunks, invalidations, rejected_calls, hbm_activation_bytes,
 * quantization_ns, preparation_ns}. */
void kunlun_common_q4_activation_statistics(const kunlun_common_q4_workspace *workspace, uint64_t out[10]);
/* out = {baseline_sd_calls, stream_sd_calls, shape_fallbacks, resident_l1d_bytes}. */
void kunlun_common_q4_mac_statistics(const kunlun_common_q4_workspace *workspace, size_t out[4]);
/* quantization(): device pointers and {rows, kp, components}. */
void kunlun_common_q4_quantization(const kunlun_common_q4_workspace *workspace, const void **values,
                                   const void **scales, int out[3]);
void kunlun_common_q4_matmul(kunlun_common_q4_workspace *workspace, int device, void *y,
                             const kunlun_common_q4_weight *weight, const void *input, int m, int type);
kunlun_common_q4_lease *kunlun_common_q4_lease_create(void);
void kunlun_common_q4_lease_destroy(kunlun_common_q4_lease *lease);
void kunlun_common_q4_lease_reset(kunlun_common_q4_lease *lease);
int kunlun_common_q4_lease_matches(const kunlun_common_q4_lease *lease, int device, int k, int rows, int type,
                                   uint64_t generation);
size_t kunlun_common_q4_lease_chunks(const kunlun_common_q4_lease *lease);
/* chunk(index): device pointers, ints = {first, rows, padded_rows, kp,
 * components}, bytes = {values_bytes, scales_bytes}. */
void kunlun_common_q4_lease_chunk(const kunlun_common_q4_lease *lease, size_t index, const void **values,
                                  const void **scales, int ints[5], size_t bytes[2]);
int kunlun_common_q4_prepare(kunlun_common_q4_workspace *workspace, int device, const void *input, int k, int rows,
                             int type, uint64_t generation, kunlun_common_q4_lease *lease);
int kunlun_common_q4_matmul_shared(kunlun_common_q4_workspace *workspace, int device, void *y,
                                   const kunlun_common_q4_weight *weight, const kunlun_common_q4_lease *lease,
                                   uint64_t generation);
int kunlun_common_q4_matmul_pair(kunlun_common_q4_workspace *workspace, int device, void *y0, void *y1,
                                 const kunlun_common_q4_weight *w0, const kunlun_common_q4_weight *w1,
                                 const kunlun_common_q4_lease *lease, uint64_t generation);
/* out = {calls, declined, l3_partial_bytes}; status as kunlun::CommonQ4PairStatus. */
void kunlun_common_q4_pair_statistics(const kunlun_common_q4_workspace *workspace, size_t out[3]);
int kunlun_common_q4_pair_last_status(const kunlun_common_q4_workspace *workspace);

/* statistics() (reference include/kunlun/k200.h:345-349) as four counters:
 * out[0..1] = matmul submissions on devices 0 and 1, out[2] = peer copies,
 * out[3] = peer bytes. */
void kunlun_statistics(size_t out[4]);
/* version() (reference include/kunlun/k200.h:350). */
const char *kunlun_version(void);

/* --- Functions of this library without a counterpart in the reference --- */

/* Matmul submissions on any device (statistics() only reports devices 0 and 1). */
size_t kunlun_matmul_count(int device);
/* The hipStream_t the library submits to on `device`, as void*. Callers that
 * time work with HIP events record them on this stream. */
void *kunlun_stream(int device);
/* Name of the kernel route the last matmul on `kernel` took (for tests and
 * profiling, e.g. "q4_gemv_dot8"); NULL before the first call. */
const char *kunlun_kernel_route(const kunlun_kernel *kernel);
/* matmul_swiglu(): Y[batch,n] = SiLU(X W_gate^T) * (X W_up^T) for two [n,k]
 * weights of one type (KUNLUN_F32, KUNLUN_F16, KUNLUN_Q4_0), with matmul()'s
 * argument rules. The reference computes this with two matmul calls and
 * swiglu; here batch >= 64 fuses both products and the SwiGLU into one GEMM,
 * and Q4_0 at batch 1..2 into one GEMV pass.
 * Submits; kunlun_select(device) + kunlun_wait() completes it. */
void kunlun_matmul_swiglu(kunlun_kernel *kernel, int device, void *y, const void *w_gate, const void *w_up,
                          const void *x, int k, int n, int batch, int type);
/* Route and tile knobs of matmul. Each knob is named by its environment
 * variable (KUNLUN_GEMM_MIN_BATCH, KUNLUN_Q4_MFMA_MIN, KUNLUN_Q4_MFMA_MAX,
 * KUNLUN_DENSE_MFMA_MIN, KUNLUN_DENSE_MFMA_MAX, KUNLUN_GEMM_TILE (BMxWN),
 * KUNLUN_GEMM_BN, KUNLUN_GEMV_GENERAL, KUNLUN_I8_FUSED_QUANT_LIMIT,
 * KUNLUN_Q4_BDIAG, KUNLUN_DENSE_STREAM,
 * KUNLUN_Q4_STREAM_MIN), which
 * the library reads once, at the first matmul. kunlun_set_tuning sets a knob
 * from text in the variable's syntax; a NULL value restores the value read
 * from the environment. Returns 0, or -1 for an unknown name or a malformed
 * value. kunlun_get_tuning returns the current value (-1: unset, the
 * built-in choice) or -2 for an unknown name. */
int kunlun_set_tuning(const char *name, const char *value);
int kunlun_get_tuning(const char *name);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): kunlun_matmul for KUNLUN_F32, KUNLUN_F16 and KUNLUN_Q4_0
 * weights on the same routes and kernels, that allocates nothing. The
 * scratch of the routes that need it (the batch >= 64 fp16-MFMA GEMM and the
 * Q4_0 MFMA GEMV) is a fixed device array of KUNLUN_NOALLOC_SCRATCH_BYTES per
 * GPU, held until the process ends; a call that needs more returns
 * KUNLUN_NOALLOC_TOO_LARGE (the GEMM needs about 2 * batch * K bytes, so
 * batch * K <= 8M fits). The caller passes device pointers for y, w and x
 * and the stream to submit on (NULL: the null stream); `route` (optional)
 * receives the kernel route's name. Makes `device` current for the calling
 * thread and takes no library lock; completion is the caller's (stream or
 * device synchronization). Calls that overlap on one GPU share its scratch
 * array and race. Returns 0, KUNLUN_NOALLOC_INVALID for an argument
 * kunlun_matmul would reject or an unsupported type (rowwise INT8), or a
 * HIP status. */
#define KUNLUN_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
enum { KUNLUN_NOALLOC_INVALID = -1, KUNLUN_NOALLOC_TOO_LARGE = -2 };
int kunlun_matmul_noalloc(int device, void *y, const void *w, const void *x, int k, int n, int batch, int type,
                          void *stream, const char **route);

#ifdef __cplusplus
}
#endif

#endif /* KUNLUN_K200_C_H */
