// Internal C ABI between the host runtime (C++) and the HIP kernel launchers.
// Each launcher validates that its grid fits the shapes it is given, submits
// to `stream` and returns 0 or a hipError_t. `route` (optional) receives a
// static string naming the kernel path taken.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

extern "C" {

// Y[batch,n] = X[batch,k] * W[n,k]^T for F32 (type 0), F16 (1) and Q4_0 (2)
// weights, F32 activations and outputs, F32 accumulation.
int kk_dense_matmul(int type, const void *w, const float *x, float *y, int k, int n, int batch,
                    hipStream_t stream, const char **route);


// Prefill GEMM on fp16 MFMA for Q4_0 (type 2) and F16 (type 1) weights. The
// workspace (kk_gemm_workspace_bytes) holds the fp16 activations and their
// row scales.
size_t kk_gemm_workspace_bytes(int k, int n, int batch);
int kk_gemm(int type, const void *w, const float *x, float *y, int k, int n, int batch, void *workspace,
            hipStream_t stream, const char **route);

// Y[batch,n] = SiLU(X W_gate^T) * (X W_up^T) on the prefill GEMM (same types,
// workspace and alignment rules as kk_gemm; both matrices [n,k]).
int kk_gemm_swiglu(int type, const void *w_gate, const void *w_up, const float *x, float *y, int k, int n,
                   int batch, void *workspace, hipStream_t stream, const char **route);

// Y[batch,n] = SiLU(X W_gate^T) * (X W_up^T) for Q4_0 weights at batch 1..2
// in one pass (the q4_gemv_dot8 GEMV with both matrices per wave and the
// swiglu element function as its epilogue). _supported tells whether these
// arguments qualify: K % 64 == 0, K <= 16384, 4-byte aligned weights,
// 16-byte aligned X, and the default GEMV kernel selection.
int kk_q4_gemv_pair_swiglu_supported(const void *w_gate, const void *w_up, const float *x, int k, int n, int batch);
int kk_q4_gemv_pair_swiglu(const void *w_gate, const void *w_up, const float *x, float *y, int k, int n, int batch,
                           hipStream_t stream);

// y = SiLU(gate) * up over `rows` rows of `width` contiguous values of
// `bytes` (4: F32, 2: F16) each; strides in bytes. F32 intermediates.
int kk_swiglu(void *y, const void *gate, const void *up, int width, int rows, int gate_stride, int up_stride,
              int output_stride, int bytes, hipStream_t stream);

// Q4_0 GEMV for batch 1..16 on fp16 MFMA (one pass over W): K % 64 == 0,
// 4-byte aligned weights; workspace of kk_q4_mfma_gemv_workspace_bytes(k)
// holds the activation fragments; `cus` sizes the grid.
size_t kk_q4_mfma_gemv_workspace_bytes(int k);
int kk_q4_mfma_gemv(const void *w, const float *x, float *y, int k, int n, int batch, void *workspace, int cus,
                    hipStream_t stream);

// The gate/up pair on the LDS-staged Q4_0 MFMA GEMV (K % 512 == 0, 16-byte
// aligned weights and X, batch <= 16): one activation prepass into
// `workspace` (kk_q4_mfma_gemv_workspace_bytes), then both products with
// SwiGLU in the epilogue: y = [batch][n] = SiLU(X w_gate^T) * (X w_up^T).
int kk_q4_mfma_pair_swiglu_supported(const void *w_gate, const void *w_up, const float *x, int k, int n, int batch);
int kk_q4_mfma_gemv_pair_swiglu(const void *w_gate, const void *w_up, const float *x, float *y, int k, int n,
                                int batch, void *workspace, hipStream_t stream);

// Q4_0 GEMV for batch 1..16 on fp16 MFMA with block-diagonal activation
// operands (one pass over W, lanes streaming whole block pairs, no
// workspace): K % 64 == 0, 4-byte aligned weights, 16-byte aligned X, and
// the activation fragments of all of K in LDS (ceil(K/1024)*4 steps x
// ceil(batch/4) x 4480 bytes <= 160 KiB); `cus` sizes the grid.
int kk_q4_bdiag_gemv_supported(const void *w, const float *x, int k, int n, int batch);
int kk_q4_bdiag_gemv(const void *w, const float *x, float *y, int k, int n, int batch, int cus, hipStream_t stream);
// The gate/up pair in one launch, SwiGLU in its epilogue: y = [batch][n] =
// SiLU(X w_gate^T) * (X w_up^T) (kk::swiglu_value).
int kk_q4_bdiag_gemv_pair_swiglu(const void *w_gate, const void *w_up, const float *x, float *y, int k, int n,
                                 int batch, int cus, hipStream_t stream);

// Q4_0 GEMV for batch 1..8 at K = 4096 on fp16 MFMA, one pass over W with
// weight rows streamed through per-wave LDS (no workspace): 16-byte aligned
// weights and X; `cus` sizes the grid.
int kk_q4_stream_gemv_supported(const void *w, const float *x, int k, int n, int batch);
int kk_q4_stream_gemv(const void *w, const float *x, float *y, int k, int n, int batch, int cus, hipStream_t stream);
// The gate/up pair in one launch, SwiGLU in its epilogue: y = [batch][n] =
// SiLU(X w_gate^T) * (X w_up^T) (kk::swiglu_value).
int kk_q4_stream_gemv_pair_swiglu(const void *w_gate, const void *w_up, const float *x, float *y, int k, int n,
                                  int batch, int cus, hipStream_t stream);

// F32 (type 0) / F16 (type 1) GEMV for batch 1..16 on fp32 MFMA, one pass over
// W; 16-byte aligned weights and activations.
int kk_dense_mfma_gemv(int type, const void *w, const float *x, float *y, int k, int n, int batch,
                       hipStream_t stream);

// Elementwise F32 op over `count` values: 0 add, 1 multiply (b of b_count
// values repeated), 2 silu, 3 rms_norm of each `width` row (eps =
// parameter), 4 scale by parameter.
int kk_elementwise(float *y, const float *a, const float *b, int count, int width, int b_count, int op,
                   float parameter, hipStream_t stream);

// Native Q4 layout (256-byte aligned): offset of the FP16 scales, and the
// exact GEMV Y[batch,n] = X[batch,k] W^T with X F32 (x_f16 = 0, 4-byte
// aligned) or F16 (x_f16 = 1, 2-byte aligned), Y F32 (4-byte aligned).
size_t kk_native_q4_payload_bytes(int k, int n);
int kk_native_q4_gemv(const void *weights, const void *x, int x_f16, float *y, int k, int n, int batch,
                      hipStream_t stream);

// Common Q4 ABI v1 (layout 1, scale order 1; weights 256-byte aligned).
// M = 1 per-tensor two-component int8 quantization of X[k] (F32 or F16) into
// the view buffer `values` (4*kp + 1024 bytes) and `params` (16 floats).
int kk_common_quant_pair(const void *x, int x_f16, int k, int kp, void *values, void *params, hipStream_t stream);
// M > 1 per-row int8 quantization of `rows` rows (zero rows up to
// defined_rows, a multiple of 32): values [defined_rows][kp], params
// [defined_rows][16], and the same codes in the GEMM's operand order in
// `tiled` (defined_rows * kp bytes).
int kk_common_quant_rows(const void *x, int x_f16, int k, int kp, int rows, int defined_rows, void *values,
                         void *params, void *tiled, hipStream_t stream);
// M = 1 GEMV over one weight (w1 null) or two sharing the activations.
// mode 0: act = the quantized view, params its scales; mode 1: act = X,
// quantized in the kernel, the view written to view_values / params; mode 2:
// act = X, exact.
size_t kk_common_gemv_lds_bytes(int kp, int exact);
int kk_common_gemv(const void *w0, float *y0, const void *w1, float *y1, const void *act, int mode, int x_f16,
                   void *params, void *view_values, int k, int kp, int n, int np, hipStream_t stream);
// M > 1 (rows <= 128) GEMM on quantized rows (codes in the tiled operand
// order of kk_common_quant_rows, row scales at row_scales[r*16]).
int kk_common_gemm(const void *w, const void *tiled, const void *row_scales, float *y, int rows, int defined_rows,
                   int kp, int n, int np, hipStream_t stream);

// rowwise_i8 at batch 1..8 with batch * K <= 16384, quantization and product
// in one launch (no workspace); the non-finite activation flag goes to
// `status` as kk_i8_quantize's does.
// Batch-1 rowwise_i8 (K % 32 == 0, K <= 4096): each wave quantizes X itself and
// streams whole weight rows with coalesced loads; int32 dot products by v_dot4.
int kk_i8_gemv_rows_supported(int k, int batch);
int kk_i8_gemv_rows(const float *x, const int8_t *w, const float *scales, const float *maxima, float *y, int k, int n,
                    int cus, int *status, hipStream_t stream);
int kk_i8_gemv_fused_supported(int k, int batch);
int kk_i8_gemv_fused(const float *x, const int8_t *w, const float *scales, const float *maxima, float *y, int k, int n,
                     int batch, int *status, hipStream_t stream);

// Bytes of device workspace kk_i8_quantize needs for `count` activations.
size_t kk_i8_workspace_bytes(int k, int batch);
// Two-pass per-tensor INT8 quantization of X[batch,k] into `workspace`
// (codes and maxima). Sets *status (device memory) to 1 on a non-finite value.
int kk_i8_quantize(const float *x, int k, int batch, void *workspace, int *status,
                   hipStream_t stream);
// Y = (P*max0/127 + R*max1/127) * scales[n] from exact int32 dot products of
// the quantized activations in `workspace` with int8 weight rows W[n,k].
int kk_i8_matmul(const void *workspace, const int8_t *w, const float *scales, const float *maxima,
                 float *y, int k, int n, int batch, hipStream_t stream, const char **route);

}
