// Route and tile selection knobs of the matmul path. Each knob is read from
// its environment variable once, the first time any knob is used, and can be
// overridden at run time (kunlun_set_tuning in the C ABI). A value of -1
// means "not set": the dispatcher then uses its built-in choice.
#pragma once

namespace kk {

enum Knob {
    kGemmMinBatch,        // KUNLUN_GEMM_MIN_BATCH: smallest batch on the prefill GEMM
    kQ4MfmaMin,           // KUNLUN_Q4_MFMA_MIN / _MAX: batch range of the Q4_0 MFMA GEMV
    kQ4MfmaMax,
    kDenseMfmaMin,        // KUNLUN_DENSE_MFMA_MIN / _MAX: batch range of the F32/F16 MFMA GEMV
    kDenseMfmaMax,
    kGemmTile,            // KUNLUN_GEMM_TILE=BMxWN: Q4_0 LDS GEMM tile, stored as BM * 1000 + WN
    kGemmBn,              // KUNLUN_GEMM_BN=64|128: register-staged GEMM tile width
    kGemvGeneral,         // KUNLUN_GEMV_GENERAL=1: every GEMV on the general kernel
    kI8FusedQuantLimit,   // KUNLUN_I8_FUSED_QUANT_LIMIT: single-workgroup quantizer limit
    kQ4Bdiag,             // KUNLUN_Q4_BDIAG=0: the Q4_0 MFMA GEMV batch range on the LDS-staged kernels instead
    kDenseStream,         // KUNLUN_DENSE_STREAM=0: F16 batch 2..8 at K <= 4096 on the K-split kernel, not the streamed one
    kQ4StreamMin,         // KUNLUN_Q4_STREAM_MIN: smallest batch (default 5, up to 8) on the streamed Q4_0 GEMV at K = 4096
    kKnobCount
};

// Current value of a knob (-1 when unset).
int tuning(Knob knob);
// Value of a knob, or `fallback` when it is unset.
inline int tuning_or(Knob knob, int fallback) {
    const int v = tuning(knob);
    return v < 0 ? fallback : v;
}

} // namespace kk
