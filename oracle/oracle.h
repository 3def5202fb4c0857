/* CPU oracle for the KunlunK200 matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * library's CPU reference and host arithmetic, used as the checker. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product library never links or calls it.
 *
 * Each function names the reference file:line it follows (paths relative to
 * the reference repository root). How each one is pinned:
 *   orc_xorshift32, orc_fixture_q4, orc_fixture_input, orc_gold,
 *   orc_i8_activation      - against the reference's own CPU oracle header
 *                            (bench/native-q4-reference.h) compiled into
 *                            oracle/_ref, and committed golden vectors;
 *   orc_half_to_float      - all 65536 bit patterns against numpy float16;
 *   orc_float_to_half      - all finite f16 values round-trip, midpoints and
 *                            a 2^20-sample sweep against numpy float16 (RNE);
 *   orc_bench_weights      - closed form: the Q4 bytes decode to the F32
 *                            weights exactly (library-bench design);
 *   orc_fused_bench_weights- closed form: gold of row r equals row r%16;
 *   orc_q4_decode          - library-bench and fused-bench closed forms above;
 *   orc_q4_quantize        - PARITY UNPINNED at bit level (ggml is absent):
 *                            pinned by properties only (round-trip error
 *                            bound, extreme element exact, nibble range);
 *   orc_i8_rows            - brute-force nearest-integer search with ties
 *                            away from zero, and the reference header's
 *                            one-component Activation on single rows;
 *   orc_i8_dots            - brute-force small cases and numpy int64 matmul;
 *   orc_i8_combine         - hand-computed known answers;
 *   orc_matvec_f32         - within f32 accumulation error of orc_gold;
 *   orc_swiglu_value       - every non-finite case of the reference rule
 *                            worked by hand, and finite inputs within a few
 *                            ulp of the FP64 closed form g*u/(1+exp(-g));
 *   orc_swiglu             - strided rows, F16 rounding and aliasing against
 *                            an element-by-element numpy loop over
 *                            orc_swiglu_value.
 *   orc_elementwise        - add, multiply and scale bit-exact against numpy
 *                            F32 with b tiled; silu within a few ulp of the
 *                            FP64 closed form; rms_norm within 1e-6 relative
 *                            of the FP64 closed form, constant rows exactly
 *                            (c / |c| = sign), and the reference
 *                            library-bench gold (max_abs < 1e-4).
 *   orc_native_q4_size     - the reference's published 4096 x 4096 figure
 *                            (9,437,184 bytes) and the closed form;
 *   orc_pack_native_q4,
 *   orc_native_q4_decode   - the reference bench's inverse-mapping check of
 *                            every nibble and scale, and decode(pack(q4))
 *                            equal to orc_q4_decode(q4) bit for bit.
 *   orc_common_q4_size,
 *   orc_common_q4_pack,
 *   orc_common_q4_decode   - the reference layout test's properties (the
 *                            weight map is a bijection onto the payload,
 *                            4.5 padded bits per weight) and decode(pack(q4))
 *                            equal to orc_q4_decode(q4) bit for bit, over
 *                            every FP16 scale pattern;
 *   orc_common_quant_pair  - codes equal orc_i8_activation's on the padded
 *                            input (pinned against the reference header);
 *                            view layout checked against the reference
 *                            bench's index formula;
 *   orc_common_quant_rows  - the reference bench's CPU row rule
 *                            (bench/common-q4-bench.cpp:43-45) restated in
 *                            numpy, and scale * code within scale/2 of x.
 */
#ifndef KUNLUN_ORACLE_H
#define KUNLUN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight type codes, as kunlun::WeightType. */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_I8 = 3 };

uint32_t orc_xorshift32(uint32_t *state);
float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float value);
uint16_t orc_bench_half(float value);
int orc_round_clamp(float value, int limit);

void orc_q4_decode(const uint8_t *q4, int k, int n, float *w);
void orc_f16_decode(const uint16_t *h, size_t count, float *w);
void orc_f16_encode(const float *w, size_t count, uint16_t *h);
void orc_q4_quantize(const float *w, int k, int n, uint8_t *q4);

void orc_bench_weights(int k, int n, float *w, uint16_t *wh, uint8_t *q4);
void orc_bench_input(int k, int batch, float *x);
void orc_fused_bench_weights(int k, int n, float *w, uint8_t *q4);
void orc_fixture_q4(int k, int n, uint8_t *q4);
void orc_fixture_input(int k, int batch, int pattern, float *x);

void orc_gold(const float *w, const float *x, int k, int n, int batch, int threads, double *y);
void orc_matvec_f32(const void *w, int type, const float *x, int k, int n, int batch, float *y);

void orc_i8_rows(const float *w, int k, int rows, int8_t *codes, float *scales);
int orc_i8_activation(const float *x, size_t count, int8_t *q0, int8_t *q1,
                      float *max0, float *max1);
void orc_i8_dots(const int8_t *a, int rows, const int8_t *w, int n, int k, int64_t *out);
void orc_i8_combine(const int64_t *primary, const int64_t *residual, const float *scales,
                    float max0, float max1, int n, int batch, float *y);

float orc_swiglu_value(float g, float u);
void orc_swiglu(const void *gate, const void *up, void *y, int width, int rows, int gate_stride,
                int up_stride, int output_stride, int bytes);
void orc_elementwise(float *y, const float *a, const float *b, int n, int width, int bn, int op, float parameter);

size_t orc_native_q4_size(int k, int n);
void orc_pack_native_q4(const uint8_t *q4, int k, int n, uint8_t *out);
void orc_native_q4_decode(const uint8_t *native, int k, int n, float *w);

size_t orc_common_q4_size(int k, int n);
void orc_common_q4_pack(const uint8_t *q4, int k, int n, uint8_t *out);
void orc_common_q4_decode(const uint8_t *packed, int k, int n, float *w);
int orc_common_quant_pair(const float *x, int k, int8_t *values, float *params);
void orc_common_quant_rows(const float *x, int k, int rows, int defined, int8_t *values, float *params);

#ifdef __cplusplus
}
#endif

#endif
