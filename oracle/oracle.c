/* CPU oracle for the KunlunK200 matmul path. TEST INFRASTRUCTURE ONLY:
 * the checker for tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, never part of the product path. See oracle.h for how each function is
 * pinned. Compiled with -ffp-contract=off so that float expressions round
 * after every operation, as the reference's host code does on x86-64.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* xorshift32 step (reference bench/native-q4-reference.h:14). */
uint32_t orc_xorshift32(uint32_t *state) {
    uint32_t s = *state;
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    *state = s;
    return s;
}

/* IEEE binary16 -> binary32, subnormals, Inf and NaN included
 * (reference kernels/kunlun-matvec.xpu:4-18, kernels/q4-device.h:3-12). */
float orc_half_to_float(uint16_t h) {
    uint32_t exponent = (h >> 10) & 31u, mantissa = h & 1023u;
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            int shift = 0;
            while ((mantissa & 1024u) == 0) { mantissa <<= 1; ++shift; }
            bits = sign | ((uint32_t)(113 - shift) << 23) | ((mantissa & 1023u) << 13);
        }
    } else {
        bits = sign | ((exponent == 31 ? 255u : exponent + 112u) << 23) | (mantissa << 13);
    }
    float value;
    memcpy(&value, &bits, 4);
    return value;
}

/* binary32 -> binary16, round to nearest even, saturating to Inf, NaN kept
 * quiet (reference kernels/fp16-device.h:14-31). */
uint16_t orc_float_to_half(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    uint32_t sign = (bits >> 16) & 0x8000u, mantissa = bits & 0x7fffffu;
    int exponent = (int)((bits >> 23) & 255u) - 112;
    if (exponent == 143) return (uint16_t)(sign | 0x7c00u | (mantissa ? ((mantissa >> 13) | 0x200u) : 0));
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    if (exponent <= 0) {
        if (exponent < -10) return (uint16_t)sign;
        uint32_t m = mantissa | 0x800000u;
        int shift = 14 - exponent;
        return (uint16_t)(sign | ((m + ((1u << (shift - 1)) - 1) + ((m >> shift) & 1u)) >> shift));
    }
    mantissa += 0xfffu + ((mantissa >> 13) & 1u);
    if (mantissa & 0x800000u) { mantissa = 0; ++exponent; }
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)exponent << 10) | (mantissa >> 13));
}

/* The library bench's truncating F16 encoder for its exactly representable
 * weights (reference bench/library-bench.cpp:11-16). Aborts where the
 * reference's require() would. */
uint16_t orc_bench_half(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    int exponent = (int)((bits >> 23) & 255u) - 127 + 15;
    if (!((exponent > 0 && exponent < 31) || value == 0)) abort();
    if (value == 0) return 0;
    return (uint16_t)(((bits >> 16) & 0x8000u) | ((uint32_t)exponent << 10) | ((bits & 0x7fffffu) >> 13));
}

/* Round half away from zero by truncating v +/- 0.5f, then clamp to
 * [-limit, limit] (reference src/k200.cpp:114,217,224;
 * bench/native-q4-reference.h:18). */
int orc_round_clamp(float value, int limit) {
    float shifted = value + (value >= 0 ? 0.5f : -0.5f);
    int q = (int)shifted;
    if (q > limit) q = limit;
    if (q < -limit) q = -limit;
    return q;
}

/* Q4_0 rows -> F32: w[32b+j] = (lo(q[j]) - 8) * d, w[32b+j+16] = (hi(q[j]) - 8) * d
 * (reference kernels/kunlun-matvec.xpu:49-59, bench/native-q4-reference.h:16,44). */
void orc_q4_decode(const uint8_t *q4, int k, int n, float *w) {
    size_t blocks = (size_t)n * (size_t)(k / 32);
    for (size_t block = 0; block < blocks; ++block) {
        const uint8_t *p = q4 + block * 18;
        float d = orc_half_to_float((uint16_t)(p[0] | (p[1] << 8)));
        float *out = w + block * 32;
        for (int j = 0; j < 16; ++j) {
            out[j] = (float)((int)(p[2 + j] & 15) - 8) * d;
            out[j + 16] = (float)((int)(p[2 + j] >> 4) - 8) * d;
        }
    }
}

void orc_f16_decode(const uint16_t *h, size_t count, float *w) {
    for (size_t i = 0; i < count; ++i) w[i] = orc_half_to_float(h[i]);
}

void orc_f16_encode(const float *w, size_t count, uint16_t *h) {
    for (size_t i = 0; i < count; ++i) h[i] = orc_float_to_half(w[i]);
}

/* Q4_0 encoder with the closed form BASELINE's configs name (ggml's
 * reference quantizer): per 32-block, max = the signed value of largest
 * magnitude (first occurrence), d = max / -8, id = d ? 1/d : 0, F16 scale by
 * RNE, nibble = min(15, (int8)(x*id + 8.5)). ggml is not in the reference
 * repository: bit-level parity with it is unpinned. */
void orc_q4_quantize(const float *w, int k, int n, uint8_t *q4) {
    size_t blocks = (size_t)n * (size_t)(k / 32);
    for (size_t block = 0; block < blocks; ++block) {
        const float *x = w + block * 32;
        uint8_t *p = q4 + block * 18;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; ++j) {
            float v = x[j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        float d = max / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t hd = orc_float_to_half(d);
        p[0] = (uint8_t)(hd & 255u);
        p[1] = (uint8_t)(hd >> 8);
        for (int j = 0; j < 16; ++j) {
            float x0 = x[j] * id, x1 = x[j + 16] * id;
            int q0 = (int8_t)(x0 + 8.5f), q1 = (int8_t)(x1 + 8.5f);
            if (q0 > 15) q0 = 15;
            if (q1 > 15) q1 = 15;
            p[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

/* The library bench's deterministic weights: w[r,j] = ((r+j)%16 - 8)/16 as
 * F32 and F16, and the same values as Q4_0 blocks with scale 0x2c00
 * (reference bench/library-bench.cpp:89-100). Any output may be NULL. */
void orc_bench_weights(int k, int n, float *w, uint16_t *wh, uint8_t *q4) {
    for (int r = 0; r < n; ++r) {
        for (int j = 0; j < k; ++j) {
            float value = (float)((r + j) % 16 - 8) * 0.0625f;
            if (w) w[(size_t)r * k + j] = value;
            if (wh) wh[(size_t)r * k + j] = orc_bench_half(value);
        }
    }
    if (!q4) return;
    size_t blocks = (size_t)n * (size_t)(k / 32);
    for (size_t block = 0; block < blocks; ++block) {
        q4[block * 18] = 0x00;
        q4[block * 18 + 1] = 0x2c;
        int row = (int)(block * 32 / (size_t)k);
        int col0 = (int)(block * 32 % (size_t)k);
        for (int j = 0; j < 16; ++j) {
            int col = col0 + j;
            q4[block * 18 + 2 + j] = (uint8_t)(((row + col) % 16) | (((row + col + 16) % 16) << 4));
        }
    }
}

/* x[j] = sin(j * 0.017f) over the flat [batch, k] index
 * (reference bench/library-bench.cpp:101). */
void orc_bench_input(int k, int batch, float *x) {
    size_t count = (size_t)k * (size_t)batch;
    for (size_t j = 0; j < count; ++j) x[j] = sinf((float)j * 0.017f);
}

/* The fused bench's periodic weights: per block d in {1/64, 1/32, 3/64} with
 * alternating sign, w = ((row+j)%16 - 8) * d with j the in-block index, so row
 * r computes the same dot product as row r%16
 * (reference bench/fused-bench.cpp:15-20,23,41). Either output may be NULL. */
void orc_fused_bench_weights(int k, int n, float *w, uint8_t *q4) {
    for (int row = 0; row < n; ++row) {
        for (int block = 0; block < k / 32; ++block) {
            float d = (block % 3 == 0 ? 0.015625f : block % 3 == 1 ? 0.03125f : 0.046875f) *
                      (block % 2 ? -1.0f : 1.0f);
            if (w)
                for (int j = 0; j < 32; ++j)
                    w[(size_t)row * k + block * 32 + j] = (float)((row + j) % 16 - 8) * d;
            if (q4) {
                uint8_t *p = q4 + ((size_t)row * (k / 32) + block) * 18;
                uint16_t h = orc_float_to_half(d);
                p[0] = (uint8_t)(h & 255u);
                p[1] = (uint8_t)(h >> 8);
                for (int j = 0; j < 16; ++j)
                    p[2 + j] = (uint8_t)(((row + j) % 16) | (((row + j + 16) % 16) << 4));
            }
        }
    }
}

/* Seeded random Q4_0 weights of the native-Q4 benches: xorshift32 from
 * 0x7340d123, per block one draw for the scale
 * d = +-ldexp((8 + h%9)/1024, (h>>4)%7 - 3), negative when bit 31 is set, zero
 * when (row*13 + b) % 257 == 0, then 16 draws for the nibble bytes
 * (reference bench/native-q4-reference.h:30-41). */
void orc_fixture_q4(int k, int n, uint8_t *q4) {
    uint32_t state = 0x7340d123u;
    for (int row = 0; row < n; ++row) {
        for (int b = 0; b < k / 32; ++b) {
            uint8_t *p = q4 + ((size_t)row * (k / 32) + b) * 18;
            uint32_t h = orc_xorshift32(&state);
            float d = ldexpf((float)(8 + (h % 9)) / 1024.0f, (int)((h >> 4) % 7) - 3);
            if (h & 0x80000000u) d = -d;
            if ((row * 13 + b) % 257 == 0) d = 0.0f;
            uint16_t hd = orc_float_to_half(d);
            p[0] = (uint8_t)(hd & 255u);
            p[1] = (uint8_t)(hd >> 8);
            for (int j = 0; j < 16; ++j) p[j + 2] = (uint8_t)orc_xorshift32(&state);
        }
    }
}

/* Seeded activations of the native-Q4 benches: xorshift32 from 0x09200abc;
 * pattern 0 normal, 1 every 113th value x1000, 2 zeros, 3 wide int32/2^31,
 * 4 wide exponents (reference bench/native-q4-reference.h:58-69). */
void orc_fixture_input(int k, int batch, int pattern, float *x) {
    uint32_t state = 0x09200abcu;
    size_t count = (size_t)k * (size_t)batch;
    for (size_t j = 0; j < count; ++j) {
        float value = (float)((int)(orc_xorshift32(&state) % 20001u) - 10000) / 8192.0f;
        if (pattern == 3) value = (float)((double)(int32_t)orc_xorshift32(&state) / 2147483648.0);
        if (pattern == 4) {
            uint32_t bits = orc_xorshift32(&state);
            bits = (bits & 0x807fffffu) | ((107u + (orc_xorshift32(&state) % 32u)) << 23);
            memcpy(&value, &bits, 4);
        }
        if (pattern == 1 && j % 113 == 0) value *= 1000.0f;
        if (pattern == 2) value = 0.0f;
        x[j] = value;
    }
}

/* FP64 gold: y[b*n + r] = sum_j double(w[r,j]) * double(x[b,j]), summed in
 * increasing j (reference bench/library-bench.cpp:121-122;
 * bench/native-q4-reference.h:98-108 runs the same sum on 6 OpenMP threads). */
void orc_gold(const float *w, const float *x, int k, int n, int batch, int threads, double *y) {
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int r = 0; r < n; ++r) {
        const float *wr = w + (size_t)r * k;
        for (int b = 0; b < batch; ++b) {
            const float *xb = x + (size_t)b * k;
            double sum = 0.0;
            for (int j = 0; j < k; ++j) sum += (double)wr[j] * (double)xb[j];
            y[(size_t)b * n + r] = sum;
        }
    }
}

/* The reference device kernel's F32 arithmetic order: per 32-block, eight
 * lanes accumulate q*x over j = l, l+8, l+16, l+24, the lanes are summed in
 * order, and sum += d * s with d = 1 for F32/F16
 * (reference kernels/kunlun-matvec.xpu:49-72). */
void orc_matvec_f32(const void *w, int type, const float *x, int k, int n, int batch, float *y) {
    const uint8_t *bytes = (const uint8_t *)w;
    size_t row_bytes = type == ORC_Q4_0 ? (size_t)(k / 32) * 18 : (size_t)k * (type == ORC_F16 ? 2 : 4);
    for (int b = 0; b < batch; ++b) {
        for (int r = 0; r < n; ++r) {
            const uint8_t *row = bytes + (size_t)r * row_bytes;
            float sum = 0.0f;
            for (int block = 0; block < k / 32; ++block) {
                float q[32], d = 1.0f;
                if (type == ORC_Q4_0) {
                    const uint8_t *p = row + (size_t)block * 18;
                    d = orc_half_to_float((uint16_t)(p[0] | (p[1] << 8)));
                    for (int j = 0; j < 16; ++j) {
                        q[j] = (float)(p[2 + j] & 15) - 8.0f;
                        q[j + 16] = (float)(p[2 + j] >> 4) - 8.0f;
                    }
                } else if (type == ORC_F16) {
                    for (int j = 0; j < 32; ++j) {
                        uint16_t h;
                        memcpy(&h, row + ((size_t)block * 32 + j) * 2, 2);
                        q[j] = orc_half_to_float(h);
                    }
                } else {
                    memcpy(q, row + (size_t)block * 32 * 4, 32 * 4);
                }
                const float *xv = x + (size_t)b * k + (size_t)block * 32;
                float acc[8];
                for (int l = 0; l < 8; ++l) acc[l] = q[l] * xv[l];
                for (int j = 8; j < 32; j += 8)
                    for (int l = 0; l < 8; ++l) acc[l] = acc[l] + q[j + l] * xv[j + l];
                float s = 0.0f;
                for (int l = 0; l < 8; ++l) s += acc[l];
                sum += d * s;
            }
            y[(size_t)b * n + r] = sum;
        }
    }
}

/* upload_i8_rows' host quantizer: per row max|v|, scale = max/127 (1 when the
 * row is zero), inv = 127/max (0 when zero), q = round-clamp(v*inv, 127)
 * (reference src/k200.cpp:107-116). */
void orc_i8_rows(const float *w, int k, int rows, int8_t *codes, float *scales) {
    for (int r = 0; r < rows; ++r) {
        const float *row = w + (size_t)r * k;
        float maximum = 0.0f;
        for (int j = 0; j < k; ++j) {
            float a = fabsf(row[j]);
            if (a > maximum) maximum = a;
        }
        scales[r] = maximum > 0 ? maximum / 127.0f : 1.0f;
        float inv = maximum > 0 ? 127.0f / maximum : 0.0f;
        for (int j = 0; j < k; ++j) {
            float value = row[j] * inv;
            codes[(size_t)r * k + j] = (int8_t)orc_round_clamp(value, 127);
        }
    }
}

/* rowwise_i8 two-pass activation quantization over the whole [batch, k]
 * tensor: max0 = max|x| (1 if zero), q0 = rnd(x * (127/max0)),
 * r = x - q0 * (max0/127), max1 = max|r| (1 if zero), q1 = rnd(r * (127/max1))
 * (reference src/k200.cpp:212-225). Returns -1 (nothing written) when a
 * value is not finite, where the reference's require() aborts. */
int orc_i8_activation(const float *x, size_t count, int8_t *q0, int8_t *q1,
                      float *max0_out, float *max1_out) {
    float max0 = 0.0f, max1 = 0.0f;
    for (size_t j = 0; j < count; ++j) {
        if (!isfinite(x[j])) return -1;
        float a = fabsf(x[j]);
        if (a > max0) max0 = a;
    }
    if (max0 == 0.0f) max0 = 1.0f;
    float *residual = (float *)malloc(count * sizeof(float) + 1);
    if (!residual) return -2;
    for (size_t j = 0; j < count; ++j) {
        float value = x[j] * (127.0f / max0);
        int q = orc_round_clamp(value, 127);
        q0[j] = (int8_t)q;
        float step = max0 / 127.0f;
        float product = (float)q * step;
        residual[j] = x[j] - product;
        float a = fabsf(residual[j]);
        if (a > max1) max1 = a;
    }
    if (max1 == 0.0f) max1 = 1.0f;
    for (size_t j = 0; j < count; ++j) {
        float value = residual[j] * (127.0f / max1);
        q1[j] = (int8_t)orc_round_clamp(value, 127);
    }
    free(residual);
    *max0_out = max0;
    *max1_out = max1;
    return 0;
}

/* Exact integer dot products out[r*n + c] = sum_j a[r,j] * w[c,j] (the raw
 * int8 x int8 FC products, reference src/k200.cpp:231). */
void orc_i8_dots(const int8_t *a, int rows, const int8_t *w, int n, int k, int64_t *out) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const int8_t *ar = a + (size_t)r * k;
        for (int c = 0; c < n; ++c) {
            const int8_t *wc = w + (size_t)c * k;
            int64_t sum = 0;
            for (int j = 0; j < k; ++j) sum += (int64_t)ar[j] * (int64_t)wc[j];
            out[(size_t)r * n + c] = sum;
        }
    }
}

/* Combine of the primary and residual products:
 * y[b,r] = (float(P)*(max0/127) + float(R)*(max1/127)) * scale[r]
 * (reference kernels/kunlun-combine.xpu:10-19). */
void orc_i8_combine(const int64_t *primary, const int64_t *residual, const float *scales,
                    float max0, float max1, int n, int batch, float *y) {
    float scale0 = max0 / 127.0f, scale1 = max1 / 127.0f;
    for (int b = 0; b < batch; ++b) {
        for (int r = 0; r < n; ++r) {
            size_t i = (size_t)b * n + r;
            float t0 = (float)primary[i] * scale0;
            float t1 = (float)residual[i] * scale1;
            float t = t0 + t1;
            y[i] = t * scales[r];
        }
    }
}

/* SiLU(g) * u in F32 with the reference's non-finite classification
 * (reference kernels/kunlun-swiglu.xpu:27-39): finite inputs give
 * (g / (1 + expf(-g))) * u; NaN if g or u is NaN or g is -Inf; +-Inf with
 * sign(g) ^ sign(u) if one side is infinite and the other side (SiLU(g) for
 * a finite g) is non-zero, NaN for Inf * 0. */
float orc_swiglu_value(float g, float u) {
    uint32_t gb, ub, bits;
    float out;
    memcpy(&gb, &g, 4);
    memcpy(&ub, &u, 4);
    uint32_t ga = gb & 0x7fffffffu, ua = ub & 0x7fffffffu;
    if (ga < 0x7f800000u && ua < 0x7f800000u) {
        float e = expf(-g);
        float den = 1.0f + e;
        float act = g / den;
        return act * u;
    }
    uint32_t sign = (gb ^ ub) & 0x80000000u;
    if (ga > 0x7f800000u || ua > 0x7f800000u || gb == 0xff800000u) {
        bits = 0x7fc00000u;
    } else if (ga == 0x7f800000u) {
        bits = ua == 0 ? 0x7fc00000u : (sign | 0x7f800000u);
    } else {
        float e = expf(-g);
        float act = g / (1.0f + e);
        uint32_t ab;
        memcpy(&ab, &act, 4);
        bits = (ab & 0x7fffffffu) == 0 ? 0x7fc00000u : (sign | 0x7f800000u);
    }
    memcpy(&out, &bits, 4);
    return out;
}

/* y = SiLU(gate) * up over rows of F32 (bytes == 4) or F16 (bytes == 2)
 * values, strides in bytes, F32 intermediates and one final rounding (RNE to
 * F16) (reference src/k200.cpp:324-368). Elements are processed in order, so
 * an output that aliases an input element for element is handled. */
void orc_swiglu(const void *gate, const void *up, void *y, int width, int rows, int gate_stride,
                int up_stride, int output_stride, int bytes) {
    const uint8_t *g8 = (const uint8_t *)gate, *u8 = (const uint8_t *)up;
    uint8_t *y8 = (uint8_t *)y;
    for (int r = 0; r < rows; ++r) {
        for (int j = 0; j < width; ++j) {
            const uint8_t *gp = g8 + (size_t)r * gate_stride + (size_t)j * bytes;
            const uint8_t *up_ = u8 + (size_t)r * up_stride + (size_t)j * bytes;
            uint8_t *yp = y8 + (size_t)r * output_stride + (size_t)j * bytes;
            float g, u, v;
            if (bytes == 4) {
                memcpy(&g, gp, 4);
                memcpy(&u, up_, 4);
            } else {
                uint16_t hg, hu;
                memcpy(&hg, gp, 2);
                memcpy(&hu, up_, 2);
                g = orc_half_to_float(hg);
                u = orc_half_to_float(hu);
            }
            v = orc_swiglu_value(g, u);
            if (bytes == 4) {
                memcpy(yp, &v, 4);
            } else {
                uint16_t h = orc_float_to_half(v);
                memcpy(yp, &h, 2);
            }
        }
    }
}

/* Elementwise F32 op over n values (reference kernels/kunlun-elementwise.xpu
 * and src/k200.cpp:280-323): 0 add and 1 multiply with b[e % bn], 2 silu
 * a / (1 + expf(-a)), 4 scale a * parameter, 3 rms_norm of each `width` row:
 * sum of squares accumulated in F32 in element order, then
 * a * (1 / sqrtf(sum / width + parameter)). y may equal a or b: every input
 * an output depends on is read before it is written (rms_norm reads its row
 * twice, and the second read of element j precedes the write of element j). */
void orc_elementwise(float *y, const float *a, const float *b, int n, int width, int bn, int op, float parameter) {
    if (op == 3) {
        for (int r = 0; r < n / width; ++r) {
            const float *row = a + (size_t)r * width;
            float *out = y + (size_t)r * width;
            float sum = 0.0f;
            for (int j = 0; j < width; ++j) sum += row[j] * row[j];
            float scale = 1.0f / sqrtf(sum / (float)width + parameter);
            for (int j = 0; j < width; ++j) out[j] = row[j] * scale;
        }
        return;
    }
    for (int e = 0; e < n; ++e) {
        float v = a[e], out;
        if (op == 0) {
            out = v + b[e % bn];
        } else if (op == 1) {
            out = v * b[e % bn];
        } else if (op == 2) {
            out = v / (1.0f + expf(-v));
        } else {
            out = v * parameter;
        }
        y[e] = out;
    }
}

/* Native Q4 layout (reference src/q4-layout.cpp:7-37). Bytes: rows = n padded
 * to 32; payload = aligned256(rows * k / 2); scales = aligned256(rows * k / 16). */
static size_t orc_align256(size_t bytes) { return (bytes + 255u) & ~(size_t)255u; }

size_t orc_native_q4_size(int k, int n) {
    if (k <= 0 || k > 16384 || k % 32 != 0 || n <= 0 || n > 90000000 / k) return 0;
    size_t rows = ((size_t)n + 31u) & ~(size_t)31u;
    return orc_align256(rows * (size_t)k / 2) + orc_align256(rows * (size_t)(k / 32) * 2);
}

/* Element e (0..31) of a Q4_0 block as the signed value q - 8: byte 2 + e % 16,
 * low nibble for e < 16, high nibble otherwise (reference q4-layout.cpp:29-30). */
static int orc_q4_signed(const uint8_t *block, int e) {
    int shift = e < 16 ? 0 : 4;
    return ((block[2 + (e % 16)] >> shift) & 15) - 8;
}

/* For row r and block b: the FP16 scale goes to the scale region at
 * ((r / 32) * (k / 32) + b) * 32 + r % 32 (two bytes each), and byte
 * ((r / 32) * (k / 32) + b) * 512 + j * 32 + r % 32 holds elements 2j (low
 * nibble) and 2j + 1 (high) as 4-bit two's complement
 * (reference q4-layout.cpp:24-35). Everything else is zero. */
void orc_pack_native_q4(const uint8_t *q4, int k, int n, uint8_t *out) {
    size_t total = orc_native_q4_size(k, n);
    size_t rows = ((size_t)n + 31u) & ~(size_t)31u;
    size_t payload = orc_align256(rows * (size_t)k / 2);
    int blocks = k / 32;
    memset(out, 0, total);
    for (int r = 0; r < n; ++r) {
        for (int b = 0; b < blocks; ++b) {
            const uint8_t *block = q4 + ((size_t)r * blocks + b) * 18;
            size_t tb = (size_t)(r / 32) * blocks + b;
            out[payload + (tb * 32 + r % 32) * 2] = block[0];
            out[payload + (tb * 32 + r % 32) * 2 + 1] = block[1];
            for (int j = 0; j < 16; ++j) {
                int lo = orc_q4_signed(block, 2 * j), hi = orc_q4_signed(block, 2 * j + 1);
                out[tb * 512 + (size_t)j * 32 + r % 32] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
            }
        }
    }
}

/* Inverse view: F32 weights [n, k] of a native layout, w = signed4 * fp16 scale. */
void orc_native_q4_decode(const uint8_t *native, int k, int n, float *w) {
    size_t rows = ((size_t)n + 31u) & ~(size_t)31u;
    size_t payload = orc_align256(rows * (size_t)k / 2);
    int blocks = k / 32;
    for (int r = 0; r < n; ++r) {
        for (int b = 0; b < blocks; ++b) {
            size_t tb = (size_t)(r / 32) * blocks + b;
            uint16_t h = (uint16_t)(native[payload + (tb * 32 + r % 32) * 2] |
                                    (native[payload + (tb * 32 + r % 32) * 2 + 1] << 8));
            float d = orc_half_to_float(h);
            for (int e = 0; e < 32; ++e) {
                int byte = native[tb * 512 + (size_t)(e / 2) * 32 + r % 32];
                int v = (e % 2 ? byte >> 4 : byte) & 15;
                w[(size_t)r * k + (size_t)b * 32 + e] = (float)(v >= 8 ? v - 16 : v) * d;
            }
        }
    }
}

/* Common Q4 ABI v1 (reference src/q4-common-pack.h:16-31, docs/q4-common-ABI.json):
 * Kp = k rounded up to 512 (k < 512) or 256, Np = n rounded up to 256,
 * weights Np*Kp/2 bytes then FP16 scales Np*Kp/16 bytes. */
static int orc_round_up(int v, int a) { return (v + a - 1) / a * a; }
static void orc_common_dims(int k, int n, int *kp, int *np, size_t *scale_offset) {
    *kp = orc_round_up(k, k < 512 ? 512 : 256);
    *np = orc_round_up(n, 256);
    *scale_offset = (size_t)*kp * (size_t)*np / 2;
}

size_t orc_common_q4_size(int k, int n) {
    if (k < 1 || k > 16384 || n < 1 || n > 32000) return 0;
    int kp, np;
    size_t off;
    orc_common_dims(k, n, &kp, &np, &off);
    return off + (size_t)kp * (size_t)np / 16;
}

/* Layout 1 ("Micro32Bank", reference q4-common-pack.h:23-29): column c, K
 * pair index pr -> kb = pr/16, p = pr%16, word row = (c%32/16)*8 + p/2,
 * bank = c%16, byte = (tile + kb)*512 + (bank*16 + row)*2 + p%2 with
 * tile = (c/32)*(Kp/32). Scale order 1 (KMajor, q4-common-pack.h:31):
 * scale_offset + (kb*Np + c)*2. */
static size_t orc_common_weight_index(int kp, int c, int pr) {
    int kb = pr / 16, p = pr % 16, row = (c % 32 / 16) * 8 + p / 2, bank = c % 16;
    size_t tile = (size_t)(c / 32) * (size_t)(kp / 32);
    return (tile + (size_t)kb) * 512 + (size_t)(bank * 16 + row) * 2 + (size_t)(p % 2);
}
static size_t orc_common_scale_index(size_t scale_offset, int np, int c, int kb) {
    return scale_offset + ((size_t)kb * (size_t)np + (size_t)c) * 2;
}

/* Pack n rows of ceil(k/32) Q4_0 blocks (reference q4-common-pack.h:32-44):
 * every byte not written is zero. */
void orc_common_q4_pack(const uint8_t *q4, int k, int n, uint8_t *out) {
    int kp, np;
    size_t off;
    orc_common_dims(k, n, &kp, &np, &off);
    int blocks = (k + 31) / 32;
    memset(out, 0, orc_common_q4_size(k, n));
    for (int c = 0; c < n; ++c) {
        for (int b = 0; b < blocks; ++b) {
            const uint8_t *src = q4 + ((size_t)c * blocks + b) * 18;
            size_t si = orc_common_scale_index(off, np, c, b);
            out[si] = src[0];
            out[si + 1] = src[1];
            for (int p = 0; p < 16; ++p) {
                int lo = orc_q4_signed(src, 2 * p), hi = orc_q4_signed(src, 2 * p + 1);
                out[orc_common_weight_index(kp, c, b * 16 + p)] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
            }
        }
    }
}

/* F32 weights [n, k] of a packed region: signed nibble * FP16 scale. */
void orc_common_q4_decode(const uint8_t *packed, int k, int n, float *w) {
    int kp, np;
    size_t off;
    orc_common_dims(k, n, &kp, &np, &off);
    for (int c = 0; c < n; ++c) {
        for (int j = 0; j < k; ++j) {
            int v = packed[orc_common_weight_index(kp, c, j / 2)] >> (j % 2 * 4) & 15;
            size_t si = orc_common_scale_index(off, np, c, j / 32);
            float d = orc_half_to_float((uint16_t)(packed[si] | (packed[si + 1] << 8)));
            w[(size_t)c * k + j] = (float)(v >= 8 ? v - 16 : v) * d;
        }
    }
}

/* M = 1 activation view (reference kernels/kunlun-common-max-exact.xpu,
 * -main-exact.xpu, -residual-exact.xpu): the two-component per-tensor
 * quantization of X padded with zeros to Kp (orc_i8_activation's rule), main
 * code of K j at values[(j/32)*64 + j%32], residual at values[2*Kp + same],
 * every other byte of values[0 .. 4*Kp + 1024) zero; params =
 * {max0/127, max1/127, max0, max1, 0 x 12}. -1 for a non-finite input. */
int orc_common_quant_pair(const float *x, int k, int8_t *values, float *params) {
    int kp, np;
    size_t off;
    orc_common_dims(k, 1, &kp, &np, &off);
    float *padded = (float *)calloc((size_t)kp, sizeof(float));
    int8_t *q0 = (int8_t *)malloc((size_t)kp), *q1 = (int8_t *)malloc((size_t)kp);
    float max0, max1;
    int rc = -2;
    if (padded && q0 && q1) {
        memcpy(padded, x, (size_t)k * sizeof(float));
        rc = orc_i8_activation(padded, (size_t)kp, q0, q1, &max0, &max1);
    }
    if (rc == 0) {
        memset(values, 0, (size_t)4 * kp + 1024);
        for (int j = 0; j < kp; ++j) {
            size_t i = (size_t)(j / 32) * 64 + (size_t)(j % 32);
            values[i] = q0[j];
            values[(size_t)2 * kp + i] = q1[j];
        }
        for (int i = 0; i < 16; ++i) params[i] = 0.0f;
        params[0] = max0 / 127.0f;
        params[1] = max1 / 127.0f;
        params[2] = max0;
        params[3] = max1;
    }
    free(padded);
    free(q0);
    free(q1);
    return rc;
}

/* M > 1 Row A8 (reference common-q4/.../quant-row-serial-fused.xpu): row r of
 * `rows` rows of X [rows, k] (rows up to `defined` are zero) -> max = max|x|
 * (1 if 0), codes rnd(x * (127/max)) at values[r*Kp + j] (zero for j >= k),
 * scale max/127 in all 16 floats of params[r*16 ..]. */
void orc_common_quant_rows(const float *x, int k, int rows, int defined, int8_t *values, float *params) {
    int kp, np;
    size_t off;
    orc_common_dims(k, 1, &kp, &np, &off);
    for (int r = 0; r < defined; ++r) {
        float mx = 0.0f;
        for (int j = 0; j < k && r < rows; ++j) {
            float a = fabsf(x[(size_t)r * k + j]);
            if (a > mx) mx = a;
        }
        if (mx == 0.0f) mx = 1.0f;
        float inv = 127.0f / mx, scale = mx / 127.0f;
        for (int j = 0; j < kp; ++j) {
            float v = (r < rows && j < k) ? x[(size_t)r * k + j] : 0.0f;
            float scaled = v * inv;
            values[(size_t)r * kp + j] = (int8_t)orc_round_clamp(scaled, 127);
        }
        for (int i = 0; i < 16; ++i) params[r * 16 + i] = scale;
    }
}
