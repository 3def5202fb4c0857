// Batch-1..N GEMV for F32, F16 and raw 18-byte Q4_0 weight rows on gfx950.
//
// Y[b, r] = sum_k X[b, k] * W[r, k]   (reference kernels/kunlun-matvec.xpu:24-79)
//
// The path is HBM-bound: every weight byte is read once, activations are
// staged in LDS once per workgroup and reused for every row the workgroup
// owns. Arithmetic is F32 with F32 accumulation; Q4_0 nibbles and F16 values
// are decoded exactly (the decoded value (q-8)*d is exact in F32).
//
// Kernels:
//   q4_gemv_pair  Q4_0, K % 64 == 0, 4-byte aligned rows. A lane owns a pair
//                 of adjacent blocks (36 bytes = 9 dwords, 64 weights) of each
//                 row, loaded with dword-aligned 16+16+4 byte loads; the
//                 first block's nibbles are re-aligned with v_alignbyte.
//   dense_gemv    F32 / F16, 16-byte aligned rows. A lane owns 16-byte chunks
//                 spaced 1 KiB apart so every load instruction is coalesced.
//   gemv_general  any format, alignment and K % 32: byte loads, one wave per
//                 row. Correct for every input the API accepts; slow.
#include "device_common.h"
#include "launch.h"

#include <algorithm>
#include <cstdlib>

namespace {

using kk::kWave;

constexpr int kThreads = 256;          // 4 waves per workgroup
constexpr int kWavesPerGroup = kThreads / kWave;

// ---------------------------------------------------------------------------
// Q4_0, pair-of-blocks lanes.
//
// LDS holds X for the batch chunk as float4 in [b][h][q][p] order, where
// block = 2p + h and q is the float4 slot (0..7) inside the 32-value block,
// so lanes (consecutive p) read consecutive float4: conflict-free. It also
// holds xsum[b][h][p], the sum of the block's 32 activations, used to apply
// the -8 nibble offset once per block: sum((q-8) x) = sum(q x) - 8 sum(x).
template <int B, int U>
__global__ __launch_bounds__(kThreads) void q4_gemv_pair(const uint8_t *__restrict__ w,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int k, int n,
                                                        int y_stride) {
    extern __shared__ float4 lds[];
    const int blocks = k >> 5;
    const int pairs = blocks >> 1;
    const size_t row_bytes = static_cast<size_t>(blocks) * 18;
    float4 *xl = lds;
    float *xs = reinterpret_cast<float *>(lds + static_cast<size_t>(B) * 8 * blocks);

    for (int idx = threadIdx.x; idx < B * blocks; idx += kThreads) {
        const int b = idx / blocks, blk = idx - b * blocks;
        const int p = blk >> 1, h = blk & 1;
        const float4 *src = reinterpret_cast<const float4 *>(x + static_cast<size_t>(b) * k + blk * 32);
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 v = src[q];
            xl[((b * 2 + h) * 8 + q) * pairs + p] = v;
            s += (v.x + v.y) + (v.z + v.w);
        }
        xs[(b * 2 + h) * pairs + p] = s;
    }
    __syncthreads();

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = blockIdx.x * kWavesPerGroup + (threadIdx.x >> 6);
    const int waves = gridDim.x * kWavesPerGroup;
    const int rowblocks = (n + U - 1) / U;

    for (int rb = wave; rb < rowblocks; rb += waves) {
        const int r0 = rb * U;
        float acc[U][B];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int b = 0; b < B; ++b) acc[u][b] = 0.0f;

        for (int p = lane; p < pairs; p += kWave) {
            uint32_t wd[U][9];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = min(r0 + u, n - 1);
                const uint32_t *src = reinterpret_cast<const uint32_t *>(
                    w + static_cast<size_t>(r) * row_bytes + static_cast<size_t>(p) * 36);
                const kk::u32x4_a4 a = kk::load_u32x4(src);
                const kk::u32x4_a4 c = kk::load_u32x4(src + 4);
                wd[u][0] = a.x; wd[u][1] = a.y; wd[u][2] = a.z; wd[u][3] = a.w;
                wd[u][4] = c.x; wd[u][5] = c.y; wd[u][6] = c.z; wd[u][7] = c.w;
                wd[u][8] = src[8];
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float xv[B][32];
                float xsum[B];
#pragma unroll
                for (int b = 0; b < B; ++b) {
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const float4 v = xl[((b * 2 + h) * 8 + q) * pairs + p];
                        xv[b][4 * q + 0] = v.x; xv[b][4 * q + 1] = v.y;
                        xv[b][4 * q + 2] = v.z; xv[b][4 * q + 3] = v.w;
                    }
                    xsum[b] = xs[(b * 2 + h) * pairs + p];
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    uint32_t nib[4];
                    float d;
                    if (h == 0) {
                        // bytes 0-1 scale, bytes 2-17 nibbles: shift by 2 bytes
                        d = kk::half_bits_to_float(wd[u][0] & 0xffffu);
#pragma unroll
                        for (int i = 0; i < 4; ++i) nib[i] = kk::align_bytes(wd[u][i + 1], wd[u][i], 2);
                    } else {
                        // bytes 18-19 scale, bytes 20-35 nibbles: dword aligned
                        d = kk::half_bits_to_float(wd[u][4] >> 16);
#pragma unroll
                        for (int i = 0; i < 4; ++i) nib[i] = wd[u][5 + i];
                    }
#pragma unroll
                    for (int b = 0; b < B; ++b) {
                        float s_lo = 0.0f, s_hi = 0.0f;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t lo = nib[i] & 0x0f0f0f0fu;   // values 4i..4i+3
                            const uint32_t hi = nib[i] & 0xf0f0f0f0u;   // 16 * values 16+4i..
                            s_lo = fmaf(kk::ubyte_to_float<0>(lo), xv[b][4 * i + 0], s_lo);
                            s_lo = fmaf(kk::ubyte_to_float<1>(lo), xv[b][4 * i + 1], s_lo);
                            s_lo = fmaf(kk::ubyte_to_float<2>(lo), xv[b][4 * i + 2], s_lo);
                            s_lo = fmaf(kk::ubyte_to_float<3>(lo), xv[b][4 * i + 3], s_lo);
                            s_hi = fmaf(kk::ubyte_to_float<0>(hi), xv[b][16 + 4 * i + 0], s_hi);
                            s_hi = fmaf(kk::ubyte_to_float<1>(hi), xv[b][16 + 4 * i + 1], s_hi);
                            s_hi = fmaf(kk::ubyte_to_float<2>(hi), xv[b][16 + 4 * i + 2], s_hi);
                            s_hi = fmaf(kk::ubyte_to_float<3>(hi), xv[b][16 + 4 * i + 3], s_hi);
                        }
                        float t = fmaf(s_hi, 0.0625f, s_lo);
                        t = fmaf(-8.0f, xsum[b], t);
                        acc[u][b] = fmaf(d, t, acc[u][b]);
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const float v = kk::wave_sum(acc[u][b]);
                if (lane == 0 && r0 + u < n) y[static_cast<size_t>(b) * y_stride + r0 + u] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_0 streaming variant. Same lane ownership (pair p = lane + 64*j of every
// row) and LDS activation layout as q4_gemv_pair, organised for HBM streaming:
//   * every wave owns a balanced contiguous row range [r_begin, r_end);
//   * work is a flat sequence of (chunk of U rows, pair slice j) items whose
//     36-byte loads are double buffered: item i+1 is in flight while item i is
//     decoded;
//   * the first item's loads are issued right after the activation loads and
//     before the activations are written to LDS, so the prologue overlaps;
//   * row sums use DPP row reductions plus four lane reads.
template <int B, int U, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void q4_gemv_stream(const uint8_t *__restrict__ w,
                                                            const float *__restrict__ x,
                                                            float *__restrict__ y, int k, int n, int y_stride) {
    extern __shared__ float4 lds[];
    constexpr int kGroupThreads = 64 * WAVES;
    const int blocks = k >> 5;
    const int pairs = blocks >> 1;
    const int slices = (pairs + kWave - 1) / kWave;
    const size_t row_bytes = static_cast<size_t>(blocks) * 18;
    float4 *xl = lds;
    float *xs = reinterpret_cast<float *>(lds + static_cast<size_t>(B) * 8 * blocks);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = blockIdx.x * WAVES + (threadIdx.x >> 6);
    const int waves = gridDim.x * WAVES;
    const int r_begin = static_cast<int>(static_cast<long long>(n) * wave / waves);
    const int r_end = static_cast<int>(static_cast<long long>(n) * (wave + 1) / waves);
    const int chunks = (r_end - r_begin + U - 1) / U;
    const int items = chunks * slices;

    auto load_item = [&](int item, uint32_t (&buf)[U][9]) {
        const int c = item / slices, j = item - c * slices;
        const int p = lane + kWave * j;
        const int r0 = r_begin + c * U;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int r = min(r0 + u, r_end - 1);
            if (p < pairs) {
                const uint32_t *src = reinterpret_cast<const uint32_t *>(
                    w + static_cast<size_t>(r) * row_bytes + static_cast<size_t>(p) * 36);
                const kk::u32x4_a4 a = kk::load_u32x4(src);
                const kk::u32x4_a4 b = kk::load_u32x4(src + 4);
                buf[u][0] = a.x; buf[u][1] = a.y; buf[u][2] = a.z; buf[u][3] = a.w;
                buf[u][4] = b.x; buf[u][5] = b.y; buf[u][6] = b.z; buf[u][7] = b.w;
                buf[u][8] = src[8];
            } else {
#pragma unroll
                for (int i = 0; i < 9; ++i) buf[u][i] = 0u;   // zero scale: contributes 0
            }
        }
    };

    // Activation loads first, then the first weight item, then the LDS writes:
    // the weight loads stay in flight across the staging barrier.
    constexpr int kStageMax = 1;   // blocks staged per thread per pass
    uint32_t wa[U][9], wb[U][9];
    for (int base = 0; base < B * blocks; base += kGroupThreads * kStageMax) {
        float4 v[kStageMax][8];
#pragma unroll
        for (int s = 0; s < kStageMax; ++s) {
            const int idx = base + s * kGroupThreads + threadIdx.x;
            if (idx < B * blocks) {
                const int b = idx / blocks, blk = idx - b * blocks;
                const float4 *src = reinterpret_cast<const float4 *>(x + static_cast<size_t>(b) * k + blk * 32);
#pragma unroll
                for (int q = 0; q < 8; ++q) v[s][q] = src[q];
            }
        }
        if (base == 0 && items > 0) load_item(0, wa);
#pragma unroll
        for (int s = 0; s < kStageMax; ++s) {
            const int idx = base + s * kGroupThreads + threadIdx.x;
            if (idx < B * blocks) {
                const int b = idx / blocks, blk = idx - b * blocks;
                const int p = blk >> 1, h = blk & 1;
                float sum = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    xl[((b * 2 + h) * 8 + q) * pairs + p] = v[s][q];
                    sum += (v[s][q].x + v[s][q].y) + (v[s][q].z + v[s][q].w);
                }
                xs[(b * 2 + h) * pairs + p] = sum;
            }
        }
    }
    __syncthreads();

    float acc[U][B];
    auto compute_item = [&](int item, const uint32_t (&buf)[U][9]) {
        const int c = item / slices, j = item - c * slices;
        if (j == 0) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int b = 0; b < B; ++b) acc[u][b] = 0.0f;
        }
        const int p = min(lane + kWave * j, pairs - 1);   // idle lanes read a valid slot, add 0
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float xv[B][32];
            float xsum[B];
#pragma unroll
            for (int b = 0; b < B; ++b) {
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 v = xl[((b * 2 + h) * 8 + q) * pairs + p];
                    xv[b][4 * q + 0] = v.x; xv[b][4 * q + 1] = v.y;
                    xv[b][4 * q + 2] = v.z; xv[b][4 * q + 3] = v.w;
                }
                xsum[b] = xs[(b * 2 + h) * pairs + p];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                uint32_t nib[4];
                float d;
                if (h == 0) {
                    d = kk::half_bits_to_float(buf[u][0] & 0xffffu);
#pragma unroll
                    for (int i = 0; i < 4; ++i) nib[i] = kk::align_bytes(buf[u][i + 1], buf[u][i], 2);
                } else {
                    d = kk::half_bits_to_float(buf[u][4] >> 16);
#pragma unroll
                    for (int i = 0; i < 4; ++i) nib[i] = buf[u][5 + i];
                }
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    float s_lo = 0.0f, s_hi = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t lo = nib[i] & 0x0f0f0f0fu;
                        const uint32_t hi = nib[i] & 0xf0f0f0f0u;
                        s_lo = fmaf(kk::ubyte_to_float<0>(lo), xv[b][4 * i + 0], s_lo);
                        s_lo = fmaf(kk::ubyte_to_float<1>(lo), xv[b][4 * i + 1], s_lo);
                        s_lo = fmaf(kk::ubyte_to_float<2>(lo), xv[b][4 * i + 2], s_lo);
                        s_lo = fmaf(kk::ubyte_to_float<3>(lo), xv[b][4 * i + 3], s_lo);
                        s_hi = fmaf(kk::ubyte_to_float<0>(hi), xv[b][16 + 4 * i + 0], s_hi);
                        s_hi = fmaf(kk::ubyte_to_float<1>(hi), xv[b][16 + 4 * i + 1], s_hi);
                        s_hi = fmaf(kk::ubyte_to_float<2>(hi), xv[b][16 + 4 * i + 2], s_hi);
                        s_hi = fmaf(kk::ubyte_to_float<3>(hi), xv[b][16 + 4 * i + 3], s_hi);
                    }
                    float t = fmaf(s_hi, 0.0625f, s_lo);
                    t = fmaf(-8.0f, xsum[b], t);
                    acc[u][b] = fmaf(d, t, acc[u][b]);
                }
            }
        }
        if (j == slices - 1) {
            const int r0 = r_begin + c * U;
#pragma unroll
            for (int u = 0; u < U; ++u) {
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    const float v = kk::wave_sum_uniform(acc[u][b]);
                    if (lane == 0 && r0 + u < r_end) y[static_cast<size_t>(b) * y_stride + r0 + u] = v;
                }
            }
        }
    };

    for (int item = 0; item < items; item += 2) {
        if (item + 1 < items) load_item(item + 1, wb);
        compute_item(item, wa);
        if (item + 2 < items) load_item(item + 2, wa);
        if (item + 1 < items) compute_item(item + 1, wb);
    }
}

// ---------------------------------------------------------------------------
// Q4_0 with integer block dot products (v_dot8_i32_i4).
//
// Each 32-value activation block is represented as X_j = rint(x_j * 2^(22-e)),
// where 2^e > max|x| of the block (frexp exponent), i.e. a 23-bit signed
// fixed-point value with block scale s = 2^(e-22); |x_j - s X_j| <= s/2 <=
// max|x|*2^-22. X_j is written in six balanced base-16 digits in [-8, 7]:
// Z = (X + 0x888888) ^ 0x888888 holds them directly as 4-bit two's-complement
// nibbles. A weight nibble q becomes the signed value q - 8 by q ^ 8. Then
//   S = sum_j (q_j - 8) X_j = sum_l 16^l sum_j (q_j - 8) digit_l(X_j)
// is computed exactly in int32 (|S| <= 32*8*2^22 = 2^30) with 24 v_dot8
// (8 products each) per block and row, accumulated from the top digit down
// (Horner), and y += float(S) * (d * s). About 1.2 VALU ops per weight,
// against about 2.4 for the F32 decode of q4_gemv_stream.
//
// Digit dwords are packed in the weight nibble order: dword i of a block's 16
// nibble bytes holds values (4i, 16+4i, 4i+1, 16+4i+1, ..., 4i+3, 16+4i+3) in
// nibbles 0..7, so digit dword D[i][l] holds digit l of the same values.
// LDS layout per batch column b and block half h of pair p: six uint4 groups
// of the 24 dwords (i*6 + l), stored [b][h][group][p] (lanes read
// consecutive uint4: conflict-free), then the block scales [b][h][p].
// A non-finite activation makes its block scale NaN: every output row of that
// batch column becomes NaN.
// Every global load is branch-free (clamped addresses, inactive lanes zero
// their block scale) and the loop issues no vector stores (row results are
// parked in LDS and written once, coalesced, at the end), so the waitcnt
// counters stay exact and DEPTH items remain in flight while one is decoded.
// All activation loads are issued before the first weight items (the memory
// counter is in order), then converted while those weights are in flight.
constexpr int kDot8MaxRowsPerWave = 64;

// PASSES = activation staging passes: B * (K/32) * 4 <= PASSES * 64 * WAVES.
// SLICES = ceil(K / 4096): 64-pair slices per row. Rows are split over the
// grid's waves as base or base+1 contiguous rows (rem waves get one more).
// PAIR (U = 2): an item is output row r of both the gate matrix w and the up
// matrix w2, and the row result is SiLU(gate) * up (the swiglu kernel's
// element function), so the pair reads X once and needs no second pass.
template <int B, int U, int WAVES, int SLICES, int DEPTH, int PASSES, bool PAIR = false>
__global__ __launch_bounds__(64 * WAVES) void q4_gemv_dot8(const uint8_t *__restrict__ w,
                                                          const uint8_t *__restrict__ w2,
                                                          const float *__restrict__ x,
                                                          float *__restrict__ y, int k, int n, int y_stride,
                                                          int rows_base, int rows_rem) {
    extern __shared__ uint4 lds4[];
    constexpr int kGroupThreads = 64 * WAVES;
    constexpr bool ONE_SLICE = SLICES == 1;
    const int blocks = k >> 5;
    const int pairs = blocks >> 1;
    constexpr int slices = SLICES;
    const size_t row_bytes = static_cast<size_t>(blocks) * 18;
    uint4 *digits = lds4;                                                                   // [B][2][6][pairs]
    float *scales = reinterpret_cast<float *>(lds4 + static_cast<size_t>(B) * 12 * pairs);  // [B][2][pairs]
    float *results = scales + static_cast<size_t>(B) * 2 * pairs;                           // [WAVES][B][64]

    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int wave = blockIdx.x * WAVES + wid;
    const int r_begin = wave * rows_base + min(wave, rows_rem);
    const int rows = rows_base + (wave < rows_rem ? 1 : 0);   // 0 <= rows <= kDot8MaxRowsPerWave
    const int r_end = r_begin + rows;
    static_assert(!PAIR || U == 2, "a pair item is one gate row and one up row");
    const int chunks = PAIR ? rows : (rows + U - 1) / U;
    const int items = chunks * slices;
    float *my_results = results + wid * B * kDot8MaxRowsPerWave;

    auto load_item = [&](int item, uint32_t (&buf)[U][9]) {
        const int it = max(0, min(item, items - 1));          // past the end: reload the last item
        const int c = ONE_SLICE ? it : it / slices;
        const int j = ONE_SLICE ? 0 : it - c * slices;
        const int p = min(lane + kWave * j, pairs - 1);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int r = max(0, min(min(r_begin + (PAIR ? c : c * U + u), r_end - 1), n - 1));
            const uint8_t *base = PAIR && u == 1 ? w2 : w;
            const uint32_t *src = reinterpret_cast<const uint32_t *>(
                base + static_cast<size_t>(r) * row_bytes + static_cast<size_t>(p) * 36);
            const kk::u32x4_a4 a = kk::load_u32x4(src);
            const kk::u32x4_a4 b = kk::load_u32x4(src + 4);
            buf[u][0] = a.x; buf[u][1] = a.y; buf[u][2] = a.z; buf[u][3] = a.w;
            buf[u][4] = b.x; buf[u][5] = b.y; buf[u][6] = b.z; buf[u][7] = b.w;
            buf[u][8] = src[8];
        }
    };

    // 1. activation loads for every staging pass: thread (b, block, i) owns the
    //    8 activations of nibble dword i of a block
    const int groups = B * blocks * 4;
    float4 xlo[PASSES], xhi[PASSES];
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const int idx = min(pass * kGroupThreads + static_cast<int>(threadIdx.x), groups - 1);
        const int b = (B > 1 && idx >= blocks * 4) ? 1 : 0;
        const int rem = idx - b * blocks * 4;
        const float *xb = x + static_cast<size_t>(b) * k + (rem >> 2) * 32 + 4 * (rem & 3);
        xlo[pass] = *reinterpret_cast<const float4 *>(xb);
        xhi[pass] = *reinterpret_cast<const float4 *>(xb + 16);
    }
    // 2. the first DEPTH weight items (kept after the activation loads)
    __builtin_amdgcn_sched_barrier(0);
    uint32_t ring[DEPTH][U][9];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        load_item(d, ring[d]);
        __builtin_amdgcn_sched_barrier(0);   // item d's loads are issued before item d+1's
    }
    // 3. activations -> block scale and six signed base-16 digit dwords
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const int idx = pass * kGroupThreads + static_cast<int>(threadIdx.x);
        const float v[8] = {xlo[pass].x, xhi[pass].x, xlo[pass].y, xhi[pass].y,
                            xlo[pass].z, xhi[pass].z, xlo[pass].w, xhi[pass].w};   // nibble order
        float m = 0.0f, bad = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float a = fabsf(v[t]);
            bad = (a <= 3.402823466e38f) ? bad : 1.0f;
            m = fmaxf(m, a);
        }
        // the four threads of a block are consecutive lanes of one quad
        m = fmaxf(m, kk::dpp_move<0xb1>(m));
        m = fmaxf(m, kk::dpp_move<0x4e>(m));
        bad = fmaxf(bad, kk::dpp_move<0xb1>(bad));
        bad = fmaxf(bad, kk::dpp_move<0x4e>(bad));
        // 2^(e-1) <= m < 2^e (e = 0 for m == 0); e is kept >= -100 so that
        // 2^(22-e) stays finite (blocks below 2^-100 lose relative precision only).
        const int e = max(__builtin_amdgcn_frexp_expf(m), -100);
        uint32_t dig[6];
        kk::fixed_point_digits(v, ldexpf(1.0f, 22 - e), dig);
        if (idx < groups) {
            const int b = (B > 1 && idx >= blocks * 4) ? 1 : 0;
            const int rem = idx - b * blocks * 4;
            const int blk = rem >> 2, i = rem & 3;
            const int p = blk >> 1, h = blk & 1;
            uint32_t *dst = reinterpret_cast<uint32_t *>(digits);
#pragma unroll
            for (int l = 0; l < 6; ++l) {
                const int pos = i * 6 + l;
                dst[((static_cast<size_t>(b * 2 + h) * 6 + (pos >> 2)) * pairs + p) * 4 + (pos & 3)] = dig[l];
            }
            if (i == 0)
                scales[(b * 2 + h) * pairs + p] = bad != 0.0f ? __builtin_nanf("") : ldexpf(1.0f, e - 22);
        }
    }
    __syncthreads();

    // 4. decode: one item = U rows x one 64-pair slice
    float acc[U][B];
    uint4 dg[B][2][6];
    float sc[B][2];
    auto read_slice = [&](int p) {
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int g = 0; g < 6; ++g) dg[b][h][g] = digits[(static_cast<size_t>(b * 2 + h) * 6 + g) * pairs + p];
                sc[b][h] = scales[(b * 2 + h) * pairs + p];
            }
    };
    if (ONE_SLICE) read_slice(min(lane, pairs - 1));

    auto compute_item = [&](int item, const uint32_t (&buf)[U][9]) {
        const int c = ONE_SLICE ? item : item / slices;
        const int j = ONE_SLICE ? 0 : item - c * slices;
        if (j == 0) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int b = 0; b < B; ++b) acc[u][b] = 0.0f;
        }
        const bool live = lane + kWave * j < pairs;           // lanes past the row end add 0
        if (!ONE_SLICE) read_slice(min(lane + kWave * j, pairs - 1));
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t q[4];
                float d;
                if (h == 0) {
                    d = kk::half_bits_to_float(buf[u][0] & 0xffffu);
#pragma unroll
                    for (int i = 0; i < 4; ++i) q[i] = kk::align_bytes(buf[u][i + 1], buf[u][i], 2) ^ 0x88888888u;
                } else {
                    d = kk::half_bits_to_float(buf[u][4] >> 16);
#pragma unroll
                    for (int i = 0; i < 4; ++i) q[i] = buf[u][5 + i] ^ 0x88888888u;
                }
                d = live ? d : 0.0f;
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    const uint32_t dd[24] = {
                        dg[b][h][0].x, dg[b][h][0].y, dg[b][h][0].z, dg[b][h][0].w, dg[b][h][1].x, dg[b][h][1].y,
                        dg[b][h][1].z, dg[b][h][1].w, dg[b][h][2].x, dg[b][h][2].y, dg[b][h][2].z, dg[b][h][2].w,
                        dg[b][h][3].x, dg[b][h][3].y, dg[b][h][3].z, dg[b][h][3].w, dg[b][h][4].x, dg[b][h][4].y,
                        dg[b][h][4].z, dg[b][h][4].w, dg[b][h][5].x, dg[b][h][5].y, dg[b][h][5].z, dg[b][h][5].w};
                    // six independent digit sums T_l, then S = sum_l 16^l T_l (|S| <= 2^30)
                    int t[6];
#pragma unroll
                    for (int l = 0; l < 6; ++l) {
                        t[l] = 0;
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            t[l] = __builtin_amdgcn_sdot8(static_cast<int>(q[i]), static_cast<int>(dd[i * 6 + l]), t[l], false);
                    }
                    int s = t[5];
#pragma unroll
                    for (int l = 4; l >= 0; --l) s = (s << 4) + t[l];
                    acc[u][b] = fmaf(static_cast<float>(s), d * sc[b][h], acc[u][b]);
                }
            }
        }
        if (j == slices - 1) {
            if (PAIR) {
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    const float gate = kk::wave_sum_uniform(acc[0][b]);
                    const float up = kk::wave_sum_uniform(acc[PAIR ? 1 : 0][b]);
                    if (lane == 0 && c < rows) my_results[b * kDot8MaxRowsPerWave + c] = kk::swiglu_value(gate, up);
                }
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int rr = c * U + u;
#pragma unroll
                    for (int b = 0; b < B; ++b) {
                        const float v = kk::wave_sum_uniform(acc[u][b]);
                        if (lane == 0 && rr < rows) my_results[b * kDot8MaxRowsPerWave + rr] = v;
                    }
                }
            }
        }
    };

    // Ring of DEPTH items in flight: after item i is decoded its buffer is
    // refilled with item i + DEPTH (clamped: past the end it re-reads the
    // last item, which hits in cache).
    for (int base = 0; base < items; base += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int item = base + d;
            if (item < items) compute_item(item, ring[d]);
            load_item(item + DEPTH, ring[d]);
        }
    }

    // 5. row results: one coalesced store per batch column
    __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int b = 0; b < B; ++b)
        if (lane < rows) y[static_cast<size_t>(b) * y_stride + r_begin + lane] = my_results[b * kDot8MaxRowsPerWave + lane];
}

// ---------------------------------------------------------------------------
// F32 / F16 rows. LDS holds X[b][k] as float4 (natural order).
template <int B, int U, bool F16>
__global__ __launch_bounds__(kThreads) void dense_gemv(const uint8_t *__restrict__ w,
                                                      const float *__restrict__ x,
                                                      float *__restrict__ y, int k, int n,
                                                      int y_stride) {
    extern __shared__ float4 lds[];
    const int k4 = k >> 2;
    for (int idx = threadIdx.x; idx < B * k4; idx += kThreads) {
        const int b = idx / k4, i = idx - b * k4;
        lds[idx] = reinterpret_cast<const float4 *>(x + static_cast<size_t>(b) * k)[i];
    }
    __syncthreads();

    constexpr int kPerLane = F16 ? 8 : 4;             // values per 16-byte chunk
    constexpr int kStep = kPerLane * kWave;           // values per wave step
    const size_t row_bytes = static_cast<size_t>(k) * (F16 ? 2 : 4);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = blockIdx.x * kWavesPerGroup + (threadIdx.x >> 6);
    const int waves = gridDim.x * kWavesPerGroup;
    const int rowblocks = (n + U - 1) / U;

    for (int rb = wave; rb < rowblocks; rb += waves) {
        const int r0 = rb * U;
        float acc[U][B];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int b = 0; b < B; ++b) acc[u][b] = 0.0f;

        for (int k0 = lane * kPerLane; k0 < k; k0 += kStep) {
            uint4 wv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int r = min(r0 + u, n - 1);
                wv[u] = *reinterpret_cast<const uint4 *>(w + static_cast<size_t>(r) * row_bytes +
                                                         static_cast<size_t>(k0) * (F16 ? 2 : 4));
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                float xv[kPerLane];
#pragma unroll
                for (int q = 0; q < kPerLane / 4; ++q) {
                    const float4 v = lds[b * k4 + (k0 >> 2) + q];
                    xv[4 * q + 0] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t words[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
                    float s = acc[u][b];
                    if (F16) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            s = fmaf(kk::half_bits_to_float(words[i] & 0xffffu), xv[2 * i], s);
                            s = fmaf(kk::half_bits_to_float(words[i] >> 16), xv[2 * i + 1], s);
                        }
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) s = fmaf(__uint_as_float(words[i]), xv[i], s);
                    }
                    acc[u][b] = s;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const float v = kk::wave_sum(acc[u][b]);
                if (lane == 0 && r0 + u < n) y[static_cast<size_t>(b) * y_stride + r0 + u] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// General fallback: any weight alignment, any K % 32, any batch. One wave per
// row, lanes stride over 32-value blocks, byte loads, up to 8 batch columns
// per pass.
constexpr int kGeneralBatch = 8;

__device__ __forceinline__ uint32_t load_u16_bytes(const uint8_t *p) {
    return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8);
}

__global__ __launch_bounds__(kThreads) void gemv_general(const uint8_t *__restrict__ w, int type,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int k, int n, int batch) {
    const int blocks = k >> 5;
    const size_t row_bytes = type == 2 ? static_cast<size_t>(blocks) * 18
                                       : static_cast<size_t>(k) * (type == 1 ? 2 : 4);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = blockIdx.x * kWavesPerGroup + (threadIdx.x >> 6);
    const int waves = gridDim.x * kWavesPerGroup;
    for (int r = wave; r < n; r += waves) {
        const uint8_t *row = w + static_cast<size_t>(r) * row_bytes;
        for (int b0 = 0; b0 < batch; b0 += kGeneralBatch) {
            float acc[kGeneralBatch];
#pragma unroll
            for (int j = 0; j < kGeneralBatch; ++j) acc[j] = 0.0f;
            for (int blk = lane; blk < blocks; blk += kWave) {
                float q[32];
                float d = 1.0f;
                if (type == 2) {
                    const uint8_t *p = row + static_cast<size_t>(blk) * 18;
                    d = kk::half_bits_to_float(load_u16_bytes(p));
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        q[j] = static_cast<float>(static_cast<int>(p[2 + j] & 15) - 8);
                        q[j + 16] = static_cast<float>(static_cast<int>(p[2 + j] >> 4) - 8);
                    }
                } else if (type == 1) {
                    const uint8_t *p = row + static_cast<size_t>(blk) * 64;
#pragma unroll
                    for (int j = 0; j < 32; ++j) q[j] = kk::half_bits_to_float(load_u16_bytes(p + 2 * j));
                } else {
                    const uint8_t *p = row + static_cast<size_t>(blk) * 128;
#pragma unroll
                    for (int j = 0; j < 32; ++j)
                        q[j] = __uint_as_float(load_u16_bytes(p + 4 * j) | (load_u16_bytes(p + 4 * j + 2) << 16));
                }
#pragma unroll
                for (int j = 0; j < kGeneralBatch; ++j) {
                    if (b0 + j < batch) {
                        const float *xb = x + static_cast<size_t>(b0 + j) * k + static_cast<size_t>(blk) * 32;
                        float s = 0.0f;
#pragma unroll
                        for (int i = 0; i < 32; ++i) s = fmaf(q[i], xb[i], s);
                        acc[j] = fmaf(d, s, acc[j]);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < kGeneralBatch; ++j) {
                const float v = kk::wave_sum(acc[j]);
                if (lane == 0 && b0 + j < batch) y[static_cast<size_t>(b0 + j) * n + r] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Launch helpers.

struct DeviceInfo {
    int cus = 256;
    int lds_max = 65536;
};

DeviceInfo device_info() {
    static thread_local int cached_device = -1;
    static thread_local DeviceInfo info;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return info;
    if (device != cached_device) {
        int value = 0;
        if (hipDeviceGetAttribute(&value, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && value > 0)
            info.cus = value;
        if (hipDeviceGetAttribute(&value, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess && value > 0)
            info.lds_max = value;
        cached_device = device;
    }
    return info;
}

int env_int(const char *name, int fallback) {
    const char *value = std::getenv(name);
    return value && *value ? std::atoi(value) : fallback;
}

// Workgroup count for a row-blocked kernel: enough waves for every row block
// up to `per_cu` waves per CU.
int groups_for(int rowblocks, int cus, int per_cu_waves) {
    const long long cap = static_cast<long long>(cus) * per_cu_waves;
    const long long waves = std::min<long long>(rowblocks, cap);
    return static_cast<int>(std::max<long long>(1, (waves + kWavesPerGroup - 1) / kWavesPerGroup));
}

template <int B>
hipError_t launch_q4_pair(const uint8_t *w, const float *x, float *y, int k, int n, int y_stride,
                          hipStream_t stream, const DeviceInfo &info) {
    constexpr int U = 4;
    const size_t lds = static_cast<size_t>(B) * k * 4 + static_cast<size_t>(B) * (k / 32) * 4;
    const int rowblocks = (n + U - 1) / U;
    const int groups = groups_for(rowblocks, info.cus, env_int("KUNLUN_GEMV_WAVES_PER_CU", 8));
    hipError_t rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&q4_gemv_pair<B, U>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    (void)rc;
    hipLaunchKernelGGL((q4_gemv_pair<B, U>), dim3(groups), dim3(kThreads), lds, stream, w, x, y, k, n, y_stride);
    return hipGetLastError();
}

template <int B, int U, int WAVES>
hipError_t launch_q4_stream(const uint8_t *w, const float *x, float *y, int k, int n, int y_stride,
                            hipStream_t stream, const DeviceInfo &info) {
    const size_t lds = static_cast<size_t>(B) * k * 4 + static_cast<size_t>(B) * (k / 32) * 4;
    const int per_cu = env_int("KUNLUN_GEMV_WAVES_PER_CU", 16);
    const long long want = std::min<long long>(n, static_cast<long long>(info.cus) * per_cu);
    const int groups = static_cast<int>(std::max<long long>(1, (want + WAVES - 1) / WAVES));
    hipError_t rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&q4_gemv_stream<B, U, WAVES>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    (void)rc;
    hipLaunchKernelGGL((q4_gemv_stream<B, U, WAVES>), dim3(groups), dim3(64 * WAVES), lds, stream, w, x, y, k, n,
                       y_stride);
    return hipGetLastError();
}

template <int B, int SLICES, int DEPTH, bool PAIR = false>
hipError_t launch_q4_dot8_depth(const uint8_t *w, const uint8_t *w2, const float *x, float *y, int k, int n,
                                int y_stride, hipStream_t stream, const DeviceInfo &info) {
    constexpr int kWaves = 8, kU = PAIR ? 2 : 1;
    constexpr int kPasses = B * SLICES;   // B * K/8 staging groups <= B * SLICES * 512
    const size_t lds = static_cast<size_t>(B) * (k / 32) * 100 + static_cast<size_t>(kWaves) * B * kDot8MaxRowsPerWave * 4;
    const int per_cu = env_int("KUNLUN_GEMV_WAVES_PER_CU", 8);
    long long want = std::min<long long>(n, static_cast<long long>(info.cus) * per_cu);
    want = std::max<long long>(want, (n + kDot8MaxRowsPerWave - 1) / kDot8MaxRowsPerWave);
    const int groups = static_cast<int>(std::max<long long>(1, (want + kWaves - 1) / kWaves));
    const int waves = groups * kWaves;
    const int rows_base = n / waves, rows_rem = n % waves;
    auto kernel = &q4_gemv_dot8<B, kU, kWaves, SLICES, DEPTH, kPasses, PAIR>;
    static bool attribute_set = false;    // per instantiation
    if (!attribute_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  64 * 1024);
        attribute_set = true;
    }
    hipLaunchKernelGGL(kernel, dim3(groups), dim3(64 * kWaves), lds, stream, w, w2, x, y, k, n, y_stride, rows_base,
                       rows_rem);
    return hipGetLastError();
}

template <int B, int SLICES, bool PAIR>
hipError_t launch_q4_dot8_slices(const uint8_t *w, const uint8_t *w2, const float *x, float *y, int k, int n,
                                 int y_stride, hipStream_t stream, const DeviceInfo &info) {
    // items in flight per wave: 3 single rows at batch 1; 2 when an item is
    // twice the work (two batch columns, or a gate/up row pair)
    switch (env_int("KUNLUN_Q4_DEPTH", B == 2 || PAIR ? 2 : 3)) {
    case 2: return launch_q4_dot8_depth<B, SLICES, 2, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
    case 4: return launch_q4_dot8_depth<B, SLICES, 4, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
    default: return launch_q4_dot8_depth<B, SLICES, 3, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
    }
}

// Q4_0 batch chunk of B (1 or 2) columns; B * K <= 16384. PAIR: w is the gate
// matrix, w2 the up matrix, y = SiLU(X w^T) * (X w2^T).
template <int B, bool PAIR = false>
hipError_t launch_q4_dot8(const uint8_t *w, const uint8_t *w2, const float *x, float *y, int k, int n, int y_stride,
                          hipStream_t stream, const DeviceInfo &info) {
    const int slices = (k + 4095) / 4096;
    if (B == 2 || slices <= 1) {
        if (slices <= 1) return launch_q4_dot8_slices<B, 1, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
        return launch_q4_dot8_slices<B, 2, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
    }
    if (slices == 2) return launch_q4_dot8_slices<1, 2, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
    if (slices == 3) return launch_q4_dot8_slices<1, 3, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
    return launch_q4_dot8_slices<1, 4, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
}

template <int B, bool F16>
hipError_t launch_dense(const uint8_t *w, const float *x, float *y, int k, int n, int y_stride,
                        hipStream_t stream, const DeviceInfo &info) {
    constexpr int U = 4;
    const size_t lds = static_cast<size_t>(B) * k * 4;
    const int rowblocks = (n + U - 1) / U;
    const int groups = groups_for(rowblocks, info.cus, env_int("KUNLUN_GEMV_WAVES_PER_CU", 8));
    hipError_t rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&dense_gemv<B, U, F16>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    (void)rc;
    hipLaunchKernelGGL((dense_gemv<B, U, F16>), dim3(groups), dim3(kThreads), lds, stream, w, x, y, k, n, y_stride);
    return hipGetLastError();
}

// Largest batch chunk (<= 4) whose staged activations fit in LDS.
int lds_batch_chunk(int type, int k, int lds_max) {
    const size_t per_column = static_cast<size_t>(k) * 4 + (type == 2 ? static_cast<size_t>(k / 32) * 4 : 0);
    for (int b = 4; b >= 1; --b)
        if (per_column * b <= static_cast<size_t>(lds_max)) return b;
    return 0;
}

} // namespace

extern "C" int kk_dense_matmul(int type, const void *w, const float *x, float *y, int k, int n, int batch,
                               hipStream_t stream, const char **route) {
    if (type < 0 || type > 2 || k <= 0 || (k & 31) || n <= 0 || batch <= 0 || !w || !x || !y)
        return hipErrorInvalidValue;
    const DeviceInfo info = device_info();
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    const bool x16 = (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const bool force_general = env_int("KUNLUN_GEMV_GENERAL", 0) != 0;

    bool fast = false;
    if (!force_general && x16) {
        if (type == 2) fast = (k % 64) == 0 && (wa & 3) == 0;
        else fast = (wa & 15) == 0;
    }
    const int chunk = fast ? lds_batch_chunk(type, k, info.lds_max) : 0;
    if (chunk == 0) {
        if (route) *route = "gemv_general";
        const int groups = groups_for(n, info.cus, 16);
        hipLaunchKernelGGL(gemv_general, dim3(groups), dim3(kThreads), 0, stream, wb, type, x, y, k, n, batch);
        return hipGetLastError();
    }
    const int q4_kernel = type == 2 ? env_int("KUNLUN_Q4_KERNEL", 0) : -1;   // 0 dot8, 1 stream, 2 pair
    if (q4_kernel == 0) {
        if (route) *route = "q4_gemv_dot8";
        const int pair_batch = k <= 8192 ? 2 : 1;   // staged digits: B * K <= 16384
        for (int b0 = 0; b0 < batch; b0 += pair_batch) {
            const int bc = std::min(pair_batch, batch - b0);
            const float *xc = x + static_cast<size_t>(b0) * k;
            float *yc = y + static_cast<size_t>(b0) * n;
            const hipError_t rc = bc == 1 ? launch_q4_dot8<1>(wb, wb, xc, yc, k, n, n, stream, info)
                                          : launch_q4_dot8<2>(wb, wb, xc, yc, k, n, n, stream, info);
            if (rc != hipSuccess) return rc;
        }
        return hipSuccess;
    }
    const bool q4_stream = q4_kernel == 1;
    if (route) *route = type == 2 ? (q4_stream ? "q4_gemv_stream" : "q4_gemv_pair") : type == 1 ? "f16_gemv" : "f32_gemv";
    if (q4_stream) {
        const int u = env_int("KUNLUN_Q4_ROWS", 2), waves = env_int("KUNLUN_Q4_WAVES", 8);
        const int sc = std::min(chunk, 2);
        for (int b0 = 0; b0 < batch; b0 += sc) {
            const int bc = std::min(sc, batch - b0);
            const float *xc = x + static_cast<size_t>(b0) * k;
            float *yc = y + static_cast<size_t>(b0) * n;
            hipError_t rc;
            if (bc == 1) {
                if (u == 4) rc = waves == 4 ? launch_q4_stream<1, 4, 4>(wb, xc, yc, k, n, n, stream, info)
                                            : launch_q4_stream<1, 4, 8>(wb, xc, yc, k, n, n, stream, info);
                else if (u == 1) rc = waves == 4 ? launch_q4_stream<1, 1, 4>(wb, xc, yc, k, n, n, stream, info)
                                                 : launch_q4_stream<1, 1, 8>(wb, xc, yc, k, n, n, stream, info);
                else rc = waves == 4 ? launch_q4_stream<1, 2, 4>(wb, xc, yc, k, n, n, stream, info)
                                     : launch_q4_stream<1, 2, 8>(wb, xc, yc, k, n, n, stream, info);
            } else {
                rc = waves == 4 ? launch_q4_stream<2, 2, 4>(wb, xc, yc, k, n, n, stream, info)
                                : launch_q4_stream<2, 2, 8>(wb, xc, yc, k, n, n, stream, info);
            }
            if (rc != hipSuccess) return rc;
        }
        return hipSuccess;
    }
    for (int b0 = 0; b0 < batch; b0 += chunk) {
        const int bc = std::min(chunk, batch - b0);
        const float *xc = x + static_cast<size_t>(b0) * k;
        float *yc = y + static_cast<size_t>(b0) * n;
        hipError_t rc = hipSuccess;
        if (type == 2) {
            switch (bc) {
            case 1: rc = launch_q4_pair<1>(wb, xc, yc, k, n, n, stream, info); break;
            case 2: rc = launch_q4_pair<2>(wb, xc, yc, k, n, n, stream, info); break;
            case 3: rc = launch_q4_pair<3>(wb, xc, yc, k, n, n, stream, info); break;
            default: rc = launch_q4_pair<4>(wb, xc, yc, k, n, n, stream, info); break;
            }
        } else if (type == 1) {
            switch (bc) {
            case 1: rc = launch_dense<1, true>(wb, xc, yc, k, n, n, stream, info); break;
            case 2: rc = launch_dense<2, true>(wb, xc, yc, k, n, n, stream, info); break;
            case 3: rc = launch_dense<3, true>(wb, xc, yc, k, n, n, stream, info); break;
            default: rc = launch_dense<4, true>(wb, xc, yc, k, n, n, stream, info); break;
            }
        } else {
            switch (bc) {
            case 1: rc = launch_dense<1, false>(wb, xc, yc, k, n, n, stream, info); break;
            case 2: rc = launch_dense<2, false>(wb, xc, yc, k, n, n, stream, info); break;
            case 3: rc = launch_dense<3, false>(wb, xc, yc, k, n, n, stream, info); break;
            default: rc = launch_dense<4, false>(wb, xc, yc, k, n, n, stream, info); break;
            }
        }
        if (rc != hipSuccess) return rc;
    }
    return hipSuccess;
}

extern "C" int kk_q4_gemv_pair_swiglu_supported(const void *w_gate, const void *w_up, const float *x, int k, int n,
                                                int batch) {
    return w_gate && w_up && x && k > 0 && n > 0 && (k % 64) == 0 && k <= 16384 && batch >= 1 && batch <= 2 &&
           (reinterpret_cast<uintptr_t>(w_gate) & 3) == 0 && (reinterpret_cast<uintptr_t>(w_up) & 3) == 0 &&
           (reinterpret_cast<uintptr_t>(x) & 15) == 0 && env_int("KUNLUN_GEMV_GENERAL", 0) == 0 &&
           env_int("KUNLUN_Q4_KERNEL", 0) == 0;
}

extern "C" int kk_q4_gemv_pair_swiglu(const void *w_gate, const void *w_up, const float *x, float *y, int k, int n,
                                     int batch, hipStream_t stream) {
    if (!y || !kk_q4_gemv_pair_swiglu_supported(w_gate, w_up, x, k, n, batch)) return hipErrorInvalidValue;
    const DeviceInfo info = device_info();
    const uint8_t *wg = static_cast<const uint8_t *>(w_gate);
    const uint8_t *wu = static_cast<const uint8_t *>(w_up);
    const int pair_batch = k <= 8192 ? 2 : 1;   // staged digits: B * K <= 16384
    for (int b0 = 0; b0 < batch; b0 += pair_batch) {
        const int bc = std::min(pair_batch, batch - b0);
        const float *xc = x + static_cast<size_t>(b0) * k;
        float *yc = y + static_cast<size_t>(b0) * n;
        const hipError_t rc = bc == 1 ? launch_q4_dot8<1, true>(wg, wu, xc, yc, k, n, n, stream, info)
                                      : launch_q4_dot8<2, true>(wg, wu, xc, yc, k, n, n, stream, info);
        if (rc != hipSuccess) return rc;
    }
    return hipSuccess;
}
