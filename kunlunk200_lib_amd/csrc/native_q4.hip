// GEMV over the native Q4 layout (reference src/q4-layout.cpp:15-37,
// src/k200.cpp:554-617) on gfx950.
//
// Layout: for N32 tile t and K32 block b, 512 bytes at (t * blocks + b) * 512
// hold byte [pair j][lane r] = signed nibbles of row 32t + r, K 32b + 2j (low)
// and 32b + 2j + 1 (high); after the 256-byte aligned payload, 32 FP16 block
// scales per tile-block at (t * blocks + b) * 32 + r. Rows past N are zero.
//
// Arithmetic is exact up to the activation representation: each 32-value
// activation block is a 23-bit signed fixed point with a power-of-two block
// scale s_b (kk::fixed_point_digits), so sum_j q_j X_j is an exact int32 from
// 24 v_dot8_i32_i4 per row and block, and y_r += float(S) * (d_rb * s_b) in F32.
//
// Work split: one workgroup per half tile (16 rows); the two halves of a tile
// run on the same XCD (workgroup i runs on XCD i % 8), so the second reads the
// tile's cache lines from L2. The workgroup's waves take items of 16 K32
// blocks in turn. In an item, lane l owns block 16i + l/4 and rows
// 16h + 4(l%4) .. +3: it loads the 16 pair dwords of those rows (stride 32
// bytes; the 4 lanes of a block read 16 contiguous bytes per pair) and turns
// each group of four pair dwords into four row dwords of 8 consecutive K
// values with a 4 x 4 byte transpose (8 v_perm_b32). Activation loads are
// issued first, then the first weight items, then the activations are
// converted while the weights are in flight (the memory counter is in order).
// Rows are reduced over lanes, then over waves in a fixed order: results are
// bitwise reproducible.
#include "device_common.h"
#include "launch.h"

#include <algorithm>

namespace {

constexpr int kNqWaves = 8;
constexpr int kNqThreads = 64 * kNqWaves;
constexpr int kNqDepth = 2;                 // items in flight per wave
constexpr int kNqLanesPerBlock = 4;         // 4 lanes x 4 rows = one half tile
constexpr int kNqItemBlocks = 64 / kNqLanesPerBlock;
constexpr int kNqRows = 16;                 // rows per workgroup
constexpr int kNqMaxColumns = 4;            // batch columns per launch
constexpr int kNqMaxPasses = 6;             // activation staging passes (8 values per thread each)
constexpr size_t kNqLdsLimit = 64 * 1024;

size_t lds_bytes(int blocks, int columns) {
    // per column and block: 24 digit dwords and one scale; per wave and
    // column: the workgroup's row partials
    return static_cast<size_t>(columns) * blocks * (96 + 4) + static_cast<size_t>(kNqWaves) * columns * kNqRows * 4;
}

int passes_for(int blocks, int columns) { return (columns * blocks * 4 + kNqThreads - 1) / kNqThreads; }

template <int B, int PASSES>
__global__ __launch_bounds__(kNqThreads) void native_q4_gemv(const uint8_t *__restrict__ w,
                                                            const uint16_t *__restrict__ scales,
                                                            const void *__restrict__ x, int x_f16,
                                                            float *__restrict__ y, int k, int n, int tiles) {
    extern __shared__ uint4 lds4[];
    // workgroup -> (tile, half): i = 16 (t / 8) + t % 8 + 8 h keeps both halves on XCD t % 8
    const int tile = (blockIdx.x >> 4) * 8 + (blockIdx.x & 7);
    const int half = (blockIdx.x >> 3) & 1;
    if (tile >= tiles) return;                    // whole workgroup: no barrier reached yet
    const int blocks = k >> 5;
    const int items = (blocks + kNqItemBlocks - 1) / kNqItemBlocks;
    uint4 *digits = lds4;                                                                      // [B][blocks][6]
    float *block_scale = reinterpret_cast<float *>(lds4 + static_cast<size_t>(B) * blocks * 6);  // [B][blocks]
    float *partial = block_scale + B * blocks;                                                 // [waves][B][16]

    const int lane = threadIdx.x & (kk::kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int c = lane & (kNqLanesPerBlock - 1);  // rows 16 half + 4c .. +3 of the tile
    const size_t tile_block0 = static_cast<size_t>(tile) * blocks;
    const int row_byte = kNqRows * half + 4 * c;

    // 1. activation loads: thread (b, block, q) of each pass owns values 8q .. 8q+7 of a block
    const int groups = B * blocks * 4;
    float xv[PASSES][8];
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const int g = min(pass * kNqThreads + static_cast<int>(threadIdx.x), groups - 1);
        const int b = g / (blocks * 4);
        const size_t base = static_cast<size_t>(b) * k + static_cast<size_t>(g - b * blocks * 4) * 8;
        if (x_f16) {
            const uint16_t *xh = static_cast<const uint16_t *>(x) + base;
#pragma unroll
            for (int t = 0; t < 8; ++t) xv[pass][t] = kk::half_bits_to_float(xh[t]);
        } else {
            const float *xf = static_cast<const float *>(x) + base;
#pragma unroll
            for (int t = 0; t < 8; ++t) xv[pass][t] = xf[t];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. the first weight items
    auto load_item = [&](int s, uint32_t (&buf)[18]) {
        const int it = min(wid + kNqWaves * s, items - 1);
        const int blk = min(it * kNqItemBlocks + lane / kNqLanesPerBlock, blocks - 1);
        const uint8_t *src = w + (tile_block0 + blk) * 512 + row_byte;
#pragma unroll
        for (int p = 0; p < 16; ++p) buf[p] = *reinterpret_cast<const uint32_t *>(src + 32 * p);
        const uint2 sc = *reinterpret_cast<const uint2 *>(scales + (tile_block0 + blk) * 32 + row_byte);
        buf[16] = sc.x;
        buf[17] = sc.y;
    };
    // every wave runs the same count of items (the last ones may add zero);
    // loads beyond that count are skipped by a uniform branch
    const int iters = (items + kNqWaves - 1) / kNqWaves;
    const int iters_padded = (iters + kNqDepth - 1) / kNqDepth * kNqDepth;
    uint32_t ring[kNqDepth][18];
#pragma unroll
    for (int d = 0; d < kNqDepth; ++d) {
        if (d < iters) load_item(d, ring[d]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // 3. activations -> block scale and six digit dwords per 8 values
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const int idx = pass * kNqThreads + static_cast<int>(threadIdx.x);
        const int g = min(idx, groups - 1);
        const int b = g / (blocks * 4);
        const int rem = g - b * blocks * 4;
        float m = 0.0f, bad = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float a = fabsf(xv[pass][t]);
            bad = (a <= 3.402823466e38f) ? bad : 1.0f;
            m = fmaxf(m, a);
        }
        // the four threads of a block are the lanes of one quad
        m = fmaxf(m, kk::dpp_move<0xb1>(m));
        m = fmaxf(m, kk::dpp_move<0x4e>(m));
        bad = fmaxf(bad, kk::dpp_move<0xb1>(bad));
        bad = fmaxf(bad, kk::dpp_move<0x4e>(bad));
        // 2^(e-1) <= m < 2^e; e >= -100 keeps 2^(22-e) finite
        const int e = max(__builtin_amdgcn_frexp_expf(m), -100);
        uint32_t dig[6];
        kk::fixed_point_digits(xv[pass], ldexpf(1.0f, 22 - e), dig);
        if (idx < groups) {
            uint32_t *dst = reinterpret_cast<uint32_t *>(digits) + static_cast<size_t>(b * blocks) * 24 + rem * 6;
#pragma unroll
            for (int l = 0; l < 6; ++l) dst[l] = dig[l];
            if ((rem & 3) == 0)
                block_scale[b * blocks + (rem >> 2)] = bad != 0.0f ? __builtin_nanf("") : ldexpf(1.0f, e - 22);
        }
    }
    __syncthreads();

    // 4. items: 4 rows x one K32 block per lane
    float acc[B][4];
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[b][r] = 0.0f;

    auto compute_item = [&](int s, const uint32_t (&buf)[18]) {
        const int it = wid + kNqWaves * s;
        const int blk_raw = it * kNqItemBlocks + lane / kNqLanesPerBlock;
        const bool live = it < items && blk_raw < blocks;
        const int blk = min(min(it, items - 1) * kNqItemBlocks + lane / kNqLanesPerBlock, blocks - 1);
        float d[4];
        d[0] = kk::half_bits_to_float(buf[16] & 0xffffu);
        d[1] = kk::half_bits_to_float(buf[16] >> 16);
        d[2] = kk::half_bits_to_float(buf[17] & 0xffffu);
        d[3] = kk::half_bits_to_float(buf[17] >> 16);
        // row dwords: o[r][q] nibble t = row 4c+r, K 8q+t (4 x 4 byte transposes)
        uint32_t o[4][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t a = buf[4 * q], bb = buf[4 * q + 1], cc = buf[4 * q + 2], dd = buf[4 * q + 3];
            const uint32_t ab_lo = __builtin_amdgcn_perm(bb, a, 0x05010400u);    // a0 b0 a1 b1
            const uint32_t ab_hi = __builtin_amdgcn_perm(bb, a, 0x07030602u);    // a2 b2 a3 b3
            const uint32_t cd_lo = __builtin_amdgcn_perm(dd, cc, 0x05010400u);
            const uint32_t cd_hi = __builtin_amdgcn_perm(dd, cc, 0x07030602u);
            o[0][q] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);          // a0 b0 c0 d0
            o[1][q] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);          // a1 b1 c1 d1
            o[2][q] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
            o[3][q] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const uint4 *dsrc = digits + (static_cast<size_t>(b) * blocks + blk) * 6;
            uint32_t dg[24];
#pragma unroll
            for (int g = 0; g < 6; ++g) {
                const uint4 v4 = dsrc[g];
                dg[4 * g] = v4.x;
                dg[4 * g + 1] = v4.y;
                dg[4 * g + 2] = v4.z;
                dg[4 * g + 3] = v4.w;
            }
            const float sb = block_scale[b * blocks + blk];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int t[6];
#pragma unroll
                for (int l = 0; l < 6; ++l) {
                    t[l] = 0;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        t[l] = __builtin_amdgcn_sdot8(static_cast<int>(o[r][q]), static_cast<int>(dg[q * 6 + l]),
                                                      t[l], false);
                }
                int sum = t[5];
#pragma unroll
                for (int l = 4; l >= 0; --l) sum = (sum << 4) + t[l];
                acc[b][r] = fmaf(static_cast<float>(sum), live ? d[r] * sb : 0.0f, acc[b][r]);
            }
        }
    };

    for (int base = 0; base < iters_padded; base += kNqDepth) {
#pragma unroll
        for (int dpt = 0; dpt < kNqDepth; ++dpt) {
            if (base + dpt < iters) compute_item(base + dpt, ring[dpt]);   // uniform; no loads inside
            if (base + dpt + kNqDepth < iters) load_item(base + dpt + kNqDepth, ring[dpt]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // 5. rows: sum the 16 lanes of each row group (fixed xor order), then the waves
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float v = acc[b][r];
            v += __shfl_xor(v, 4, kk::kWave);
            v += __shfl_xor(v, 8, kk::kWave);
            v += __shfl_xor(v, 16, kk::kWave);
            v += __shfl_xor(v, 32, kk::kWave);
            if (lane < kNqLanesPerBlock) partial[(wid * B + b) * kNqRows + 4 * c + r] = v;
        }
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < kNqRows * B) {
        const int b = threadIdx.x / kNqRows, row = threadIdx.x % kNqRows;
        float v = 0.0f;
#pragma unroll
        for (int wv = 0; wv < kNqWaves; ++wv) v += partial[(wv * B + b) * kNqRows + row];
        const int gr = tile * 32 + kNqRows * half + row;
        if (gr < n) y[static_cast<size_t>(b) * n + gr] = v;
    }
}

template <int B, int PASSES>
hipError_t launch_columns(const uint8_t *w, const uint16_t *scales, const void *x, int x_f16, float *y, int k,
                          int n, hipStream_t stream) {
    const int tiles = (n + 31) / 32;
    const int groups = 16 * ((tiles + 7) / 8);      // 8 tiles x 2 halves per group of 16 workgroups
    const size_t lds = lds_bytes(k >> 5, B);
    hipLaunchKernelGGL((native_q4_gemv<B, PASSES>), dim3(groups), dim3(kNqThreads), lds, stream, w, scales, x,
                       x_f16, y, k, n, tiles);
    return hipGetLastError();
}

template <int B>
hipError_t launch_passes(int passes, const uint8_t *w, const uint16_t *scales, const void *x, int x_f16, float *y,
                         int k, int n, hipStream_t stream) {
    switch (passes) {
    case 1: return launch_columns<B, 1>(w, scales, x, x_f16, y, k, n, stream);
    case 2: return launch_columns<B, 2>(w, scales, x, x_f16, y, k, n, stream);
    case 3: return launch_columns<B, 3>(w, scales, x, x_f16, y, k, n, stream);
    case 4: return launch_columns<B, 4>(w, scales, x, x_f16, y, k, n, stream);
    case 5: return launch_columns<B, 5>(w, scales, x, x_f16, y, k, n, stream);
    case 6: return launch_columns<B, 6>(w, scales, x, x_f16, y, k, n, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace

extern "C" size_t kk_native_q4_payload_bytes(int k, int n) {
    const size_t rows = (static_cast<size_t>(n) + 31) & ~static_cast<size_t>(31);
    return (rows * k / 2 + 255) & ~static_cast<size_t>(255);
}

extern "C" int kk_native_q4_gemv(const void *weights, const void *x, int x_f16, float *y, int k, int n, int batch,
                                 hipStream_t stream) {
    if (!weights || !x || !y || k <= 0 || k % 32 != 0 || k > 16384 || n <= 0 || batch <= 0)
        return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(weights) & 255) != 0) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(x) & (x_f16 ? 1 : 3)) != 0 || (reinterpret_cast<uintptr_t>(y) & 3) != 0)
        return hipErrorInvalidValue;
    const uint8_t *w = static_cast<const uint8_t *>(weights);
    const uint16_t *scales = reinterpret_cast<const uint16_t *>(w + kk_native_q4_payload_bytes(k, n));
    const int blocks = k >> 5;
    // columns per launch: LDS within the limit and activation passes within the register budget
    auto fits = [&](int cols) {
        return lds_bytes(blocks, cols) <= kNqLdsLimit && passes_for(blocks, cols) <= kNqMaxPasses;
    };
    if (!fits(1)) return hipErrorInvalidValue;
    int fit = 1;
    while (fit < kNqMaxColumns && fits(fit + 1)) ++fit;
    const size_t x_bytes = x_f16 ? 2 : 4;
    for (int c0 = 0; c0 < batch; c0 += fit) {
        const int cols = std::min(fit, batch - c0);
        const int passes = passes_for(blocks, cols);
        const void *xc = static_cast<const uint8_t *>(x) + static_cast<size_t>(c0) * k * x_bytes;
        float *yc = y + static_cast<size_t>(c0) * n;
        hipError_t status;
        switch (cols) {
        case 1: status = launch_passes<1>(passes, w, scales, xc, x_f16, yc, k, n, stream); break;
        case 2: status = launch_passes<2>(passes, w, scales, xc, x_f16, yc, k, n, stream); break;
        case 3: status = launch_passes<3>(passes, w, scales, xc, x_f16, yc, k, n, stream); break;
        default: status = launch_passes<4>(passes, w, scales, xc, x_f16, yc, k, n, stream); break;
        }
        if (status != hipSuccess) return status;
    }
    return hipSuccess;
}
