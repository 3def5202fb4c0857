// Small-batch (1..8) Q4_0 GEMV for K = 4096 on gfx950 fp16 MFMA: the weight
// rows streamed in whole 16-byte pieces, staged per wave in LDS, and one
// v_mfma_f32_16x16x32_f16 per Q4_0 block for 16 rows and all batch columns.
//
// Y[b, r] = sum_k X[b, k] * W[r, k]  (reference kernels/kunlun-matvec.xpu:24-79,
// which re-reads W once per batch column). HBM-bound by design, VALU-bound in
// practice (per block and 16 rows: one nibble dword decoded per lane, four
// scale FMAs per lane).
//
// Work split. A workgroup of 8 waves owns T tiles of 32 rows (T = tiles / CUs
// rounded up, at most 4); wave c takes K chunk c (values 512c .. 512c + 511,
// Q4_0 blocks 16c .. 16c + 15, 288 bytes) of every tile row. A tile's 32 x 288
// bytes are 576 16-byte pieces, 9 loads of one piece per lane (piece i of the
// chunk row is lane-contiguous), through a buffer resource per tile whose
// extent ends at the last row, so rows past n read as zero. One tile is in
// flight per wave (a 9-entry register ring refilled piece by piece). Each
// arrived piece goes into the wave's own LDS area (row stride 296 bytes: 16
// rows x 2 lane groups reading one dword each fall on 32 distinct banks); no
// workgroup barrier until the final sum of the 8 waves' partial sums, which
// are added in wave order.
//
// Operands. For block j of the chunk, lane (n, g) of the B operand holds the
// 8 values of nibble dword g of row n's block (kk::q4_dword_halves order:
// values 4g + (0, 2, 1, 3) from the low nibbles, 16 + 4g + (0, 2, 1, 3) from
// the high nibbles), exact fp16 q - 8. Row r of the A operand is batch column r
// (r < 8) as fp16 hi part, row r + 8 its lo part, of x * 2^s, in the same value
// order; 2^s per column and chunk brings the chunk's max |x| below 2^14, and
// |x 2^s - hi - lo| <= 2^-22 |x 2^s| + 2^-25. The products are exact in F32;
// D[r][n] of the block is scaled by the block's F16 scale d (v_fma_mix) into a
// per-row accumulator, and the hi and lo rows are added and multiplied by
// 2^-s at the end. A column whose chunk holds an Inf or NaN gets 2^-s = NaN:
// that batch column becomes NaN in every output row (the batch-1 GEMV's rule).
//
// Activations. Each wave reads its chunk of X lane-contiguously (lane l:
// column l / 8, values 4 (l % 8) .. + 3 of each 32), moves quad g (hi lanes)
// or quad 4 + g (lo lanes) of column r % 8 to lane (r, g) with ds_bpermute,
// and converts it to hi and lo; a lane keeps the parts of its own row and
// takes the other half of its 8 values from lane r ^ 8 by DPP (bank-masked
// moves: banks 0-1 are the hi rows, banks 2-3 the lo rows).
#include "device_common.h"
#include "launch.h"
#include "lds_opt_in.h"

#include <algorithm>

namespace {

using kk::half8;
using kk::kWave;

typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kK = 4096;                      // the one K this kernel takes
constexpr int kWaves = 8;                     // one K chunk of 512 values each
constexpr int kRowBytes = kK / 32 * 18;       // 2304
constexpr int kChunkBytes = 16 * 18;          // 288
constexpr int kTileRows = 32;
constexpr int kPiecesPerLane = kTileRows * kChunkBytes / 16 / kWave;   // 9
constexpr int kStageStride = 296;
constexpr int kStageBytes = kTileRows * kStageStride;
constexpr int kMaxTiles = 4;
constexpr int kLdsBytes = kWaves * kStageBytes + kMaxTiles * 2 * kWaves * 32 * 16;
static_assert(kTileRows * kChunkBytes == kPiecesPerLane * kWave * 16, "whole pieces per tile");

constexpr int kXor8 = 0x128;                  // DPP row_ror:8: lane r ^ 8 within 16

__device__ __forceinline__ uint32_t bit_insert(uint32_t mask, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(a), "v"(b));   // (a & mask) | (b & ~mask)
    return r;
}

template <int BANKS>
__device__ __forceinline__ uint32_t from_partner(uint32_t old, uint32_t src) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(src), kXor8, 0xf, BANKS, false));
}

// w2 (gate/up pair, else null): tile i holds rows 16i .. 16i + 15 of w (the
// gate matrix) as its rows 0..15 and the same rows of w2 (the up matrix) as
// rows 16..31, and y = SiLU(gate) * up ([batch][n], kk::swiglu_value).
template <bool PAIR>
__global__ __launch_bounds__(kWave * kWaves) void q4_stream_gemv(const uint8_t *__restrict__ w,
                                                               const uint8_t *__restrict__ w2,
                                                               const float *__restrict__ x, float *__restrict__ y,
                                                               int n, int batch, int tiles_per_group) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int tile_out = PAIR ? kTileRows / 2 : kTileRows;       // output rows per tile
    const int tiles = (n + tile_out - 1) / tile_out;
    const int tile0 = blockIdx.x * tiles_per_group;
    const int c = wid;                                            // this wave's K chunk
    uint8_t *stage = lds + wid * kStageBytes;
    float4v *partial = reinterpret_cast<float4v *>(lds + kWaves * kStageBytes);   // [T][2][waves][32]

    // 1. X, lane-contiguous: lane l holds values 512c + 32j + 4(l % 8) .. + 3 of column l / 8
    float xv[16][4];
    {
        const float *xl = x + static_cast<size_t>(min(lane >> 3, batch - 1)) * kK + c * 512 + 4 * (lane & 7);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float4 a = *reinterpret_cast<const float4 *>(xl + 32 * j);
            xv[j][0] = a.x; xv[j][1] = a.y; xv[j][2] = a.z; xv[j][3] = a.w;
        }
    }
    // 2. the first two tiles' pieces (issued after X: the memory counter is in order)
    __builtin_amdgcn_sched_barrier(0);
    const size_t total = static_cast<size_t>(n) * kRowBytes;
    // rows [row0, row0 + rows) of `base`, the ones past n reading as zero
    auto rows_buffer = [&](const uint8_t *base, size_t row0, size_t rows) {
        const size_t off = min(row0 * kRowBytes, total);
        const uint32_t extent = static_cast<uint32_t>(min(min(total - off, rows * kRowBytes), static_cast<size_t>(0xfffffff0u)));
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base + off), 0, extent, 0x00020000);
    };
    uint32_t goff[kPiecesPerLane], loff[kPiecesPerLane];   // piece offsets in the tile and in the stage
#pragma unroll
    for (int i = 0; i < kPiecesPerLane; ++i) {
        const int idx = i * kWave + lane, row = idx / 18, piece = idx - row * 18;
        goff[i] = static_cast<uint32_t>(row * kRowBytes + c * kChunkBytes + piece * 16);
        loff[i] = static_cast<uint32_t>(row * kStageStride + piece * 16);
    }
    auto load_at = [&](__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(off), 0, 2));
    };
    // pair tiles: pieces 0..255 are gate rows 0..13, 288..575 up rows 16..31;
    // load 4 (pieces 256..319) spans both: each half's lanes read the other
    // matrix's buffer out of bounds (zero); the up half goes to a slot of its
    // own and the two are or-ed when the piece is staged, not at the load
    // (which would wait for it there)
    constexpr uint32_t kOutOfBounds = 0x7ffffff0u;
    constexpr uint32_t kUpHalf = (kTileRows / 2) * kRowBytes;
    constexpr int kSplit = kTileRows / 2 * 18 / kWave;             // the load spanning both halves
    u32x4 ring[kPiecesPerLane], ring_up{0u, 0u, 0u, 0u};
    auto load = [&](int t, int i) {
        if (!PAIR) {
            ring[i] = load_at(rows_buffer(w, static_cast<size_t>(tile0 + t) * kTileRows, kTileRows), goff[i]);
            return;
        }
        const size_t row0 = static_cast<size_t>(tile0 + t) * (kTileRows / 2);
        if (i < kSplit) {
            ring[i] = load_at(rows_buffer(w, row0, kTileRows / 2), goff[i]);
        } else if (i > kSplit) {
            ring[i] = load_at(rows_buffer(w2, row0, kTileRows / 2), goff[i] - kUpHalf);
        } else {
            const bool up = i * kWave + lane >= kTileRows / 2 * 18;
            ring[i] = load_at(rows_buffer(w, row0, kTileRows / 2), up ? kOutOfBounds : goff[i]);
            ring_up = load_at(rows_buffer(w2, row0, kTileRows / 2), up ? goff[i] - kUpHalf : kOutOfBounds);
        }
    };
#pragma unroll
    for (int i = 0; i < kPiecesPerLane; ++i) load(0, i);
    __builtin_amdgcn_sched_barrier(0);

    // 3. X into the A layout: lane (r, g) takes quad g (r < 8) or 4 + g (r >= 8) of column r % 8
    {
        const int src = ((r16 & 7) * 8 + g + 4 * (r16 >> 3)) * 4;
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t)
                xv[j][t] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(xv[j][t])));
    }
    // the column's max |x| and non-finite values, from integer maxima of the
    // raw bits: positive values order as int32, negative ones as uint32
    int pos_max = 0;
    uint32_t any_max = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            pos_max = max(pos_max, __float_as_int(xv[j][t]));
            any_max = max(any_max, static_cast<uint32_t>(__float_as_int(xv[j][t])));
        }
    uint32_t mag = max(static_cast<uint32_t>(pos_max), any_max >= 0x80000000u ? any_max & 0x7fffffffu : 0u);
    mag = max(mag, from_partner<0xf>(0, mag));
    mag = max(mag, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mag), 16, kWave)));
    mag = max(mag, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mag), 32, kWave)));
    const bool bad = mag >= 0x7f800000u;                                   // Inf or NaN in the column's chunk
    const int e = max(min(__builtin_amdgcn_frexp_expf(__uint_as_float(mag)), 128), -110);   // max < 2^e
    const float scale = bad ? 0.0f : ldexpf(1.0f, 14 - e);
    const float inv_self = bad ? __builtin_nanf("") : ldexpf(1.0f, e - 14);
    float inv[4];   // 2^-s of columns 4 (g % 2) + r, held by lanes 4 (g % 2) + r
#pragma unroll
    for (int r = 0; r < 4; ++r)
        inv[r] = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * (g & 1) + r) * 4, __float_as_int(inv_self)));
    // hi and lo parts of the lane's own 4 values as dwords (values 0, 2 | 1, 3);
    // hi rows keep their hi parts and take the partner's (values 16..), lo rows
    // keep their lo parts and take the partner's (values 0..)
    u32x2 a_first[16], a_last[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float v0 = xv[j][0] * scale, v1 = xv[j][1] * scale, v2 = xv[j][2] * scale, v3 = xv[j][3] * scale;
        half2v h02, h13, l02, l13;
        h02[0] = static_cast<_Float16>(v0); h02[1] = static_cast<_Float16>(v2);
        h13[0] = static_cast<_Float16>(v1); h13[1] = static_cast<_Float16>(v3);
        l02[0] = static_cast<_Float16>(v0 - static_cast<float>(h02[0]));
        l02[1] = static_cast<_Float16>(v2 - static_cast<float>(h02[1]));
        l13[0] = static_cast<_Float16>(v1 - static_cast<float>(h13[0]));
        l13[1] = static_cast<_Float16>(v3 - static_cast<float>(h13[1]));
        const uint32_t hi0 = __builtin_bit_cast(uint32_t, h02), hi1 = __builtin_bit_cast(uint32_t, h13);
        const uint32_t lo0 = __builtin_bit_cast(uint32_t, l02), lo1 = __builtin_bit_cast(uint32_t, l13);
        a_first[j] = u32x2{from_partner<0xc>(hi0, lo0), from_partner<0xc>(hi1, lo1)};
        a_last[j] = u32x2{from_partner<0x3>(lo0, hi0), from_partner<0x3>(lo1, hi1)};
    }
    auto a_frag = [&](int j) {
        return __builtin_bit_cast(half8, u32x4{a_first[j][0], a_first[j][1], a_last[j][0], a_last[j][1]});
    };

    // 4. per 16-row group: one MFMA per block, then the block scales
    // (0x6400 | q) is 1024 + q: minus 1032 gives q - 8; a high nibble left in
    // place, (0x6400 | 16 q) = 1024 + 16 q, times 1/16 minus 72 gives q - 8
    // (both exact in fp16, one shift per dword)
    uint32_t low_mask = 0x000f000fu, high_mask = 0x00f000f0u, magic = 0x64006400u;
    asm volatile("" : "+v"(low_mask), "+v"(high_mask), "+v"(magic));   // held in VGPRs for v_bfi
    auto decode = [&](uint32_t qs) {
        const half2v off = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
        const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
        const half2v off16 = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
        const uint32_t s8 = qs >> 8;
        const half2v a = __builtin_bit_cast(half2v, bit_insert(low_mask, qs, magic)) + off;
        const half2v b = __builtin_bit_cast(half2v, bit_insert(low_mask, s8, magic)) + off;
        const half2v cc =
            __builtin_elementwise_fma(__builtin_bit_cast(half2v, bit_insert(high_mask, qs, magic)), sixteenth, off16);
        const half2v d =
            __builtin_elementwise_fma(__builtin_bit_cast(half2v, bit_insert(high_mask, s8, magic)), sixteenth, off16);
        return __builtin_bit_cast(half8, u32x4{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                               __builtin_bit_cast(uint32_t, cc), __builtin_bit_cast(uint32_t, d)});
    };
    auto group_compute = [&](int t, int rg) {
        // block pair p of row n: dwords 9p .. 9p + 8 (scale 0, nibbles, scale 1, nibbles)
        const uint32_t *row = reinterpret_cast<const uint32_t *>(stage + (rg * 16 + r16) * kStageStride);
        float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int p0 = 0; p0 < 8; p0 += 4) {
            float4v dq[8];
            uint32_t scales[4];
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
                const uint32_t *pd = row + 9 * (p0 + pp);
                scales[pp] = (pd[0] & 0xffffu) | (pd[4] & 0xffff0000u);
                const half8 b0 = decode(kk::align_bytes(pd[g + 1], pd[g], 2));
                const half8 b1 = decode(pd[5 + g]);
                const float4v z = {0.0f, 0.0f, 0.0f, 0.0f};
                dq[2 * pp] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_frag(2 * (p0 + pp)), b0, z, 0, 0, 0);
                dq[2 * pp + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_frag(2 * (p0 + pp) + 1), b1, z, 0, 0, 0);
            }
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
                const float d0 = kk::half_bits_to_float(scales[pp] & 0xffffu);
                const float d1 = kk::half_bits_to_float(scales[pp] >> 16);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc[r] = fmaf(dq[2 * pp][r], d0, acc[r]);
                    acc[r] = fmaf(dq[2 * pp + 1][r], d1, acc[r]);
                }
            }
        }
        // lane (n, g < 2): hi rows 4g .. 4g + 3 (columns), lane + 32 their lo rows
        float4v out;
#pragma unroll
        for (int r = 0; r < 4; ++r) out[r] = (acc[r] + __shfl_xor(acc[r], 32, kWave)) * inv[r];
        if (lane < 32) partial[((t * 2 + rg) * kWaves + wid) * 32 + lane] = out;
    };
    auto stage_piece = [&](int i, const u32x4 &v) {
        *reinterpret_cast<u32x2 *>(stage + loff[i]) = u32x2{v[0], v[1]};       // 8-byte aligned rows
        *reinterpret_cast<u32x2 *>(stage + loff[i] + 8) = u32x2{v[2], v[3]};
    };
    // rows 0..15 of a tile are pieces 0..287: staged with piece set 4. One
    // tile is in flight per wave: each piece's slot is refilled with the next
    // tile's piece as soon as it is staged (K4096 x N14336 batch 8: 13.9 us
    // against 14.8 us with two tiles in flight)
    for (int tt = 0; tt < tiles_per_group; ++tt) {
#pragma unroll
        for (int i = 0; i < kPiecesPerLane; ++i) {
            stage_piece(i, PAIR && i == kSplit ? ring[i] | ring_up : ring[i]);
            if (tt + 1 < tiles_per_group) load(tt + 1, i);
            if (i == 4) group_compute(tt, 0);
        }
        group_compute(tt, 1);
    }
    __syncthreads();
    // 5. column m, tile row 16 rg + nn: lane (nn, m / 4) element m % 4 of every
    //    wave, added in wave order (pair tiles: rg 0 the gate row, rg 1 the up row)
    auto row_sum = [&](int t, int rg, int m, int nn) {
        const int src = (m >> 2) * 16 + nn;
        float sum = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) sum += partial[((t * 2 + rg) * kWaves + ww) * 32 + src][m & 3];
        return sum;
    };
    const int per_tile = PAIR ? 128 : 256;
    for (int idx = threadIdx.x; idx < tiles_per_group * per_tile; idx += kWave * kWaves) {
        const int t = idx / per_tile, rg = PAIR ? 0 : (idx >> 7) & 1, m = (idx >> 4) & 7, nn = idx & 15;
        const int gt = tile0 + t;
        const int out_row = gt * tile_out + rg * 16 + nn;
        if (m >= batch || gt >= tiles || out_row >= n) continue;
        const float v = PAIR ? kk::swiglu_value(row_sum(t, 0, m, nn), row_sum(t, 1, m, nn)) : row_sum(t, rg, m, nn);
        y[static_cast<size_t>(m) * n + out_row] = v;
    }
}

} // namespace

extern "C" int kk_q4_stream_gemv_supported(const void *w, const float *x, int k, int n, int batch) {
    return w && x && k == kK && n >= 1 && batch >= 1 && batch <= 8 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

// Tiles per workgroup: ceil(tiles / CUs), at most 4 (then more workgroups than CUs).
namespace {
hipError_t launch_stream(const void *w, const void *w2, const float *x, float *y, int n, int batch, int cus,
                         hipStream_t stream) {
    const hipError_t rc = w2 ? kk::opt_in_lds(reinterpret_cast<const void *>(&q4_stream_gemv<true>), kLdsBytes)
                             : kk::opt_in_lds(reinterpret_cast<const void *>(&q4_stream_gemv<false>), kLdsBytes);
    if (rc != hipSuccess) return rc;
    const int tile_out = w2 ? kTileRows / 2 : kTileRows;     // a pair tile: 16 gate and 16 up rows
    const int tiles = (n + tile_out - 1) / tile_out;
    const int t = std::max(1, std::min(kMaxTiles, (tiles + cus - 1) / cus));
    if (w2)
        hipLaunchKernelGGL(q4_stream_gemv<true>, dim3((tiles + t - 1) / t), dim3(kWave * kWaves), kLdsBytes, stream,
                           static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(w2), x, y, n, batch, t);
    else
        hipLaunchKernelGGL(q4_stream_gemv<false>, dim3((tiles + t - 1) / t), dim3(kWave * kWaves), kLdsBytes, stream,
                           static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(w2), x, y, n, batch, t);
    return hipGetLastError();
}
} // namespace

extern "C" int kk_q4_stream_gemv(const void *w, const float *x, float *y, int k, int n, int batch, int cus,
                                 hipStream_t stream) {
    if (!kk_q4_stream_gemv_supported(w, x, k, n, batch) || !y || cus <= 0) return hipErrorInvalidValue;
    return launch_stream(w, nullptr, x, y, n, batch, cus, stream);
}

// Gate/up pair: both matrices in one launch (X read once per workgroup),
// y = [batch][n] = SiLU(X w_gate^T) * (X w_up^T).
extern "C" int kk_q4_stream_gemv_pair_swiglu(const void *w_gate, const void *w_up, const float *x, float *y, int k,
                                             int n, int batch, int cus, hipStream_t stream) {
    if (!kk_q4_stream_gemv_supported(w_gate, x, k, n, batch) || !kk_q4_stream_gemv_supported(w_up, x, k, n, batch) ||
        !y || cus <= 0)
        return hipErrorInvalidValue;
    return launch_stream(w_gate, w_up, x, y, n, batch, cus, stream);
}
