// Prefill GEMM for Q4_0 and F16 weights on gfx950 fp16 MFMA (f32 accumulate).
//
// Y[m, n] = sum_k X[m, k] * W[n, k] for batch (M) in the hundreds, where the
// GEMV kernels would re-read every weight byte per pair of batch rows.
//
// 1. x_to_f16 (prepass): X f32 [M, K] -> X16 fp16 [M_pad, K_pad], each row
//    scaled by a power of two s_m so that max|x_m * s_m| < 2^14 (exact; no
//    fp16 overflow), zero padded, and with the values of each 32-block stored
//    in the order a Q4_0 nibble dword decodes to (block order below, Q4_0 only);
//    row_inv[m] = 1 / s_m.
// 2. mfma_gemm: tiles of 128 (M) x 64 (N) x 128 (K). Each step, the
//    workgroup loads the X16 tile and the raw Q4_0 (or F16) weight tile,
//    dequantizes Q4_0 to fp16 (q - 8) * d / 8 in registers (the 1/8 keeps
//    |value| <= 65504 for any F16 scale; undone in the epilogue) and writes
//    both to double-buffered LDS; eight waves run v_mfma_f32_32x32x16_f16
//    tiles, two k-groups of four. Epilogue: y = acc * row_inv[m] * 8.
// Precision: fp16 inputs, f32 accumulation: relative error ~2^-11 per
// product (the fp16-MFMA tolerance of the path is 2e-3 relative).
#include "device_common.h"
#include "launch.h"
#include "lds_opt_in.h"
#include "tuning.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>

namespace {

using kk::kWave;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBK = 128;            // tile N (64 or 128) is a template parameter
constexpr int kGemmThreads = 512;              // 8 waves: 2 k-groups x (2 x 2) wave tiles of 64 x BN/2
constexpr int kLdsStride = kBK + 8;            // halves per LDS row: 272 B rows read conflict-free
constexpr int kPrepassThreads = 256;
constexpr int kXcds = 8;                       // MI355X: workgroups go round-robin to 8 XCDs

// Block order (Q4_0 only): position 8i + t of a 32-value block holds value
// (4i, 4i+2, 4i+1, 4i+3, 16+4i, 16+4i+2, 16+4i+1, 16+4i+3)[t], the order in
// which nibble dword i of a Q4_0 block decodes to packed fp16 pairs.
size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

// ---------------------------------------------------------------------------
// Prepass: one workgroup per padded row; PER groups of 8 values per thread
// (PER * 8 * kPrepassThreads >= k_pad). Every load is issued before the
// first wait: the row and group indices are clamped into X and the slots
// past the row (or of a padding row) are zeroed afterwards.
template <bool PERMUTE, int PER>
__global__ __launch_bounds__(kPrepassThreads) void x_to_f16(const float *__restrict__ x, int m_rows, int k,
                                                           int k_pad, _Float16 *__restrict__ x16,
                                                           float *__restrict__ row_inv) {
    __shared__ float scratch[kPrepassThreads / kWave];
    const int row = blockIdx.x;
    const int groups = k >> 3;                       // 8 values per group
    float v[PER][8];
    float m = 0.0f;
    const bool real = row < m_rows;
    const float *src_row = x + static_cast<size_t>(min(row, m_rows - 1)) * k;
#pragma unroll
    for (int g = 0; g < PER; ++g) {
        const int grp = min(g * kPrepassThreads + static_cast<int>(threadIdx.x), groups - 1);
        const int blk = grp >> 2, i = grp & 3;
        const float *src = src_row + blk * 32;
        if (PERMUTE) {   // positions 8i..8i+7 <- values 4i, 4i+2, 4i+1, 4i+3, 16+4i, ...
            const float4 lo = *reinterpret_cast<const float4 *>(src + 4 * i);
            const float4 hi = *reinterpret_cast<const float4 *>(src + 16 + 4 * i);
            v[g][0] = lo.x; v[g][1] = lo.z; v[g][2] = lo.y; v[g][3] = lo.w;
            v[g][4] = hi.x; v[g][5] = hi.z; v[g][6] = hi.y; v[g][7] = hi.w;
        } else {
            const float4 a = *reinterpret_cast<const float4 *>(src + 8 * i);
            const float4 b = *reinterpret_cast<const float4 *>(src + 8 * i + 4);
            v[g][0] = a.x; v[g][1] = a.y; v[g][2] = a.z; v[g][3] = a.w;
            v[g][4] = b.x; v[g][5] = b.y; v[g][6] = b.z; v[g][7] = b.w;
        }
    }
#pragma unroll
    for (int g = 0; g < PER; ++g) {
        if (!real || g * kPrepassThreads + static_cast<int>(threadIdx.x) >= groups) {
#pragma unroll
            for (int t = 0; t < 8; ++t) v[g][t] = 0.0f;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) m = fmaxf(m, fabsf(v[g][t]));
    }
    m = kk::wave_max(m);
    if ((threadIdx.x & (kWave - 1)) == 0) scratch[threadIdx.x / kWave] = m;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPrepassThreads / kWave; ++i) m = fmaxf(m, scratch[i]);
    // s = 2^(14 - e) with 2^(e-1) <= m < 2^e; non-finite or zero rows keep s = 1
    int e = __builtin_amdgcn_frexp_expf(m);
    const bool finite = m <= 3.402823466e38f && m > 0.0f;
    e = finite ? max(min(e, 126), -100) : 14;
    const float s = ldexpf(1.0f, 14 - e);
    if (threadIdx.x == 0) row_inv[row] = ldexpf(1.0f, e - 14);
    _Float16 *dst = x16 + static_cast<size_t>(row) * k_pad;
#pragma unroll
    for (int g = 0; g < PER; ++g) {
        const int grp = g * kPrepassThreads + threadIdx.x;
        if (grp < (k_pad >> 3)) {
            half8 h;
#pragma unroll
            for (int t = 0; t < 8; ++t) h[t] = static_cast<_Float16>(v[g][t] * s);
            *reinterpret_cast<half8 *>(dst + grp * 8) = h;
        }
    }
}

// x_to_f16 with the fewest groups per thread that cover k_pad (k_pad <= 16384
// + alignment: at most 8 x 8 x 256 = 16384 values, checked by the callers'
// k <= 16384 and kKAlign | 16384).
void launch_x_to_f16(bool permute, const float *x, int batch, int k, int m_pad, int k_pad, _Float16 *x16,
                     float *row_inv, hipStream_t stream) {
    const int per_needed = (k_pad / 8 + kPrepassThreads - 1) / kPrepassThreads;
    const dim3 grid(m_pad), block(kPrepassThreads);
#define KK_X16(P, PER) hipLaunchKernelGGL((x_to_f16<P, PER>), grid, block, 0, stream, x, batch, k, k_pad, x16, row_inv)
    if (permute) {
        if (per_needed <= 1) KK_X16(true, 1);
        else if (per_needed <= 2) KK_X16(true, 2);
        else if (per_needed <= 4) KK_X16(true, 4);
        else KK_X16(true, 8);
    } else {
        if (per_needed <= 1) KK_X16(false, 1);
        else if (per_needed <= 2) KK_X16(false, 2);
        else if (per_needed <= 4) KK_X16(false, 4);
        else KK_X16(false, 8);
    }
#undef KK_X16
}

// ---------------------------------------------------------------------------
// Subnormal block scales. For an F16 scale d below 2^-14 (exponent field 0)
// the fp16 product (q - 8) / 8 * d lies on the 2^-24 grid of F16 subnormals
// and keeps only a few bits. The decode goes on as for any block and only
// sets `tiny` (one class test; the flag is a lane mask in SGPRs); a workgroup
// that met such a block adds the difference between its exact F32 values and
// what the decode made of them in its epilogue (tiny_scale_dots).
__device__ __forceinline__ void note_tiny_scale(uint32_t bits, bool &tiny) {
    union { uint16_t u; _Float16 h; } du;
    du.u = static_cast<uint16_t>(bits);
    tiny = tiny || __builtin_amdgcn_classh(du.h, 0x090);   // -subnormal | +subnormal
}

// Q4_0 decode to fp16 (q - 8) * d / 8 (the 1/8 keeps |value| <= 65504 for
// any F16 scale). dd = d / 8 in both halves (zero for a dead block); a live
// block's subnormal scale sets `tiny`.
__device__ __forceinline__ half2v q4_scale8(uint32_t bits, bool live, bool &tiny) {
    union { uint16_t u; _Float16 h; } du;
    du.u = static_cast<uint16_t>(bits & 0xffffu);
    if (live) note_tiny_scale(bits, tiny);
    const _Float16 d8 = live ? static_cast<_Float16>(du.h * static_cast<_Float16>(0.125f)) : static_cast<_Float16>(0.0f);
    return half2v{d8, d8};
}

// Nibble dword i of a block (bytes 4i .. 4i+3) -> the 8 values at block
// positions 8i .. 8i+7 in block order.
__device__ __forceinline__ half8 decode_q4_dword(uint32_t n, half2v dd) {
    const half2v off_lo = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    const half2v off_hi = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    const uint32_t t = n >> 8;
    union { uint32_t u; half2v h; } p0, p1, p2, p3;
    p0.u = (n & 0x000f000fu) | 0x64006400u;   // 1024 + q(4i),    1024 + q(4i+2)
    p1.u = (t & 0x000f000fu) | 0x64006400u;   // 1024 + q(4i+1),  1024 + q(4i+3)
    p2.u = (n & 0x00f000f0u) | 0x64006400u;   // 1024 + 16 q(16+4i), ...
    p3.u = (t & 0x00f000f0u) | 0x64006400u;
    const half2v h0 = (p0.h + off_lo) * dd;   // (q - 8) exact, then one rounding
    const half2v h1 = (p1.h + off_lo) * dd;
    const half2v h2 = (p2.h * sixteenth + off_hi) * dd;
    const half2v h3 = (p3.h * sixteenth + off_hi) * dd;
    half8 o;
    o[0] = h0[0]; o[1] = h0[1]; o[2] = h1[0]; o[3] = h1[1];
    o[4] = h2[0]; o[5] = h2[1]; o[6] = h3[0]; o[7] = h3[1];
    return o;
}

// Half a block (nibble dwords 2*half, 2*half+1 -> 16 values); e = the 18
// block bytes as 5 dwords.
__device__ __forceinline__ void decode_q4_half(const uint32_t (&e)[5], int half, bool live, half8 (&out)[2],
                                               bool &tiny) {
    const half2v dd = q4_scale8(e[0], live, tiny);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t lo = half ? e[2 + j] : e[j], hi = half ? e[3 + j] : e[1 + j];
        out[j] = decode_q4_dword(kk::align_bytes(hi, lo, 2), dd);   // nibble bytes 4i .. 4i+3, i = 2*half + j
    }
}

// (a & mask) | bits in one VALU op (the compiler splits it in two when the
// mask is a literal: gfx9 VOP3 takes none).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(mask), "v"(bits));
    return r;
}

// Nibble dword i of a block -> (q - 8) / 8 * d for block positions 8i .. 8i+7
// in block order, d = the block's F16 scale bits. (q - 8) / 8 is exact:
// p = 1024 + q gives p / 8 - 129, p = 1024 + 16 q gives p / 128 - 9; one
// rounding in the product, |value| <= |d|.
__device__ __forceinline__ half8 decode_q4_scaled(uint32_t n, uint32_t dbits) {
    const uint32_t magic = 0x64006400u, mask_lo = 0x000f000fu, mask_hi = 0x00f000f0u;
    const half2v lo_mul = {static_cast<_Float16>(0.125f), static_cast<_Float16>(0.125f)};
    const half2v lo_add = {static_cast<_Float16>(-129.0f), static_cast<_Float16>(-129.0f)};
    const half2v hi_mul = {static_cast<_Float16>(0.0078125f), static_cast<_Float16>(0.0078125f)};
    const half2v hi_add = {static_cast<_Float16>(-9.0f), static_cast<_Float16>(-9.0f)};
    union { uint16_t u; _Float16 h; } du;
    du.u = static_cast<uint16_t>(dbits);
    const half2v dd = {du.h, du.h};
    const uint32_t t = n >> 8;
    union { uint32_t u; half2v h; } p0, p1, p2, p3;
    p0.u = and_or(n, mask_lo, magic);   // 1024 + q(4i),    1024 + q(4i+2)
    p1.u = and_or(t, mask_lo, magic);   // 1024 + q(4i+1),  1024 + q(4i+3)
    p2.u = and_or(n, mask_hi, magic);   // 1024 + 16 q(16+4i), ...
    p3.u = and_or(t, mask_hi, magic);
    const half2v h0 = (p0.h * lo_mul + lo_add) * dd;
    const half2v h1 = (p1.h * lo_mul + lo_add) * dd;
    const half2v h2 = (p2.h * hi_mul + hi_add) * dd;
    const half2v h3 = (p3.h * hi_mul + hi_add) * dd;
    half8 o;
    o[0] = h0[0]; o[1] = h0[1]; o[2] = h1[0]; o[3] = h1[1];
    o[4] = h2[0]; o[5] = h2[1]; o[6] = h3[0]; o[7] = h3[1];
    return o;
}

// Blocks with subnormal scales (note_tiny_scale), found and corrected only
// in a workgroup that met one. kTinyMaskWords words per B-tile row mark its
// blocks with a subnormal scale (K <= 16384: at most 512 blocks).
constexpr int kTinyMaskWords = 16;

// All `threads` threads of the workgroup: masks[j * kTinyMaskWords + b / 32]
// bit b % 32 is set when block b of tile row j (row_ptr(j); nullptr past the
// matrix) has a subnormal scale. Two workgroup barriers.
template <typename RowPtr>
__device__ void build_tiny_masks(int rows, int blocks, RowPtr row_ptr, uint32_t *masks, int threads) {
    for (int i = threadIdx.x; i < rows * kTinyMaskWords; i += threads) masks[i] = 0u;
    __syncthreads();
    // kU scales per thread and round: their loads go out together, then the marks
    constexpr int kU = 8;
    for (int base = threadIdx.x; base < rows * blocks; base += kU * threads) {
        uint32_t bits[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int i = base + u * threads;
            const int j = i / blocks, b = i - j * blocks;
            const uint8_t *wrow = i < rows * blocks ? row_ptr(j) : nullptr;
            bits[u] = wrow ? wrow[18 * b] | (static_cast<uint32_t>(wrow[18 * b + 1]) << 8) : 0u;
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int i = base + u * threads;
            const int j = i / blocks, b = i - j * blocks;
            if ((bits[u] & 0x7c00u) == 0 && (bits[u] & 0x3ffu) != 0)
                atomicOr(&masks[j * kTinyMaskWords + (b >> 5)], 1u << (b & 31));
        }
    }
    __syncthreads();
}

// The correction for the marked blocks of one weight row `wrow` (mask: its
// kTinyMaskWords words) and the R activation rows row_of(0 .. R-1) of x16
// (block order, row stride k_pad): adds to out[r], block by block in
// increasing order, x16 . (v - decode(v)) with v = (q - 8) / 8 * d in F32,
// d = +-m * 2^-24 the block's subnormal scale, and decode(nibble dword, scale
// bits) the fp16 values the kernel's decode gave the block (each one rounding
// of the exact (q - 8) / 8 * d, so the same in any context). v, decode(v)
// (both on the 2^-27 grid, below 2^-13) and their difference are exact in
// F32; the products and sums round.
template <int R, typename RowOf, typename Decode>
__device__ void tiny_scale_dots(const uint8_t *wrow, const uint32_t *mask, int blocks, const _Float16 *x16, int k_pad,
                                RowOf row_of, Decode decode, float (&out)[R]) {
#pragma unroll 1
    for (int word = 0; word < (blocks + 31) / 32; ++word) {
        uint32_t bitsleft = mask[word];
#pragma unroll 1
        while (bitsleft) {
            const int b = 32 * word + __builtin_ctz(bitsleft);
            bitsleft &= bitsleft - 1u;
            // the block's 18 bytes, all loads issued before the first use
            const uint8_t *blk = wrow + 18 * b;
            uint32_t by[18];
#pragma unroll
            for (int t = 0; t < 18; ++t) by[t] = blk[t];
            const uint32_t bits = by[0] | (by[1] << 8);
            const float d = ldexpf(static_cast<float>(bits & 0x3ffu), -27) * ((bits & 0x8000u) ? -1.0f : 1.0f);   // d / 8
            float wv[4][8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {   // nibble dword i -> block-order positions 8i .. 8i+7
                const uint32_t *nb = by + 2 + 4 * i;
                const uint32_t nib = nb[0] | nb[1] << 8 | nb[2] << 16 | nb[3] << 24;
                const half8 dec = decode(nib, bits);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const uint32_t byte = nb[(t & 1) << 1 | (t & 2) >> 1];   // bytes 0, 2, 1, 3
                    const uint32_t q = t < 4 ? byte & 15u : byte >> 4;
                    wv[i][t] = (static_cast<float>(q) - 8.0f) * d - static_cast<float>(dec[t]);
                }
            }
            // per activation row: its four 8-value pieces loaded together, then
            // added piece by piece in block order
#pragma unroll 2
            for (int r = 0; r < R; ++r) {
                half8 xv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    xv[i] = *reinterpret_cast<const half8 *>(x16 + static_cast<size_t>(row_of(r)) * k_pad + 32 * b + 8 * i);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int t = 0; t < 8; ++t) out[r] += static_cast<float>(xv[i][t]) * wv[i][t];
            }
        }
    }
}

// Workgroup tile 128 (M) x BN (N) x 128 (K) per step, 8 waves: two
// k-groups (waves 0-3 take k sub-steps 0-3 of each step, waves 4-7 sub-steps
// 4-7), each a 2 x 2 arrangement of 64 x BN/2 wave tiles (2 x BN/64
// v_mfma_f32_32x32x16_f16 tiles). Two waves per SIMD let one wave's MFMAs
// overlap the other's LDS traffic, loads and Q4_0 decode. Global loads run
// kStages steps ahead into register sets (all loads branch-free, so the
// memory-counter waits stay exact); each step's tiles are written to one of
// two LDS buffers after the MFMAs of the step before. The k-groups' partial
// sums meet in LDS at the end, in a fixed order.
//
// Tiles are numbered m-major and dealt to the 8 XCDs in contiguous ranges,
// so the workgroups of one XCD share few activation row tiles in its L2.
constexpr int kLdsA = kBM * kLdsStride;
#ifndef KUNLUN_GEMM_STAGES
#define KUNLUN_GEMM_STAGES 2
#endif
constexpr int kStages = KUNLUN_GEMM_STAGES;    // register sets in flight (even)
constexpr int kKAlign = kStages * kBK;         // k_pad granularity: whole main-loop iterations
static_assert(16384 % kKAlign == 0, "k <= 16384 keeps k_pad <= 16384, within x_to_f16<., 8>");
static_assert(kStages % 2 == 0, "LDS buffer parity follows the register set index");

template <int BN>
constexpr size_t gemm_lds_bytes() {
    return 2 * static_cast<size_t>(kLdsA + BN * kLdsStride) * sizeof(_Float16);
}

// PAIR (gate/up): the B tile holds 64 rows of each of two weight matrices w
// and w2 (same shape); B row j is row (j >> 6) * 32 + (j & 31) of the output
// tile from matrix (j >> 5) & 1, so each wave's first 32-column MFMA tile is
// gate and its second is up for the same 32 output columns, and the epilogue
// writes y = SiLU(gate) * up.
template <bool F16W, int BN, bool PAIR>
__global__ __launch_bounds__(kGemmThreads) void mfma_gemm(const uint8_t *__restrict__ w,
                                                         const uint8_t *__restrict__ w2,
                                                         const _Float16 *__restrict__ x16,
                                                         const float *__restrict__ row_inv,
                                                         float *__restrict__ y, int m_rows, int n_rows,
                                                         int k, int k_pad, size_t w_bytes, int n_tiles,
                                                         int tiles, int tiles_per_xcd) {
    static_assert(BN == 64 || BN == 128, "tile N");
    static_assert(!PAIR || BN == 128, "a pair tile holds 64 rows of each matrix");
    constexpr int kLdsB = BN * kLdsStride;
    constexpr int kNT = BN / 64;                         // 32-column MFMA tiles per wave
    constexpr int kOutN = PAIR ? 64 : BN;                // output columns per tile
    extern __shared__ __align__(16) _Float16 lds[];      // 2 x (A tile + B tile)

    const int bid = blockIdx.x;
    const int tile = (bid % kXcds) * tiles_per_xcd + bid / kXcds;
    if (tile >= tiles) return;                           // whole workgroup, before any barrier
    const int mt = tile / n_tiles;
    const int nt = tile - mt * n_tiles;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = wid >> 2;                             // k-group
    const int wm = wid & 1, wn = (wid >> 1) & 1;         // wave tile rows 64*wm, columns wn*BN/2
    const int m0 = mt * kBM;
    const int n0 = nt * kOutN;
    const int blocks = k >> 5;
    const size_t row_bytes = F16W ? static_cast<size_t>(k) * 2 : static_cast<size_t>(blocks) * 18;
    const int steps = k_pad / kBK;                       // multiple of kStages

    // A: 16-byte chunks tid + 512 i of the 128 x 128 tile (16 chunks per row)
    const _Float16 *a_src[4];
    int a_dst[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + kGemmThreads * i;
        const int r = c >> 4, col = (c & 15) * 8;
        a_src[i] = x16 + static_cast<size_t>(m0 + r) * k_pad + col;
        a_dst[i] = r * kLdsStride + col;
    }
    // B, Q4_0, BN = 128: thread = block (tid & 3) of weight row tid >> 2;
    //          BN = 64: half (tid & 1) of block ((tid >> 1) & 3) of row tid >> 3.
    // B, F16: 16-byte chunks tid + 512 i of the BN x 128 fp16 tile.
    constexpr int kQShift = BN == 128 ? 2 : 3;
    // B tile row j -> weight matrix and output column of the tile
    auto b_matrix = [](int j) { return PAIR ? (j >> 5) & 1 : 0; };
    auto b_column = [](int j) { return PAIR ? ((j >> 6) << 5) | (j & 31) : j; };
    const int qb_row = tid >> kQShift;
    const int qb_blk = BN == 128 ? (tid & 3) : ((tid >> 1) & 3);
    const int qb_half = BN == 128 ? 0 : (tid & 1);
    const int q_wrow = min(n0 + b_column(qb_row), n_rows - 1);
    const bool q_live_row = n0 + b_column(qb_row) < n_rows;
    const uint8_t *q_w = b_matrix(qb_row) ? w2 : w;
    const size_t w_mis = reinterpret_cast<uintptr_t>(q_w) & 3;
    const size_t w_last_dword = (w_mis + w_bytes - 1) >> 2;
    const uint32_t *w_base32 = reinterpret_cast<const uint32_t *>(q_w - w_mis);

    // Register sets: 4 A chunks plus the B words (6 raw Q4_0 dwords with their
    // byte shift and liveness, or BN/32 fp16 chunks).
    constexpr int kF16Chunks = BN / 32;
    constexpr int kBWords = F16W ? 4 * kF16Chunks : 6;
    u32x4 a_reg[kStages][4];
    uint32_t b_reg[kStages][kBWords];
    uint32_t shift_reg[kStages];
    bool live_reg[kStages];
    bool tiny = false;   // Q4_0: set once this thread skipped a block with a subnormal scale

    auto load = [&](int step, int set) {
        const int ks = min(step, steps - 1);              // past the end: reload the last step
#pragma unroll
        for (int i = 0; i < 4; ++i)
            a_reg[set][i] = *reinterpret_cast<const u32x4 *>(a_src[i] + static_cast<size_t>(ks) * kBK);
        if constexpr (F16W) {
#pragma unroll
            for (int i = 0; i < kF16Chunks; ++i) {
                const int c = tid + kGemmThreads * i;
                const int r = min(n0 + b_column(c >> 4), n_rows - 1);
                const int kk0 = min(ks * kBK + (c & 15) * 8, k - 8);
                const uint8_t *src = b_matrix(c >> 4) ? w2 : w;
                const u32x4 v = *reinterpret_cast<const u32x4 *>(src + static_cast<size_t>(r) * row_bytes +
                                                                 static_cast<size_t>(kk0) * 2);
#pragma unroll
                for (int t = 0; t < 4; ++t) b_reg[set][4 * i + t] = v[t];
            }
        } else {
            const int blk = ks * (kBK / 32) + qb_blk;
            live_reg[set] = q_live_row && blk < blocks;
            const int bc = min(blk, blocks - 1);
            const size_t pos = w_mis + static_cast<size_t>(q_wrow) * row_bytes + static_cast<size_t>(bc) * 18;
            shift_reg[set] = static_cast<uint32_t>(pos & 3);
            // the block's 18 bytes lie in dwords d0 .. d0 + 4 (+ d0 + 5 when shift == 3): the
            // 16-byte load and d0 + 4 are inside the matrix, d0 + 5 is clamped to its last dword
            const size_t d0 = pos >> 2;
            const kk::u32x4_a4 v = kk::load_u32x4(w_base32 + d0);
#pragma unroll
            for (int t = 0; t < 4; ++t) b_reg[set][t] = v[t];
            b_reg[set][4] = w_base32[d0 + 4];
            b_reg[set][5] = w_base32[min(d0 + 5, w_last_dword)];
        }
    };

    auto store = [&](int step, int set, int buf) {
        _Float16 *a_lds = lds + buf * (kLdsA + kLdsB);
        _Float16 *b_lds = a_lds + kLdsA;
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4 *>(a_lds + a_dst[i]) = a_reg[set][i];
        if constexpr (F16W) {
            const int ks = min(step, steps - 1);
#pragma unroll
            for (int i = 0; i < kF16Chunks; ++i) {
                const int c = tid + kGemmThreads * i;
                const bool in = n0 + b_column(c >> 4) < n_rows && ks * kBK + (c & 15) * 8 < k;
                u32x4 v;
#pragma unroll
                for (int t = 0; t < 4; ++t) v[t] = in ? b_reg[set][4 * i + t] : 0u;
                *reinterpret_cast<u32x4 *>(b_lds + (c >> 4) * kLdsStride + (c & 15) * 8) = v;
            }
        } else {
            uint32_t e[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) e[i] = kk::align_bytes(b_reg[set][i + 1], b_reg[set][i], shift_reg[set]);
            half8 *bd = reinterpret_cast<half8 *>(b_lds + qb_row * kLdsStride + qb_blk * 32 + qb_half * 16);
            if constexpr (BN == 128) {
                half8 lo[2], hi[2];
                decode_q4_half(e, 0, live_reg[set], lo, tiny);
                decode_q4_half(e, 1, live_reg[set], hi, tiny);
                bd[0] = lo[0]; bd[1] = lo[1]; bd[2] = hi[0]; bd[3] = hi[1];
            } else {
                half8 out[2];
                decode_q4_half(e, qb_half, live_reg[set], out, tiny);
                bd[0] = out[0]; bd[1] = out[1];
            }
        }
    };

    float16v acc[2][kNT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < kNT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    auto mma = [&](int buf) {
        const _Float16 *a_lds = lds + buf * (kLdsA + kLdsB);
        const _Float16 *b_lds = a_lds + kLdsA;
#pragma unroll
        for (int s = 0; s < kBK / 32; ++s) {
            const int kc = (kh * (kBK / 32) + s) * 16 + 8 * (lane >> 5);
            half8 a[2], b[kNT];
#pragma unroll
            for (int it = 0; it < 2; ++it)
                a[it] = *reinterpret_cast<const half8 *>(a_lds + (wm * 64 + it * 32 + (lane & 31)) * kLdsStride + kc);
#pragma unroll
            for (int jt = 0; jt < kNT; ++jt)
                b[jt] = *reinterpret_cast<const half8 *>(b_lds + (wn * (BN / 2) + jt * 32 + (lane & 31)) * kLdsStride + kc);
#pragma unroll
            for (int it = 0; it < 2; ++it)
#pragma unroll
                for (int jt = 0; jt < kNT; ++jt)
                    acc[it][jt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[it], b[jt], acc[it][jt], 0, 0, 0);
        }
    };

    // Prologue: steps 0 .. kStages-1 in flight, step 0 in LDS buffer 0.
#pragma unroll
    for (int j = 0; j < kStages; ++j) load(j, j);
    store(0, 0, 0);
    __syncthreads();
    // At step s: LDS buffer s&1 holds step s, register sets hold steps
    // s+1 .. s+kStages-1, and set s % kStages (stored already) is free.
    for (int s0 = 0; s0 < steps; s0 += kStages) {
#pragma unroll
        for (int j = 0; j < kStages; ++j) {
            // sched_barrier keeps the loads issued before the MFMAs of the
            // step; the decode and LDS stores of the next step may interleave
            // with the MFMAs (the barrier of the previous step ended all reads
            // of the buffer they write).
            load(s0 + j + kStages, j);
            __builtin_amdgcn_sched_barrier(0);
            mma(j & 1);
            store(s0 + j + 1, (j + 1) % kStages, (j + 1) & 1);
            __syncthreads();
        }
    }

    // k-group 1 hands its sums to k-group 0 through LDS (all reads of the
    // tile buffers ended at the last barrier). D reg r of lane l: row
    // 8*(r/4) + 4*(l/32) + r%4, column l%32 of the 32 x 32 tile.
    float *red = reinterpret_cast<float *>(lds);
    const int sw = wid & 3;
    if (kh == 1) {
#pragma unroll
        for (int it = 0; it < 2; ++it)
#pragma unroll
            for (int jt = 0; jt < kNT; ++jt)
#pragma unroll
                for (int r = 0; r < 16; ++r) red[(((sw * 2 + it) * kNT + jt) * 16 + r) * kWave + lane] = acc[it][jt][r];
    }
    const bool any_tiny = __syncthreads_or(tiny) != 0;   // workgroup-uniform
    // subnormal-scale block masks of the B tile rows, after the k-group exchange
    uint32_t *tiny_masks = reinterpret_cast<uint32_t *>(red + 2 * 4 * kNT * 16 * kWave);
    static_assert(2 * 4 * kNT * 16 * kWave * 4 + BN * kTinyMaskWords * 4 <= gemm_lds_bytes<BN>(), "mask space");
    if (!F16W && any_tiny)
        build_tiny_masks(BN, blocks, [&](int j) -> const uint8_t * {
            const int n = n0 + b_column(j);
            return n < n_rows ? (b_matrix(j) ? w2 : w) + static_cast<size_t>(n) * row_bytes : nullptr;
        }, tiny_masks, kGemmThreads);
    if (kh == 1) return;
    const float wscale = F16W ? 1.0f : 8.0f;
    // Q4_0 blocks with subnormal scales (given the decode's fp16 rounding)
    // corrected in F32 into acc: lane column n of MFMA tile jt, rows m(it, r).
    if (!F16W && any_tiny) {
#pragma unroll
        for (int jt = 0; jt < kNT; ++jt) {
            const int j = wn * (BN / 2) + jt * 32 + (lane & 31);            // B tile row
            const int n = PAIR ? n0 + wn * 32 + (lane & 31) : n0 + j;
            if (n >= n_rows) continue;
            const uint8_t *wrow = (PAIR && jt == 1 ? w2 : w) + static_cast<size_t>(n) * row_bytes;
            const uint32_t *mask = tiny_masks + j * kTinyMaskWords;
#pragma unroll
            for (int it = 0; it < 2; ++it) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {   // D regs 4c .. 4c+3: rows 8c + 4(lane/32) + 0..3
                    auto row_of = [&](int r) { return m0 + wm * 64 + it * 32 + 8 * c + 4 * (lane >> 5) + r; };
                    float fix[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    auto decode = [](uint32_t nib, uint32_t bits) {
                        bool unused = false;
                        return decode_q4_dword(nib, q4_scale8(bits, true, unused));
                    };
                    tiny_scale_dots<4>(wrow, mask, blocks, x16, k_pad, row_of, decode, fix);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[it][jt][4 * c + r] += fix[r];
                }
            }
        }
    }
    if constexpr (PAIR) {
        const int n = n0 + wn * 32 + (lane & 31);
#pragma unroll
        for (int it = 0; it < 2; ++it) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + it * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const float s = row_inv[m] * wscale;
                const float g = (acc[it][0][r] + red[(((sw * 2 + it) * kNT + 0) * 16 + r) * kWave + lane]) * s;
                const float u = (acc[it][1][r] + red[(((sw * 2 + it) * kNT + 1) * 16 + r) * kWave + lane]) * s;
                if (m < m_rows && n < n_rows) y[static_cast<size_t>(m) * n_rows + n] = kk::swiglu_value(g, u);
            }
        }
        return;
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
#pragma unroll
        for (int jt = 0; jt < kNT; ++jt) {
            const int n = n0 + wn * (BN / 2) + jt * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + it * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const float v = acc[it][jt][r] + red[(((sw * 2 + it) * kNT + jt) * 16 + r) * kWave + lane];
                if (m < m_rows && n < n_rows) y[static_cast<size_t>(m) * n_rows + n] = v * (row_inv[m] * wscale);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// q4_lds_gemm: Q4_0 weights, K % 256 == 0, 16-byte aligned weight pointers.
//
// Workgroup tile: BM activation rows x CW*WN weight rows; 2*CW waves (CW = 4,
// or 8 for the 64 x 128 tile of one matrix: 16 waves, four per SIMD, hide
// more of each wave's read -> decode -> MFMA latency). Wave w owns weight
// rows WN*(w%CW) .. +WN over all BM rows and takes K32 slices 2*(w/CW),
// 2*(w/CW)+1 of every 128-K stage (two k-groups, whose sums meet in LDS at
// the end in a fixed order, so every tile sums in the same order).
//
// The waves copy the activation tile (BM x 128 fp16 per stage) and the raw
// Q4_0 bytes of the tile's weight rows (8 blocks = 144 B = nine 16-byte
// chunks per row and stage pair) from global memory straight into LDS
// (buffer_load_dwordx4 ... lds: 1 KB of LDS per wave instruction, no
// registers), two stages ahead: a ring of three activation stages and two
// weight stage pairs. Each wave decodes its own columns' blocks from LDS into
// v_mfma_f32_16x16x32_f16 B operands: a K32 slice is one Q4_0 block, and lane
// l takes column l%16 and nibble dword l/16, whose 8 values are block
// positions 8(l/16) .. +8 in the prepass's block order. No weight value is
// decoded twice and no decoded weight passes through LDS.
//
// LONG (the 64 x 128 tile, which leaves LDS to spare): 256-K stages, each
// one stage pair of weights, in rings of three activation stages and three
// weight buffers; a wave takes blocks 2*(w/CW), +1 and 4 + 2*(w/CW), +1 of a
// stage, the blocks and order two 128-K stages give it, so every tile sums
// in the same order. Half the stage barriers (K4096 x N4096 at batch 512:
// 38.9-39.4 -> 37.4 us per call).
//
// Activation row r of a stage is 16 (LONG: 32) chunks of 16 B; chunk c sits
// at position c ^ (r & 15), so the 16 lanes reading one operand row group hit
// 16 distinct bank quads. MFMA layout (wave64): A[l%16][8(l/16) .. +8),
// B[8(l/16) .. +8)[l%16], D[4(l/16) + r][l%16].
//
// Tiles are numbered weight-tile major and dealt to the 8 XCDs in contiguous
// ranges: the M tiles of one weight tile share an XCD and its L2.
constexpr int kQlK = 128;                   // K per stage (4 Q4_0 blocks)
constexpr int kQlABufs = 3;                 // activation stages in LDS
constexpr int kQlRowPair = 144;             // raw weight bytes per row and stage pair (8 blocks = 9 x 16 B)

template <int BM, int WN, bool PAIR, bool LONG, int CW = 4>
struct QlShape {
    static_assert(CW == 4 || (CW == 8 && !PAIR), "column waves per k-group");
    static constexpr int Waves = 2 * CW;                                // two k-groups
    static constexpr int Threads = 64 * Waves;
    static constexpr int BN = CW * WN;                                  // weight rows per tile
    static constexpr int RG = BM / 16, CG = WN / 16;                    // MFMA tiles per wave
    static constexpr int KS = LONG ? 2 * kQlK : kQlK;                   // K per stage
    static constexpr int Chunks = KS / 8;                               // 16-byte chunks per activation row
    static constexpr int ABytes = BM * KS * 2;                          // one stage of activations
    static constexpr int ACopiesPerWave = BM * Chunks / 64 / Waves;     // 1 KB each, per stage
    static_assert(ACopiesPerWave * 64 * Waves == BM * Chunks, "whole activation copies per wave");
    static constexpr int BBufs = LONG ? 3 : 2;                          // weight buffers (stage pairs)
    // weights: 1 KB copies per stage pair; PAIR: the gate rows' copies, then
    // the up rows' from HalfCopies on (each half padded to whole copies; the
    // up rows start at UpBase in the stage-pair buffer)
    static constexpr int HalfCopies = (BN / 2 * (kQlRowPair / 16) + 63) / 64;
    static constexpr int BCopies = PAIR ? 2 * HalfCopies : BN * (kQlRowPair / 16) / 64;
    static_assert(PAIR || BCopies * 64 == BN * (kQlRowPair / 16), "whole weight copies");
    static constexpr int UpBase = PAIR ? HalfCopies * 1024 : BN / 2 * kQlRowPair;
    static constexpr int BBytes = PAIR ? BCopies * 1024 : BN * kQlRowPair;   // one stage pair of weights
    static constexpr int BCopiesPerWave = (BCopies + Waves - 1) / Waves;   // waves below BCopies % Waves
    static constexpr int BCopiesRem = BCopies % Waves;                     // (if not 0) issue one more
    static constexpr int TileStride = BN + 4;                           // floats per LDS output row
    static constexpr int XferBytes = BM * TileStride * 4;
    static constexpr int CopyBytes = kQlABufs * ABytes + BBufs * BBytes;
    static constexpr int RingBytes = CopyBytes > XferBytes ? CopyBytes : XferBytes;
    static constexpr int LdsBytes = RingBytes + BM * 4;                 // + the tile's row scales
    static_assert(ACopiesPerWave + BCopiesPerWave <= 15, "vmcnt immediate");
    static_assert(LdsBytes <= 160 * 1024, "LDS");
};

// The subnormal-scale corrections of one wave's work items (item = one
// weight row of the tile and 64 activation rows, a lane per row; items it0,
// it0 + stride, ... below n_items): for each item, the sum over its row's
// marked blocks, in increasing order, of x16 . (v - decode(v)), exactly as
// tiny_scale_dots sums it, added to the lane's output (out_of). The walk over
// the items' marked blocks is wave-uniform; NB marked blocks (of one item or
// of several) are loaded at once (weight bytes at one address for all lanes,
// and each lane's activations), then added in order. Lane p < 32 computes the
// difference for block position p once, every lane takes it by readlane.
// Items without marked blocks are not touched.
template <int NB, typename MaskOf, typename RowOf, typename XOf, typename OutOf>
__device__ void tiny_fix_items(int it0, int stride, int n_items, int blocks, MaskOf mask_of, RowOf wrow_of, XOf xrow_of,
                               OutOf out_of) {
    const int lane = threadIdx.x & (kWave - 1);
    const int pi = (lane >> 3) & 3, pt = lane & 7;               // block position 8 pi + pt of lanes 0..31
    const int words = (blocks + 31) / 32;
    int it = it0, word = 0;
    uint32_t left = it < n_items && wrow_of(it) ? __builtin_amdgcn_readfirstlane(mask_of(it)[0]) : 0u;
    int cur = -1;
    float fix = 0.0f;
    for (;;) {
        int pit[NB], pb[NB];
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            while (left == 0u && it < n_items) {                 // wave-uniform walk
                if (word + 1 < words) {
                    left = __builtin_amdgcn_readfirstlane(mask_of(it)[++word]);
                } else {
                    it += stride;
                    word = 0;
                    left = it < n_items && wrow_of(it) ? __builtin_amdgcn_readfirstlane(mask_of(it)[0]) : 0u;
                }
            }
            pit[c] = left ? it : -1;
            pb[c] = left ? 32 * word + __builtin_ctz(left) : 0;
            left &= left - 1u;
        }
        if (pit[0] < 0) break;
        uint32_t hw[NB][9];
        half8 xv[NB][4];
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            const int ic = pit[c] >= 0 ? pit[c] : pit[0], bc = pit[c] >= 0 ? pb[c] : pb[0];   // an empty slot re-reads
            const uint16_t *hp = reinterpret_cast<const uint16_t *>(wrow_of(ic) + 18 * bc);
#pragma unroll
            for (int t = 0; t < 9; ++t) hw[c][t] = hp[t];
            const _Float16 *xp = xrow_of(ic) + 32 * bc;
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[c][i] = *reinterpret_cast<const half8 *>(xp + 8 * i);
        }
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            if (pit[c] < 0) break;                               // wave-uniform
            if (pit[c] != cur) {
                if (cur >= 0) *out_of(cur) += fix;
                cur = pit[c];
                fix = 0.0f;
            }
            const uint32_t bits = hw[c][0];
            const float d = ldexpf(static_cast<float>(bits & 0x3ffu), -27) * ((bits & 0x8000u) ? -1.0f : 1.0f);   // d / 8
            // this lane's position 8 pi + pt (nibble dword pi, slot pt)
            const uint32_t nib = pi == 0 ? hw[c][1] | hw[c][2] << 16
                               : pi == 1 ? hw[c][3] | hw[c][4] << 16
                               : pi == 2 ? hw[c][5] | hw[c][6] << 16 : hw[c][7] | hw[c][8] << 16;
            const half8 dec = decode_q4_scaled(nib, bits);
            const uint32_t byte = (nib >> (8 * ((pt & 1) << 1 | (pt & 2) >> 1))) & 0xffu;   // bytes 0, 2, 1, 3
            const uint32_t q = pt < 4 ? byte & 15u : byte >> 4;
            _Float16 dl = dec[0];
#pragma unroll
            for (int t = 1; t < 8; ++t) dl = pt == t ? dec[t] : dl;
            const float wv = (static_cast<float>(q) - 8.0f) * d - static_cast<float>(dl);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wv), 8 * i + t));
                    fix += static_cast<float>(xv[c][i][t]) * ws;
                }
        }
        if (pit[NB - 1] < 0) break;
    }
    if (cur >= 0) *out_of(cur) += fix;
}

// build_tiny_masks for a workgroup of W waves with one weight row per wave
// task: wave w takes rows w, w + W, ..., lane l blocks l, l + 64, ...; each
// 64-block group's marks are one ballot, written by lane 0 (no atomics, no
// division). Rows are processed RB at a time with all their scale loads
// issued together. Every mask word below (blocks + 31) / 32 of every row is
// written; two workgroup barriers.
template <int W, typename RowPtr>
__device__ void build_tiny_masks_rows(int rows, int blocks, RowPtr row_ptr, uint32_t *masks) {
    constexpr int RB = 4;
    constexpr int kGroups = kTinyMaskWords / 2;                 // 64-block groups (K <= 16384)
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int groups = (blocks + 63) / 64;
    __syncthreads();                                            // the LDS the masks go into is idle
    for (int j0 = wid * RB; j0 < rows; j0 += W * RB) {          // wave-uniform
        uint32_t bits[RB][kGroups];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const uint8_t *wrow = j0 + r < rows ? row_ptr(j0 + r) : nullptr;
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                const int b = 64 * g + lane;
                bits[r][g] = wrow && g < groups && b < blocks ? *reinterpret_cast<const uint16_t *>(wrow + 18 * b) : 0u;
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            if (j0 + r >= rows) break;                          // wave-uniform
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                if (g >= groups) break;                         // wave-uniform
                const bool t = (bits[r][g] & 0x7c00u) == 0 && (bits[r][g] & 0x3ffu) != 0;
                const uint64_t m = __ballot(t);
                if (lane == 0) {
                    masks[(j0 + r) * kTinyMaskWords + 2 * g] = static_cast<uint32_t>(m);
                    masks[(j0 + r) * kTinyMaskWords + 2 * g + 1] = static_cast<uint32_t>(m >> 32);
                }
            }
        }
    }
    __syncthreads();
}

// Copies of a q4_lds_gemm workgroup's wave `wid` (buffer_load_dwordx4 ... lds,
// 1 KB of LDS each): the activation copies wid + Waves*t of stage s into A
// buffer s % 3, and the weight copies wid + Waves*t (below BCopies; PAIR: below
// HalfCopies from the gate matrix, the rest from the up matrix) of stage pair
// p into B buffer p % 2. Offsets are per lane and fixed over stages; the stage
// offset is the SGPR soffset. (Separate functions, not lambdas of the kernel:
// the host pass rejects a kernel-local lambda that hands captured values to
// these builtins, and then drops the launch stub.)
template <typename S>
__device__ __forceinline__ void ql_copy_a(const uint32_t (&a_off)[S::ACopiesPerWave], _Float16 *a_tile, int a_extent,
                                          int wid, int s) {
    extern __shared__ __align__(16) uint8_t ql_lds[];
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(a_tile, 0, a_extent, 0x00020000);
    const int buf = (s % kQlABufs) * S::ABytes;
#pragma unroll
    for (int t = 0; t < S::ACopiesPerWave; ++t)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) uint8_t *)ql_lds + buf + (wid + S::Waves * t) * 1024,
                                                 16, a_off[t], s * (S::KS * 2), 0, 0);
}

template <typename S, bool PAIR>
__device__ __forceinline__ void ql_copy_b(const uint32_t (&b_off)[S::BCopiesPerWave], uint8_t *b_tile,
                                          uint8_t *b_tile2, int b_extent, int wid, int p) {
    extern __shared__ __align__(16) uint8_t ql_lds[];
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(b_tile, 0, b_extent, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsrc2 = __builtin_amdgcn_make_buffer_rsrc(b_tile2, 0, b_extent, 0x00020000);
    const int buf = kQlABufs * S::ABytes + (p % S::BBufs) * S::BBytes;
#pragma unroll
    for (int t = 0; t < S::BCopiesPerWave; ++t) {
        const int i = wid + S::Waves * t;
        if (i < S::BCopies)                                     // wave-uniform
            __builtin_amdgcn_raw_ptr_buffer_load_lds(PAIR && i >= S::HalfCopies ? rsrc2 : rsrc,
                                                     (__attribute__((address_space(3))) uint8_t *)ql_lds + buf + i * 1024,
                                                     16, b_off[t], p * kQlRowPair, 0, 0);
    }
}

// PAIR: the stage's weight rows are the tile's BN/2 gate rows (matrix w), then
// its BN/2 up rows (matrix w2, from S::UpBase); waves 0-1 (tile columns
// 0 .. BN/2) take the gate rows and waves 2-3 the up rows of the same output
// columns, which the epilogue pairs in LDS.
template <int BM, int WN, bool PAIR, bool LONG, int CW = 4>
__global__ __launch_bounds__(128 * CW) void q4_lds_gemm(const uint8_t *__restrict__ w, const uint8_t *__restrict__ w2,
                                                         const _Float16 *__restrict__ x16,
                                                         const float *__restrict__ row_inv, float *__restrict__ y,
                                                         int m_rows, int n_rows, int k_pad, int stages,
                                                         uint32_t row_bytes, int m_tiles, int tiles, int tiles_per_xcd) {
    using S = QlShape<BM, WN, PAIR, LONG, CW>;
    constexpr int kOut = PAIR ? S::BN / 2 : S::BN;             // output columns per tile
    constexpr int kQlThreads = S::Threads;
    extern __shared__ __align__(16) uint8_t ql_lds[];

    const int bid = blockIdx.x;
    const int tile = (bid % kXcds) * tiles_per_xcd + bid / kXcds;
    if (tile >= tiles) return;                                  // whole workgroup, before any barrier
    const int nt = tile / m_tiles;
    const int mt = tile - nt * m_tiles;
    const int m0 = mt * BM, n0 = nt * kOut;
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int kh = wid / CW, wn = wid % CW;
    const int g = lane >> 4, c16 = lane & 15;
    // The tile's row scales, loaded before the first copy and handed to the
    // epilogue through LDS: no global load there (on gfx9 a wait for a load
    // also waits for every store issued before it). The load is unconditional
    // (threads past BM repeat row BM - 1 of the padded rows) and its value is
    // first used in the epilogue, so no wait for it precedes the copies.
    const float row_inv_raw = row_inv[m0 + min(static_cast<int>(threadIdx.x), BM - 1)];
    float *scale_lds = reinterpret_cast<float *>(ql_lds + S::RingBytes);

    // Copies are raw buffer loads into LDS (buffer_load ... lds): the tile's
    // base and extent in a buffer resource, the per-lane byte offset (fixed
    // over stages) in a VGPR and the stage offset (256 B of activations per
    // row and stage, 144 B of weights per row and stage pair) in an SGPR, so a
    // copy costs no address arithmetic; reads past the extent return 0.
    // A copy i: rows 4i .. 4i+3 of the tile, lane -> row 4i + lane/16, LDS
    // position lane%16, which holds chunk (lane%16) ^ (row & 15).
    _Float16 *const a_tile = const_cast<_Float16 *>(x16 + static_cast<size_t>(m0) * k_pad);
    const int a_extent = BM * k_pad * 2;
    uint32_t a_off[S::ACopiesPerWave];
#pragma unroll
    for (int t = 0; t < S::ACopiesPerWave; ++t) {
        constexpr int kRowsPerCopy = 64 / S::Chunks;
        const int r = kRowsPerCopy * (wid + S::Waves * t) + lane / S::Chunks, pos = lane % S::Chunks;
        a_off[t] = static_cast<uint32_t>(r * k_pad + 8 * (pos ^ (r & 15))) * 2;
    }
    // B copy i: 16-byte chunks 64c .. 64c+63 (c = i, or i - HalfCopies for the
    // up rows of PAIR) of the [row][144 B] stage-pair bytes, 9 chunks per row.
    constexpr int kRows = PAIR ? S::BN / 2 : S::BN;             // weight rows per matrix and tile
    const int b_extent = min(kRows, n_rows - n0) * static_cast<int>(row_bytes);
    uint8_t *const b_tile = const_cast<uint8_t *>(w + static_cast<size_t>(n0) * row_bytes);
    uint8_t *const b_tile2 = const_cast<uint8_t *>(w2 + static_cast<size_t>(n0) * row_bytes);
    uint32_t b_off[S::BCopiesPerWave];
#pragma unroll
    for (int t = 0; t < S::BCopiesPerWave; ++t) {
        const int i = wid + S::Waves * t;
        const int q = (PAIR && i >= S::HalfCopies ? i - S::HalfCopies : i) * 64 + lane;   // past the rows: clamped
        const int row = min(q / (kQlRowPair / 16), kRows - 1);
        const int chunk = q - (q / (kQlRowPair / 16)) * (kQlRowPair / 16);
        const int wrow = min(n0 + row, n_rows - 1) - n0;
        b_off[t] = static_cast<uint32_t>(wrow) * row_bytes + 16 * chunk;
    }
    // this wave's copies per stage (activations) and per stage pair (weights)
    const int my_b_copies = S::BCopiesRem == 0 || wid < S::BCopiesRem ? S::BCopiesPerWave : S::BCopiesPerWave - 1;

    float4v acc[S::RG][S::CG];
#pragma unroll
    for (int i = 0; i < S::RG; ++i)
#pragma unroll
        for (int j = 0; j < S::CG; ++j) acc[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    bool tiny = false;   // set once this lane skipped a block with a subnormal scale

    // One stage: this k-group's two K32 slices. Operand reads run one MFMA
    // group ahead (the next two A row tiles, or the next slice's weight bytes
    // and first A tiles, are read before the current group's MFMAs issue), so
    // LDS latency hides behind MFMA work.
    // b_lds: this stage's 72 bytes of each weight row (row stride 144 B; the
    // 16 rows of one read land in 16 distinct banks).
    auto read_b = [&](const uint8_t *b_lds, int j, uint32_t (&nib)[S::CG], uint32_t (&sbits)[S::CG]) {
#pragma unroll
        for (int cg = 0; cg < S::CG; ++cg) {
            const uint8_t *blk = !PAIR ? b_lds + (wn * WN + cg * 16 + c16) * kQlRowPair + 18 * j
                                       : b_lds + (wn >= 2 ? S::UpBase : 0) +
                                             ((wn & 1) * WN + cg * 16 + c16) * kQlRowPair + 18 * j;
            sbits[cg] = *reinterpret_cast<const uint16_t *>(blk);
            if ((j & 1) == 0) {   // even block: starts on a dword, nibble dword g at +2 + 4g
                const uint32_t *p = reinterpret_cast<const uint32_t *>(blk + 4 * g);
                nib[cg] = __builtin_amdgcn_alignbyte(p[1], p[0], 2);
            } else {              // odd block: starts 2 B past a dword, nibble dword g on a dword
                nib[cg] = *reinterpret_cast<const uint32_t *>(blk + 2 + 4 * g);
            }
        }
    };
    auto read_a = [&](const uint8_t *a_lds, int j, int rg) {
        return *reinterpret_cast<const half8 *>(a_lds + (rg * 16 + c16) * (S::KS * 2) + ((4 * j + g) ^ c16) * 16);
    };
    // blocks jb, jb + 1 of the stage (jb = 2 kh, and for LONG also 4 + 2 kh)
    auto compute = [&](const uint8_t *a_lds, const uint8_t *b_lds, int jb) {
        const int j0 = jb, j1 = j0 + 1;
        uint32_t nib[S::CG], sbits[S::CG];
        half8 b0[S::CG], b1[S::CG];
        read_b(b_lds, j0, nib, sbits);
        half8 a0 = read_a(a_lds, j0, 0), a1 = read_a(a_lds, j0, 1);
#pragma unroll
        for (int cg = 0; cg < S::CG; ++cg) {
            note_tiny_scale(sbits[cg], tiny);
            b0[cg] = decode_q4_scaled(nib[cg], sbits[cg]);
        }
        // Block j0: the first MFMA group also reads block j1's weight bytes,
        // and each later group decodes some of them after issuing its MFMAs
        // (the decode overlaps MFMA execution instead of stalling it).
#pragma unroll
        for (int rg = 0; rg < S::RG; rg += 2) {
            const int grp = rg / 2;
            half8 n0, n1;
            if (rg + 2 < S::RG) {
                n0 = read_a(a_lds, j0, rg + 2);
                n1 = read_a(a_lds, j0, rg + 3);
            } else {
                n0 = read_a(a_lds, j1, 0);
                n1 = read_a(a_lds, j1, 1);
            }
            if (grp == 0) read_b(b_lds, j1, nib, sbits);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int cg = 0; cg < S::CG; ++cg) {
                acc[rg][cg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0[cg], acc[rg][cg], 0, 0, 0);
                acc[rg + 1][cg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b0[cg], acc[rg + 1][cg], 0, 0, 0);
            }
#pragma unroll
            for (int cg = 0; cg < S::CG; ++cg)
                if (grp > 0 && (cg + 1 < S::RG / 2 ? cg + 1 : S::RG / 2 - 1) == grp) {
                    note_tiny_scale(sbits[cg], tiny);
                    b1[cg] = decode_q4_scaled(nib[cg], sbits[cg]);
                }
            // one MFMA, then up to 3 VALU (the decode), alternately
#pragma unroll
            for (int m = 0; m < 2 * S::CG; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            a0 = n0;
            a1 = n1;
        }
        // Block j1.
#pragma unroll
        for (int rg = 0; rg < S::RG; rg += 2) {
            half8 n0 = a0, n1 = a1;
            if (rg + 2 < S::RG) {
                n0 = read_a(a_lds, j1, rg + 2);
                n1 = read_a(a_lds, j1, rg + 3);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int cg = 0; cg < S::CG; ++cg) {
                acc[rg][cg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b1[cg], acc[rg][cg], 0, 0, 0);
                acc[rg + 1][cg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1[cg], acc[rg + 1][cg], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            a0 = n0;
            a1 = n1;
        }
    };

    // Issue order: A(0), B(0), A(1); then at stage s (after its wait and the
    // barrier) A(s+2) and, at even s, B(s/2 + 1). The memory counter is in
    // order, so at the top of stage s: even s needs A(s) and B(s/2), which
    // leaves A(s+1) in flight; odd s needs A(s), which leaves A(s+1) and
    // B((s+1)/2) in flight. The barrier then makes every wave's copies
    // visible and ends all reads of the buffers the next copies refill
    // (stage s-1's activations, stage pair s/2 - 1's weights).
    // LONG (256-K stages, one stage pair of weights each, three weight
    // buffers): A(0), B(0), A(1), B(1); at stage s A(s+2) and B(s+2); the top
    // of stage s leaves A(s+1) and B(s+1) in flight. The k-groups take the
    // same blocks in the same order as two 128-K stages would give them.
    ql_copy_a<S>(a_off, a_tile, a_extent, wid, 0);
    ql_copy_b<S, PAIR>(b_off, b_tile, b_tile2, b_extent, wid, 0);
    if (stages > 1) {
        ql_copy_a<S>(a_off, a_tile, a_extent, wid, 1);
        if (LONG) ql_copy_b<S, PAIR>(b_off, b_tile, b_tile2, b_extent, wid, 1);
    }
    for (int s = 0; s < stages; ++s) {
        if (s + 1 >= stages)
            __builtin_amdgcn_s_waitcnt(0x0F70);
        else if (!LONG && (s & 1) == 0)
            __builtin_amdgcn_s_waitcnt(0x0F70 | S::ACopiesPerWave);
        else if (my_b_copies == S::BCopiesPerWave)              // wave-uniform
            __builtin_amdgcn_s_waitcnt(0x0F70 | (S::ACopiesPerWave + S::BCopiesPerWave));
        else
            __builtin_amdgcn_s_waitcnt(0x0F70 | (S::ACopiesPerWave + S::BCopiesPerWave - 1));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        if (s + 2 < stages) {
            ql_copy_a<S>(a_off, a_tile, a_extent, wid, s + 2);
            if (LONG)
                ql_copy_b<S, PAIR>(b_off, b_tile, b_tile2, b_extent, wid, s + 2);
            else if ((s & 1) == 0)
                ql_copy_b<S, PAIR>(b_off, b_tile, b_tile2, b_extent, wid, s / 2 + 1);
        }
        const uint8_t *a_lds = ql_lds + (s % kQlABufs) * S::ABytes;
        if (LONG) {
            const uint8_t *b_lds = ql_lds + kQlABufs * S::ABytes + (s % S::BBufs) * S::BBytes;
            compute(a_lds, b_lds, 2 * kh);
            compute(a_lds, b_lds, 4 + 2 * kh);
        } else {
            compute(a_lds, ql_lds + kQlABufs * S::ABytes + ((s >> 1) & 1) * S::BBytes + (s & 1) * (kQlRowPair / 2),
                    2 * kh);
        }
    }

    // Epilogue. k-group 1 writes its sums into a row-major LDS tile (row
    // stride BN + 4 floats: the 4 rows of one write land 16 banks apart);
    // k-group 0 adds its own (acc0 + acc1, a fixed order) and applies the row
    // scales in place; then all waves store whole tile rows.
    __syncthreads();                                            // ring idle
    constexpr int kTs = S::TileStride;
    float *tile_lds = reinterpret_cast<float *>(ql_lds);
    if (threadIdx.x < BM) scale_lds[threadIdx.x] = row_inv_raw * 8.0f;
    if (kh == 1) {
#pragma unroll
        for (int rg = 0; rg < S::RG; ++rg)
#pragma unroll
            for (int cg = 0; cg < S::CG; ++cg)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    tile_lds[(rg * 16 + 4 * g + r) * kTs + wn * WN + cg * 16 + c16] = acc[rg][cg][r];
    }
    if (__syncthreads_or(tiny)) {   // workgroup-uniform
        // Q4_0 blocks with subnormal scales (given the decode's fp16
        // rounding) corrected in F32 into k-group 1's sums: the marked blocks
        // of each B tile row j.
        static_assert(S::XferBytes + S::BN * kTinyMaskWords * 4 <= S::RingBytes, "mask space");
        uint32_t *tiny_masks = reinterpret_cast<uint32_t *>(ql_lds + S::XferBytes);
        const int nblocks = static_cast<int>(row_bytes / 18);
        build_tiny_masks_rows<S::Waves>(S::BN, nblocks, [&](int j) -> const uint8_t * {
            const int h = PAIR ? j / (S::BN / 2) : 0, jr = PAIR ? j % (S::BN / 2) : j;
            return n0 + jr < n_rows ? (h ? w2 : w) + static_cast<size_t>(n0 + jr) * row_bytes : nullptr;
        }, tiny_masks);
        // work item = (tile column j, 64 activation rows rh), a lane per row
        static_assert(BM % 64 == 0, "fixup rows");
        auto wrow_of = [&](int item) -> const uint8_t * {
            const int j = item % S::BN;
            const int h = PAIR ? j / (S::BN / 2) : 0, jr = PAIR ? j % (S::BN / 2) : j;   // matrix, row in it
            return n0 + jr < n_rows ? (h ? w2 : w) + static_cast<size_t>(n0 + jr) * row_bytes : nullptr;
        };
        tiny_fix_items<2>(wid, S::Waves, S::BN * (BM / 64), nblocks,
                          [&](int item) { return tiny_masks + (item % S::BN) * kTinyMaskWords; }, wrow_of,
                          [&](int item) { return x16 + static_cast<size_t>(m0 + 64 * (item / S::BN) + lane) * k_pad; },
                          [&](int item) { return tile_lds + (64 * (item / S::BN) + lane) * kTs + item % S::BN; });
        __syncthreads();
    }
    if (kh == 0) {
#pragma unroll
        for (int rg = 0; rg < S::RG; ++rg)
#pragma unroll
            for (int cg = 0; cg < S::CG; ++cg)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = rg * 16 + 4 * g + r;
                    float *t = tile_lds + row * kTs + wn * WN + cg * 16 + c16;
                    *t = (acc[rg][cg][r] + *t) * scale_lds[row];
                }
    }
    __syncthreads();
    // PAIR: output column c is SiLU(tile column c) * (tile column BN/2 + c)
    constexpr int kQuads = kOut / 4;
    const bool vec = (n_rows & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    for (int i = threadIdx.x; i < BM * kQuads; i += kQlThreads) {
        const int row = i / kQuads, q = i - row * kQuads;
        const int m = m0 + row, n = n0 + 4 * q;
        if (m >= m_rows || n >= n_rows) continue;
        float4v v = *reinterpret_cast<const float4v *>(tile_lds + row * kTs + 4 * q);
        if constexpr (PAIR) {
            const float4v u = *reinterpret_cast<const float4v *>(tile_lds + row * kTs + S::BN / 2 + 4 * q);
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = kk::swiglu_value(v[t], u[t]);
        }
        float *dst = y + static_cast<size_t>(m) * n_rows + n;
        if (vec && n + 3 < n_rows) {
            __builtin_nontemporal_store(v, reinterpret_cast<float4v *>(dst));   // streamed out, not kept in L2
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (n + t < n_rows) dst[t] = v[t];
        }
    }
}

struct GemmPlan {
    int m_pad, k_pad, m_tiles, bn, n_tiles;
    size_t x16_bytes, row_inv_bytes;
};

// Tile N: 128 (fewer LDS reads per MFMA) when that still gives every CU a
// tile, else 64. The kGemmBn knob (KUNLUN_GEMM_BN=64|128) overrides.
GemmPlan plan(int k, int n, int batch) {
    GemmPlan p;
    p.m_pad = static_cast<int>(round_up(static_cast<size_t>(batch), kBM));
    p.k_pad = static_cast<int>(round_up(static_cast<size_t>(k), kKAlign));
    p.m_tiles = p.m_pad / kBM;
    const int want = kk::tuning(kk::kGemmBn);
    p.bn = want == 64 || want == 128 ? want : (p.m_tiles * ((n + 127) / 128) >= 256 ? 128 : 64);
    p.n_tiles = (n + p.bn - 1) / p.bn;
    p.x16_bytes = round_up(static_cast<size_t>(p.m_pad) * p.k_pad * 2, 256);
    p.row_inv_bytes = round_up(static_cast<size_t>(p.m_pad) * 4, 256);
    return p;
}

template <bool F16W, int BN, bool PAIR = false>
hipError_t launch_gemm(const void *w, const void *w2, const _Float16 *x16, const float *row_inv, float *y, int batch,
                       int n, int k, const GemmPlan &p, size_t w_bytes, hipStream_t stream) {
    const hipError_t rc =
        kk::opt_in_lds(reinterpret_cast<const void *>(&mfma_gemm<F16W, BN, PAIR>), gemm_lds_bytes<BN>());
    if (rc != hipSuccess) return rc;
    const int tiles = p.m_tiles * p.n_tiles;
    const int tiles_per_xcd = (tiles + kXcds - 1) / kXcds;
    hipLaunchKernelGGL((mfma_gemm<F16W, BN, PAIR>), dim3(tiles_per_xcd * kXcds), dim3(kGemmThreads),
                       gemm_lds_bytes<BN>(), stream, static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(w2),
                       x16, row_inv, y, batch, n, k, p.k_pad, w_bytes, p.n_tiles, tiles, tiles_per_xcd);
    return hipGetLastError();
}

int device_cus() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return 256;
    return kk::cu_count(device);
}

struct QlTile {
    int bm, wn;
};

// The candidate with the smallest estimated time: whole rounds of tiles over
// the CUs x tile work, with penalties for the LDS activation reads per MFMA
// (~1/WN) and the weight decode per MFMA (~1/BM). The kGemmTile knob
// (KUNLUN_GEMM_TILE=BMxWN, e.g. 128x48) forces a candidate.
QlTile pick_ql_tile(int batch, int n, bool pair) {
    static const QlTile kAll[] = {{128, 48}, {128, 32}, {64, 64}, {64, 32}};
    auto allowed = [](const QlTile &) { return true; };
    const int forced = kk::tuning(kk::kGemmTile);
    if (forced > 0)
        for (const QlTile &t : kAll)
            if (t.bm * 1000 + t.wn == forced && allowed(t)) return t;
    const long cus = device_cus();
    QlTile pick = {128, 32};
    double best = 0.0;
    for (const QlTile &t : kAll) {
        if (!allowed(t)) continue;
        const long out = pair ? 2 * t.wn : 4 * t.wn;
        const long tiles = (static_cast<long>(batch) + t.bm - 1) / t.bm * ((n + out - 1) / out);
        const long rounds = (tiles + cus - 1) / cus;
        const double cost = static_cast<double>(rounds) * t.bm * 4 * t.wn * (1.0 + 16.0 / t.wn) * (1.0 + 32.0 / t.bm);
        if (best == 0.0 || cost < best) {
            best = cost;
            pick = t;
        }
    }
    return pick;
}

template <int BM, int WN, bool PAIR, bool LONG = false, int CW = 4>
hipError_t launch_ql_gemm(const void *w, const void *w2, const _Float16 *x16, const float *row_inv, float *y, int batch,
                          int n, int k, int k_pad, hipStream_t stream) {
    using S = QlShape<BM, WN, PAIR, LONG, CW>;
    hipError_t rc = kk::opt_in_lds(reinterpret_cast<const void *>(&q4_lds_gemm<BM, WN, PAIR, LONG, CW>), S::LdsBytes);
    if (rc != hipSuccess) return rc;
    const int out = PAIR ? S::BN / 2 : S::BN;
    const int m_tiles = (batch + BM - 1) / BM;
    const int tiles = m_tiles * ((n + out - 1) / out);
    const int tiles_per_xcd = (tiles + kXcds - 1) / kXcds;
    const uint32_t row_bytes = static_cast<uint32_t>(k / 32 * 18);
    hipLaunchKernelGGL((q4_lds_gemm<BM, WN, PAIR, LONG, CW>), dim3(tiles_per_xcd * kXcds), dim3(S::Threads), S::LdsBytes,
                       stream, static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(w2), x16, row_inv, y, batch,
                       n, k_pad, k / S::KS, row_bytes, m_tiles, tiles, tiles_per_xcd);
    return hipGetLastError();
}

template <bool PAIR>
hipError_t launch_ql(const void *w, const void *w2, const _Float16 *x16, const float *row_inv, float *y, int batch,
                     int n, int k, int k_pad, hipStream_t stream) {
    const QlTile t = pick_ql_tile(batch, n, PAIR);
    if (t.bm == 128 && t.wn == 32) return launch_ql_gemm<128, 32, PAIR>(w, w2, x16, row_inv, y, batch, n, k, k_pad, stream);
    if (t.bm == 64 && t.wn == 64) return launch_ql_gemm<64, 64, PAIR>(w, w2, x16, row_inv, y, batch, n, k, k_pad, stream);
    if (t.bm == 64 && t.wn == 32) {
        // 64 x 128 tile: 16 waves of 64 x 16 for one matrix (twice the waves per SIMD to hide
        // the read -> decode -> MFMA latency; same k-groups, so the same bits), 8 of 64 x 32 for a pair
        if constexpr (PAIR) return launch_ql_gemm<64, 32, true, true>(w, w2, x16, row_inv, y, batch, n, k, k_pad, stream);
        else return launch_ql_gemm<64, 16, false, true, 8>(w, w2, x16, row_inv, y, batch, n, k, k_pad, stream);
    }
    if (t.bm == 128 && t.wn == 48) return launch_ql_gemm<128, 48, PAIR>(w, w2, x16, row_inv, y, batch, n, k, k_pad, stream);
    return hipErrorInvalidValue;
}

// The LDS-copy Q4_0 GEMM takes K in whole stage pairs (256) and 16-byte aligned
// weights (rows of (K / 256) * 144 bytes, copied 16 bytes per lane).
bool ql_shape(int k, const void *w, const void *w2) {
    return k % (2 * kQlK) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(w2) & 15) == 0;
}

} // namespace

extern "C" size_t kk_gemm_workspace_bytes(int k, int n, int batch) {
    const GemmPlan p = plan(k, n, batch);
    return p.x16_bytes + p.row_inv_bytes;
}

extern "C" int kk_gemm(int type, const void *w, const float *x, float *y, int k, int n, int batch, void *workspace,
                       hipStream_t stream, const char **route) {
    if ((type != 1 && type != 2) || !w || !x || !y || !workspace || k <= 0 || (k & 31) || n <= 0 || batch <= 0 ||
        k > 16384)
        return hipErrorInvalidValue;
    if (type == 1 && ((reinterpret_cast<uintptr_t>(w) & 15) || (k & 15))) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(x) & 15)) return hipErrorInvalidValue;
    const GemmPlan p = plan(k, n, batch);
    char *ws = static_cast<char *>(workspace);
    _Float16 *x16 = reinterpret_cast<_Float16 *>(ws);
    float *row_inv = reinterpret_cast<float *>(ws + p.x16_bytes);
    launch_x_to_f16(type == 2, x, batch, k, p.m_pad, p.k_pad, x16, row_inv, stream);
    hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) return rc;
    const size_t w_bytes = type == 1 ? static_cast<size_t>(n) * k * 2 : static_cast<size_t>(n) * (k / 32) * 18;
    if (route) *route = type == 2 ? "q4_gemm_mfma" : "f16_gemm_mfma";
    if (type == 2 && ql_shape(k, w, w)) return launch_ql<false>(w, w, x16, row_inv, y, batch, n, k, p.k_pad, stream);
    if (type == 2)
        return p.bn == 128 ? launch_gemm<false, 128>(w, w, x16, row_inv, y, batch, n, k, p, w_bytes, stream)
                           : launch_gemm<false, 64>(w, w, x16, row_inv, y, batch, n, k, p, w_bytes, stream);
    return p.bn == 128 ? launch_gemm<true, 128>(w, w, x16, row_inv, y, batch, n, k, p, w_bytes, stream)
                       : launch_gemm<true, 64>(w, w, x16, row_inv, y, batch, n, k, p, w_bytes, stream);
}

extern "C" int kk_gemm_swiglu(int type, const void *w_gate, const void *w_up, const float *x, float *y, int k, int n,
                              int batch, void *workspace, hipStream_t stream, const char **route) {
    if ((type != 1 && type != 2) || !w_gate || !w_up || !x || !y || !workspace || k <= 0 || (k & 31) || n <= 0 ||
        batch <= 0 || k > 16384)
        return hipErrorInvalidValue;
    if (type == 1 && ((reinterpret_cast<uintptr_t>(w_gate) & 15) || (reinterpret_cast<uintptr_t>(w_up) & 15)))
        return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(x) & 15)) return hipErrorInvalidValue;
    GemmPlan p = plan(k, n, batch);
    p.bn = 128;                                 // 64 rows of each matrix per tile
    p.n_tiles = (n + 63) / 64;
    char *ws = static_cast<char *>(workspace);
    _Float16 *x16 = reinterpret_cast<_Float16 *>(ws);
    float *row_inv = reinterpret_cast<float *>(ws + p.x16_bytes);
    launch_x_to_f16(type == 2, x, batch, k, p.m_pad, p.k_pad, x16, row_inv, stream);
    hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) return rc;
    const size_t w_bytes = type == 1 ? static_cast<size_t>(n) * k * 2 : static_cast<size_t>(n) * (k / 32) * 18;
    if (route) *route = type == 2 ? "q4_gemm_swiglu_mfma" : "f16_gemm_swiglu_mfma";
    if (type == 2 && ql_shape(k, w_gate, w_up))
        return launch_ql<true>(w_gate, w_up, x16, row_inv, y, batch, n, k, p.k_pad, stream);
    if (type == 2) return launch_gemm<false, 128, true>(w_gate, w_up, x16, row_inv, y, batch, n, k, p, w_bytes, stream);
    return launch_gemm<true, 128, true>(w_gate, w_up, x16, row_inv, y, batch, n, k, p, w_bytes, stream);
}
