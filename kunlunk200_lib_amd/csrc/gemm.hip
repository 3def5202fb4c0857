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

#include <algorithm>
#include <cstdlib>

namespace {

using kk::kWave;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
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
// Prepass: one workgroup per padded row.
template <bool PERMUTE>
__global__ __launch_bounds__(kPrepassThreads) void x_to_f16(const float *__restrict__ x, int m_rows, int k,
                                                           int k_pad, _Float16 *__restrict__ x16,
                                                           float *__restrict__ row_inv) {
    __shared__ float scratch[kPrepassThreads / kWave];
    const int row = blockIdx.x;
    const int groups = k >> 3;                       // 8 values per group
    constexpr int kMaxGroupsPerThread = 16384 / 8 / kPrepassThreads;
    float v[kMaxGroupsPerThread][8];
    float m = 0.0f;
    const bool real = row < m_rows;
#pragma unroll
    for (int g = 0; g < kMaxGroupsPerThread; ++g) {
        const int grp = g * kPrepassThreads + threadIdx.x;
        if (real && grp < groups) {
            const int blk = grp >> 2, i = grp & 3;
            const float *src = x + static_cast<size_t>(row) * k + blk * 32;
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
        } else {
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
    for (int g = 0; g < kMaxGroupsPerThread; ++g) {
        const int grp = g * kPrepassThreads + threadIdx.x;
        if (grp < (k_pad >> 3)) {
            half8 h;
#pragma unroll
            for (int t = 0; t < 8; ++t) h[t] = static_cast<_Float16>(v[g][t] * s);
            *reinterpret_cast<half8 *>(dst + grp * 8) = h;
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_0: half a block (nibble dwords 2*half, 2*half+1 -> 16 values) to fp16
// (q - 8) * d / 8 in block order; e = the 18 block bytes as 5 dwords.
__device__ __forceinline__ void decode_q4_half(const uint32_t (&e)[5], int half, bool live, half8 (&out)[2]) {
    union { uint16_t u; _Float16 h; } du;
    du.u = static_cast<uint16_t>(e[0] & 0xffffu);
    const _Float16 d8 = live ? static_cast<_Float16>(du.h * static_cast<_Float16>(0.125f)) : static_cast<_Float16>(0.0f);
    const half2v dd = {d8, d8};
    const half2v off_lo = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    const half2v off_hi = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t lo = half ? e[2 + j] : e[j], hi = half ? e[3 + j] : e[1 + j];
        const uint32_t n = kk::align_bytes(hi, lo, 2);   // nibble bytes 4i .. 4i+3, i = 2*half + j
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
        out[j] = o;
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
                decode_q4_half(e, 0, live_reg[set], lo);
                decode_q4_half(e, 1, live_reg[set], hi);
                bd[0] = lo[0]; bd[1] = lo[1]; bd[2] = hi[0]; bd[3] = hi[1];
            } else {
                half8 out[2];
                decode_q4_half(e, qb_half, live_reg[set], out);
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
    __syncthreads();
    if (kh == 1) return;
    const float wscale = F16W ? 1.0f : 8.0f;
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

struct GemmPlan {
    int m_pad, k_pad, m_tiles, bn, n_tiles;
    size_t x16_bytes, row_inv_bytes;
};

// Tile N: 128 (fewer LDS reads per MFMA) when that still gives every CU a
// tile, else 64. KUNLUN_GEMM_BN=64|128 overrides.
GemmPlan plan(int k, int n, int batch) {
    GemmPlan p;
    p.m_pad = static_cast<int>(round_up(static_cast<size_t>(batch), kBM));
    p.k_pad = static_cast<int>(round_up(static_cast<size_t>(k), kKAlign));
    p.m_tiles = p.m_pad / kBM;
    const char *forced = std::getenv("KUNLUN_GEMM_BN");
    const int want = forced && *forced ? std::atoi(forced) : 0;
    p.bn = want == 64 || want == 128 ? want : (p.m_tiles * ((n + 127) / 128) >= 256 ? 128 : 64);
    p.n_tiles = (n + p.bn - 1) / p.bn;
    p.x16_bytes = round_up(static_cast<size_t>(p.m_pad) * p.k_pad * 2, 256);
    p.row_inv_bytes = round_up(static_cast<size_t>(p.m_pad) * 4, 256);
    return p;
}

template <bool F16W, int BN, bool PAIR = false>
hipError_t launch_gemm(const void *w, const void *w2, const _Float16 *x16, const float *row_inv, float *y, int batch,
                       int n, int k, const GemmPlan &p, size_t w_bytes, hipStream_t stream) {
    // dynamic LDS above 64 KiB is opted into once per device (callers hold the runtime lock)
    constexpr int kMaxDevices = 64;
    static bool configured[kMaxDevices] = {};
    int device = 0;
    hipError_t rc = hipGetDevice(&device);
    if (rc != hipSuccess) return rc;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    if (!configured[device]) {
        rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&mfma_gemm<F16W, BN, PAIR>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(gemm_lds_bytes<BN>()));
        if (rc != hipSuccess) return rc;
        configured[device] = true;
    }
    const int tiles = p.m_tiles * p.n_tiles;
    const int tiles_per_xcd = (tiles + kXcds - 1) / kXcds;
    hipLaunchKernelGGL((mfma_gemm<F16W, BN, PAIR>), dim3(tiles_per_xcd * kXcds), dim3(kGemmThreads),
                       gemm_lds_bytes<BN>(), stream, static_cast<const uint8_t *>(w), static_cast<const uint8_t *>(w2),
                       x16, row_inv, y, batch, n, k, p.k_pad, w_bytes, p.n_tiles, tiles, tiles_per_xcd);
    return hipGetLastError();
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
    if (type == 2)
        hipLaunchKernelGGL(x_to_f16<true>, dim3(p.m_pad), dim3(kPrepassThreads), 0, stream, x, batch, k, p.k_pad, x16,
                           row_inv);
    else
        hipLaunchKernelGGL(x_to_f16<false>, dim3(p.m_pad), dim3(kPrepassThreads), 0, stream, x, batch, k, p.k_pad, x16,
                           row_inv);
    hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) return rc;
    const size_t w_bytes = type == 1 ? static_cast<size_t>(n) * k * 2 : static_cast<size_t>(n) * (k / 32) * 18;
    if (route) *route = type == 2 ? "q4_gemm_mfma" : "f16_gemm_mfma";
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
    if (type == 2)
        hipLaunchKernelGGL(x_to_f16<true>, dim3(p.m_pad), dim3(kPrepassThreads), 0, stream, x, batch, k, p.k_pad, x16,
                           row_inv);
    else
        hipLaunchKernelGGL(x_to_f16<false>, dim3(p.m_pad), dim3(kPrepassThreads), 0, stream, x, batch, k, p.k_pad, x16,
                           row_inv);
    hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) return rc;
    const size_t w_bytes = type == 1 ? static_cast<size_t>(n) * k * 2 : static_cast<size_t>(n) * (k / 32) * 18;
    if (route) *route = type == 2 ? "q4_gemm_swiglu_mfma" : "f16_gemm_swiglu_mfma";
    if (type == 2) return launch_gemm<false, 128, true>(w_gate, w_up, x16, row_inv, y, batch, n, k, p, w_bytes, stream);
    return launch_gemm<true, 128, true>(w_gate, w_up, x16, row_inv, y, batch, n, k, p, w_bytes, stream);
}
