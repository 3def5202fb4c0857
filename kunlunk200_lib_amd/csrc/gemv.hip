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
//   q4_gemv_dot8  Q4_0, K % 64 == 0, 4-byte aligned rows: exact integer block
//                 sums of nibbles and fixed-point activation digits (v_dot8).
//   dense_stream  F32 / F16, one batch column, 16-byte aligned rows: every
//                 load instruction is 1 KiB of one row, 4 in flight per wave.
//   dense_gemv    F32 / F16, 2..4 batch columns per pass, 16-byte aligned
//                 rows. A lane owns 16-byte chunks spaced 1 KiB apart so every
//                 load instruction is coalesced.
//   gemv_general  any format, alignment and K % 32: byte loads, one wave per
//                 row. Correct for every input the API accepts; slow.
#include "device_common.h"
#include "launch.h"
#include "lds_opt_in.h"
#include "tuning.h"

#include <algorithm>
#include <cstdlib>

namespace {

using kk::kWave;

constexpr int kThreads = 256;          // 4 waves per workgroup
constexpr int kWavesPerGroup = kThreads / kWave;

// ---------------------------------------------------------------------------
// Q4_0 with integer block dot products (v_dot8_i32_i4).
//
// Each 32-value activation block is represented as X_j = rint(x_j * 2^(F-e)),
// where 2^e > max|x| of the block (frexp exponent) and F = 4 * DIGITS - 2,
// i.e. an (F+1)-bit signed fixed-point value with block scale s = 2^(e-F);
// |x_j - s X_j| <= s/2 <= max|x| * 2^-F. X_j is written in DIGITS balanced
// base-16 digits in [-8, 7] (kk::fixed_point_digits). A weight nibble q
// becomes the signed value q - 8 by q ^ 8. Then
//   S = sum_j (q_j - 8) X_j = sum_l 16^l sum_j (q_j - 8) digit_l(X_j)
// is computed exactly in int32 (|S| <= 32*8*2^F <= 2^30) with 4 * DIGITS
// v_dot8 (8 products each) per block and row, accumulated from the top digit
// down (Horner), and y += float(S) * (d * s).
// Error: per element |e_j| <= m_b 2^-F with m_b the block's max |x| (2^(e-1)
// <= m_b), so |sum_j w_j e_j| <= ||w|| ||e|| <= 2^-F sqrt(32) ||x|| ||w||:
// 2.2e-5 ||x|| ||w|| for DIGITS = 5 (F = 18), 1.4e-6 for DIGITS = 6 (F = 22),
// inside the 1e-4 ||x|| ||w|| bound of the F32-accumulate GEMV either way.
//
// Digit dwords are packed in the weight nibble order: dword i of a block's 16
// nibble bytes holds values (4i, 16+4i, 4i+1, 16+4i+1, ..., 4i+3, 16+4i+3) in
// nibbles 0..7, so digit dword D[i][l] holds digit l of the same values.
// LDS layout per batch column b and block half h of pair p: DIGITS uint4
// groups of the 4 * DIGITS dwords (i * DIGITS + l), stored [b][h][group][p]
// (lanes read consecutive uint4: conflict-free), then the block scales
// [b][h][p]. A non-finite activation makes its block scale NaN: every output
// row of that batch column becomes NaN.
// Every global load is branch-free (clamped addresses, inactive lanes zero
// their block scale) and the loop issues no vector stores (row results are
// parked in LDS and written once, coalesced, at the end), so the waitcnt
// counters stay exact. A wave issues its first DEPTH items at entry; when it
// owns at most DEPTH items, all of its weight bytes are requested before its
// first wait and no refill loads follow. Otherwise a ring refills a slot with
// item i + DEPTH: after item i is decoded, or (EARLY, DEPTH + 1 slots) before
// item i is waited for, into the slot item i - 1 used, so a refill does not
// wait for a decode. All activation loads are issued before the first weight
// items (the memory counter is in order), then converted while those weights
// are in flight.
constexpr int kDot8MaxRowsPerWave = 64;

constexpr int dot8_block_lds_bytes(int digits) { return 16 * digits + 4; }

// PASSES = activation staging passes: B * (K/32) * 4 <= PASSES * 64 * WAVES.
// SLICES = ceil(K / 4096): 64-pair slices per row. Rows are split over the
// grid's waves as base or base+1 contiguous rows (rem waves get one more),
// or, STRIDED, wave w of the grid's nw waves takes rows w, w + nw, w + 2 nw,
// ...: then the i-th items of all waves are consecutive rows, so the grid
// streams the matrix front to back (at N11008 and N32000 5-9% faster than
// contiguous ranges whenever a wave's rows do not all fit in its ring).
// PAIR (U = 2): an item is output row r of both the gate matrix w and the up
// matrix w2, and the row result is SiLU(gate) * up (the swiglu kernel's
// element function), so the pair reads X once and needs no second pass.
template <int B, int U, int WAVES, int SLICES, int DEPTH, int PASSES, bool PAIR, int DIGITS, bool STRIDED,
          bool EARLY = false>
__global__ __launch_bounds__(64 * WAVES) void q4_gemv_dot8(const uint8_t *__restrict__ w,
                                                          const uint8_t *__restrict__ w2,
                                                          const float *__restrict__ x,
                                                          float *__restrict__ y, int k, int n, int y_stride,
                                                          int rows_base, int rows_rem) {
    extern __shared__ uint4 lds4[];
    constexpr int kGroupThreads = 64 * WAVES;
    constexpr bool ONE_SLICE = SLICES == 1;
    constexpr int kFrac = 4 * DIGITS - 2;
    const int blocks = k >> 5;
    const int pairs = blocks >> 1;
    constexpr int slices = SLICES;
    const size_t row_bytes = static_cast<size_t>(blocks) * 18;
    uint4 *digits = lds4;                                                                        // [B][2][DIGITS][pairs]
    float *scales = reinterpret_cast<float *>(lds4 + static_cast<size_t>(B) * 2 * DIGITS * pairs);  // [B][2][pairs]
    float *results = scales + static_cast<size_t>(B) * 2 * pairs;                                // [WAVES][B][64]

    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int wave = blockIdx.x * WAVES + wid;
    const int nwaves = gridDim.x * WAVES;
    const int r_begin = STRIDED ? wave : wave * rows_base + min(wave, rows_rem);
    const int rows = STRIDED ? (wave < n ? (n - 1 - wave) / nwaves + 1 : 0)
                             : rows_base + (wave < rows_rem ? 1 : 0);   // 0 <= rows <= kDot8MaxRowsPerWave
    const int row_step = STRIDED ? nwaves : 1;
    static_assert(!PAIR || U == 2, "a pair item is one gate row and one up row");
    const int chunks = PAIR ? rows : (rows + U - 1) / U;
    const int items = chunks * slices;
    float *my_results = results + wid * B * kDot8MaxRowsPerWave;

    // Weight loads go through buffer resources over the whole matrix (at most
    // INT_MAX bytes): an item past the wave's last one (the ring's trailing
    // refills, unused slots) is read at an offset past the resource's extent,
    // which returns zeros without a memory access, so the final wait for the
    // refills costs no round trip.
    const uint32_t extent = static_cast<uint32_t>(static_cast<size_t>(n) * row_bytes);
    const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), 0, extent, 0x00020000);
    const __amdgpu_buffer_rsrc_t w2_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(PAIR ? w2 : w), 0, extent, 0x00020000);
    constexpr uint32_t kPastExtent = 0x80000000u;
    auto load_item = [&](int item, uint32_t (&buf)[U][9]) {
        const bool past = item >= items;                       // wave-uniform
        const int it = max(0, min(item, items - 1));
        const int c = ONE_SLICE ? it : it / slices;
        const int j = ONE_SLICE ? 0 : it - c * slices;
        const int p = min(lane + kWave * j, pairs - 1);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int ordinal = max(0, min(PAIR ? c : c * U + u, rows - 1));
            const int r = min(r_begin + ordinal * row_step, n - 1);
            const uint32_t off = past ? kPastExtent : static_cast<uint32_t>(r) * static_cast<uint32_t>(row_bytes) +
                                                          static_cast<uint32_t>(p) * 36u;
            const __amdgpu_buffer_rsrc_t rs = PAIR && u == 1 ? w2_rsrc : w_rsrc;
            typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
            const u32x4v a = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off), 0, 0));
            const u32x4v b = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off + 16), 0, 0));
            buf[u][0] = a[0]; buf[u][1] = a[1]; buf[u][2] = a[2]; buf[u][3] = a[3];
            buf[u][4] = b[0]; buf[u][5] = b[1]; buf[u][6] = b[2]; buf[u][7] = b[3];
            buf[u][8] = __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(off + 32), 0, 0);
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
    constexpr int kSlots = EARLY ? DEPTH + 1 : DEPTH;
    uint32_t ring[kSlots][U][9];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        load_item(d, ring[d]);
        __builtin_amdgcn_sched_barrier(0);   // item d's loads are issued before item d+1's
    }
    // 3. activations -> block scale and DIGITS signed base-16 digit dwords
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
        // 2^(F-e) stays finite (blocks below 2^-100 lose relative precision only).
        const int e = max(__builtin_amdgcn_frexp_expf(m), -100);
        uint32_t dig[DIGITS];
        kk::fixed_point_digits<DIGITS>(v, ldexpf(1.0f, kFrac - e), dig);
        if (idx < groups) {
            const int b = (B > 1 && idx >= blocks * 4) ? 1 : 0;
            const int rem = idx - b * blocks * 4;
            const int blk = rem >> 2, i = rem & 3;
            const int p = blk >> 1, h = blk & 1;
            uint32_t *dst = reinterpret_cast<uint32_t *>(digits);
#pragma unroll
            for (int l = 0; l < DIGITS; ++l) {
                const int pos = i * DIGITS + l;
                dst[((static_cast<size_t>(b * 2 + h) * DIGITS + (pos >> 2)) * pairs + p) * 4 + (pos & 3)] = dig[l];
            }
            if (i == 0)
                scales[(b * 2 + h) * pairs + p] = bad != 0.0f ? __builtin_nanf("") : ldexpf(1.0f, e - kFrac);
        }
    }
    __syncthreads();

    // 4. decode: one item = U rows x one 64-pair slice
    float acc[U][B];
    uint4 dg[B][2][DIGITS];
    float sc[B][2];
    auto read_slice = [&](int p) {
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int g = 0; g < DIGITS; ++g)
                    dg[b][h][g] = digits[(static_cast<size_t>(b * 2 + h) * DIGITS + g) * pairs + p];
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
                    uint32_t dd[4 * DIGITS];
#pragma unroll
                    for (int g = 0; g < DIGITS; ++g) {
                        dd[4 * g + 0] = dg[b][h][g].x;
                        dd[4 * g + 1] = dg[b][h][g].y;
                        dd[4 * g + 2] = dg[b][h][g].z;
                        dd[4 * g + 3] = dg[b][h][g].w;
                    }
                    // DIGITS independent digit sums T_l, then S = sum_l 16^l T_l (|S| <= 2^30)
                    int t[DIGITS];
#pragma unroll
                    for (int l = 0; l < DIGITS; ++l) {
                        t[l] = 0;
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            t[l] = __builtin_amdgcn_sdot8(static_cast<int>(q[i]), static_cast<int>(dd[i * DIGITS + l]),
                                                          t[l], false);
                    }
                    int s = t[DIGITS - 1];
#pragma unroll
                    for (int l = DIGITS - 2; l >= 0; --l) s = (s << 4) + t[l];
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

    if (EARLY && items > DEPTH) {
        // DEPTH + 1 slots: before item i is waited for, item i + DEPTH goes out
        // into the slot item i - 1 used, so the refill does not wait for the
        // decode of item i
        for (int base = 0; base < items; base += kSlots) {
#pragma unroll
            for (int d = 0; d < kSlots; ++d) {
                const int item = base + d;
                load_item(item + DEPTH, ring[(d + DEPTH) % kSlots]);
                __builtin_amdgcn_sched_barrier(0);
                if (item < items) compute_item(item, ring[d]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
    } else if (items <= DEPTH) {
        // every item is already in flight: consume them in issue order. Items
        // past the wave's own (clamped loads of its last item) are computed
        // too and their results dropped (no row below `rows`), so the path has
        // no branch and each item waits only for its own loads.
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) compute_item(d, ring[d]);
    } else {
        // ring of DEPTH items in flight: after item i is decoded its buffer is
        // refilled with item i + DEPTH (clamped: past the end it re-reads the
        // last item, which hits in cache)
        for (int base = 0; base < items; base += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                const int item = base + d;
                if (item < items) compute_item(item, ring[d]);
                load_item(item + DEPTH, ring[d]);
            }
        }
        // the ring's last refills (clamped re-reads) end here, so that where
        // this path joins the other the compiler's memory-counter waits of the
        // other path stay exact
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
    }

    // 5. row results: one coalesced store per batch column
    __builtin_amdgcn_s_waitcnt(0xc07f);    // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int b = 0; b < B; ++b)
        if (lane < rows)
            y[static_cast<size_t>(b) * y_stride + r_begin + lane * row_step] = my_results[b * kDot8MaxRowsPerWave + lane];
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
// F32 / F16 rows, one batch column, streamed: an item is one 1 KiB chunk of
// one row (lane l holds bytes 16 l .. 16 l + 15 of it), so every load
// instruction reads 1 KiB of contiguous row bytes; each wave keeps DEPTH
// items in flight and refills a slot as soon as it has used it. Wave w of
// the grid's nw waves owns rows w, w + nw, ... (the i-th rows of all waves
// are consecutive), at most kDot8MaxRowsPerWave of them. X is staged in LDS
// (F32) once per workgroup; the row sums are parked in LDS and stored once
// at the end, so the loop issues no vector stores and the memory-counter
// waits stay exact. A chunk's lanes past the row end read the row's last
// 16 bytes and use weight 0 (not their value: 0 * Inf would be NaN).
// Row results are exact F32 products (an F16 weight widens exactly) summed
// in F32, in a fixed order.
template <bool F16, int WAVES, int DEPTH, int XPASSES, bool EARLY = false>
__global__ __launch_bounds__(64 * WAVES) void dense_stream(const uint8_t *__restrict__ w,
                                                          const float *__restrict__ x, float *__restrict__ y,
                                                          int k, int n) {
    extern __shared__ float4 ds_lds[];
    constexpr int kPer = F16 ? 8 : 4;                  // values per lane and chunk
    constexpr int kChunkValues = kPer * kWave;
    const int k4 = k >> 2;
    float *results = reinterpret_cast<float *>(ds_lds + k4);   // [WAVES][64]
    const int chunks = (k + kChunkValues - 1) / kChunkValues;
    const uint32_t row_bytes = static_cast<uint32_t>(k) * (F16 ? 2 : 4);
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int wave = blockIdx.x * WAVES + wid;
    const int nwaves = gridDim.x * WAVES;
    const int rows = wave < n ? (n - 1 - wave) / nwaves + 1 : 0;   // <= kDot8MaxRowsPerWave
    const int items = rows * chunks;
    float *my_results = results + wid * kDot8MaxRowsPerWave;

    // X loads first (the memory counter is in order), then the first items;
    // XPASSES * 64 * WAVES >= K / 4 float4 (checked by the launcher)
    float4 xv[XPASSES];
    constexpr int xthreads = 64 * WAVES;
#pragma unroll
    for (int p = 0; p < XPASSES; ++p) {
        const int i = min(p * xthreads + static_cast<int>(threadIdx.x), k4 - 1);
        xv[p] = reinterpret_cast<const float4 *>(x)[i];
    }
    __builtin_amdgcn_sched_barrier(0);
    auto load_item = [&](int item, uint4 &v) {
        const int it = max(0, min(item, items - 1));
        const int ord = it / chunks, c = it - ord * chunks;
        const int r = min(wave + ord * nwaves, n - 1);
        const uint32_t off = min(static_cast<uint32_t>(c) * 1024u + 16u * lane, row_bytes - 16u);
        typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
        const u32x4v t = __builtin_nontemporal_load(reinterpret_cast<const u32x4v *>(w + static_cast<size_t>(r) * row_bytes + off));
        v = make_uint4(t[0], t[1], t[2], t[3]);
    };
    constexpr int kSlots = EARLY ? DEPTH + 1 : DEPTH;
    uint4 ring[kSlots];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        load_item(d, ring[d]);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int p = 0; p < XPASSES; ++p) {
        const int i = p * xthreads + static_cast<int>(threadIdx.x);
        if (i < k4) ds_lds[i] = xv[p];
    }
    kk::lds_barrier();

    float acc = 0.0f;
    auto compute_item = [&](int item, const uint4 &v) {
        const int ord = item / chunks, c = item - ord * chunks;
        const int k0 = c * kChunkValues + lane * kPer;
        const bool live = k0 < k;
        const int xi = (live ? k0 : 0) >> 2;
        const uint32_t words[4] = {v.x, v.y, v.z, v.w};
        if (F16) {
            const float4 x0 = ds_lds[xi], x1 = ds_lds[xi + 1];
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float w0 = live ? kk::half_bits_to_float(words[i] & 0xffffu) : 0.0f;
                const float w1 = live ? kk::half_bits_to_float(words[i] >> 16) : 0.0f;
                acc = fmaf(w0, xs[2 * i], acc);
                acc = fmaf(w1, xs[2 * i + 1], acc);
            }
        } else {
            const float4 x0 = ds_lds[xi];
            const float xs[4] = {x0.x, x0.y, x0.z, x0.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) acc = fmaf(live ? __uint_as_float(words[i]) : 0.0f, xs[i], acc);
        }
        if (c == chunks - 1) {
            const float sum = kk::wave_sum_uniform(acc);
            if (lane == 0 && ord < rows) my_results[ord] = sum;
            acc = 0.0f;
        }
    };
    if (EARLY && items > DEPTH) {
        // item i + DEPTH goes out into the slot item i - 1 used before item i
        // is waited for
        for (int base = 0; base < items; base += kSlots) {
#pragma unroll
            for (int d = 0; d < kSlots; ++d) {
                const int item = base + d;
                load_item(item + DEPTH, ring[(d + DEPTH) % kSlots]);
                __builtin_amdgcn_sched_barrier(0);
                if (item < items) compute_item(item, ring[d]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): the clamped refills end here
    } else if (items <= DEPTH) {
        // every item is in flight: all slots computed without a branch (slots
        // past the last item re-read it and store nothing)
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) compute_item(d, ring[d]);
    } else {
        for (int base = 0; base < items; base += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                const int item = base + d;
                if (item < items) compute_item(item, ring[d]);
                load_item(item + DEPTH, ring[d]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): the clamped refills end here
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);       // lgkmcnt(0): this wave's LDS writes are done
    __builtin_amdgcn_wave_barrier();
    if (lane < rows) y[wave + lane * nwaves] = my_results[lane];
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


// Workgroup count for a row-blocked kernel: enough waves for every row block
// up to `per_cu` waves per CU.
int groups_for(int rowblocks, int cus, int per_cu_waves) {
    const long long cap = static_cast<long long>(cus) * per_cu_waves;
    const long long waves = std::min<long long>(rowblocks, cap);
    return static_cast<int>(std::max<long long>(1, (waves + kWavesPerGroup - 1) / kWavesPerGroup));
}

// One launch of q4_gemv_dot8 with WAVES waves per workgroup and up to
// `per_cu` waves per CU (fewer when a wave would own no row).
template <int B, int SLICES, int DEPTH, bool PAIR, int DIGITS, int WAVES, bool STRIDED = false, bool EARLY = false>
hipError_t launch_q4_dot8_cfg(const uint8_t *w, const uint8_t *w2, const float *x, float *y, int k, int n,
                              int y_stride, hipStream_t stream, const DeviceInfo &info, int per_cu) {
    constexpr int kU = PAIR ? 2 : 1;
    constexpr int kPasses = (B * SLICES * 8 + WAVES - 1) / WAVES;   // B * K/8 staging groups <= B * SLICES * 512
    const size_t lds = static_cast<size_t>(B) * (k / 32) * dot8_block_lds_bytes(DIGITS) +
                       static_cast<size_t>(WAVES) * B * kDot8MaxRowsPerWave * 4;
    long long want = std::min<long long>(n, static_cast<long long>(info.cus) * per_cu);
    want = std::max<long long>(want, (n + kDot8MaxRowsPerWave - 1) / kDot8MaxRowsPerWave);
    const int groups = static_cast<int>(std::max<long long>(1, (want + WAVES - 1) / WAVES));
    const int waves = groups * WAVES;
    const int rows_base = n / waves, rows_rem = n % waves;
    if (rows_base + (rows_rem ? 1 : 0) > kDot8MaxRowsPerWave) return hipErrorInvalidValue;
    auto kernel = &q4_gemv_dot8<B, kU, WAVES, SLICES, DEPTH, kPasses, PAIR, DIGITS, STRIDED, EARLY>;
    // B * K <= 16384: at most 512 * 100 + 16 * 2 * 64 * 4 bytes, inside the 64 KiB default
    hipLaunchKernelGGL(kernel, dim3(groups), dim3(64 * WAVES), lds, stream, w, w2, x, y, k, n, y_stride, rows_base,
                       rows_rem);
    return hipGetLastError();
}

// Six activation digits (F = 22). Five (F = 18) meet the 1e-4 ||x|| ||w||
// bound and run 5-8% faster, but miss the reference's own 1e-3 (1 + |gold|)
// tolerance on its large-magnitude fixture activations (pattern 4), which
// the F32-exact reference kernel meets.
template <int B, int SLICES, int DEPTH, bool PAIR = false>
hipError_t launch_q4_dot8_depth(const uint8_t *w, const uint8_t *w2, const float *x, float *y, int k, int n,
                                int y_stride, hipStream_t stream, const DeviceInfo &info) {
    return launch_q4_dot8_cfg<B, SLICES, DEPTH, PAIR, 6, 8, false, true>(w, w2, x, y, k, n, y_stride, stream, info, 8);
}

template <int B, int SLICES, bool PAIR>
hipError_t launch_q4_dot8_slices(const uint8_t *w, const uint8_t *w2, const float *x, float *y, int k, int n,
                                 int y_stride, hipStream_t stream, const DeviceInfo &info) {
    if constexpr (B == 1 && !PAIR) {
        // single column. K <= 4096: 4 waves per CU, each with all of its rows
        // in flight when they fit a 4-item ring (contiguous ranges), else a
        // 3-item ring over strided rows (K4096: N4096 3.9 against 4.8 us with
        // 8 waves per CU, N11008 6.9 against 7.3 us, N32000 13.6 against
        // 14.9 us, before the early refill). Longer rows: 8 waves per CU over
        // strided rows (K11008 x N4096: 7.9 against 8.5 us).
        if (SLICES == 1) {
            const long long waves = std::max<long long>(1, std::min<long long>(n, static_cast<long long>(info.cus) * 4));
            if ((n + waves - 1) / waves <= 4)
                return launch_q4_dot8_cfg<1, 1, 4, false, 6, 4>(w, w2, x, y, k, n, y_stride, stream, info, 4);
            // the ring's refill goes out before each item is waited for
            // (alternating runs, one box: N11008 6.55-6.66 against 6.99-7.02
            // us, N32000 13.25 against 13.9-14.3 us)
            return launch_q4_dot8_cfg<1, 1, 3, false, 6, 4, true, true>(w, w2, x, y, k, n, y_stride, stream, info, 4);
        }
        // 2 slices in flight with the early refill (K11008 x N4096: 7.59 us
        // against 7.80-7.83 us for 3 refilled after each decode, 8.0 for 3
        // with the early refill, 8.55 for 4, 9.3-10.0 with all 6 in flight)
        const long long waves = std::max<long long>(1, std::min<long long>(n, static_cast<long long>(info.cus) * 8));
        if ((n + waves - 1) / waves * SLICES <= 2)
            return launch_q4_dot8_cfg<1, SLICES, 2, false, 6, 8>(w, w2, x, y, k, n, y_stride, stream, info, 8);
        return launch_q4_dot8_cfg<1, SLICES, 2, false, 6, 8, true, true>(w, w2, x, y, k, n, y_stride, stream, info, 8);
    }
    if constexpr (B == 1 && PAIR && SLICES == 1) {
        // gate/up pair, K <= 4096: 4 waves per CU over strided rows, 2 row
        // pairs in flight (K4096 x 2 x N11008: 12.0 against 12.7 us with 8
        // waves per CU and contiguous rows; 12.4 us with 3 in flight)
        // (early refill: 11.1-11.2 against 12.0 us)
        return launch_q4_dot8_cfg<1, 1, 2, true, 6, 4, true, true>(w, w2, x, y, k, n, y_stride, stream, info, 4);
    }
    // items in flight per wave: 3 single-column items, 2 when an item is twice
    // the work (two batch columns, or a gate/up row pair) or when a wave owns
    // at most 2 items (then all of them are in flight and a third would be a
    // wasted re-read: 4.48 vs 4.9 us at K4096 x N4096). 8 waves per CU.
    const long long waves = std::max<long long>(1, std::min<long long>(n, static_cast<long long>(info.cus) * 8));
    const long long items = (n + waves - 1) / waves * SLICES;
    if (B == 2 || PAIR || items <= 2)
        return launch_q4_dot8_depth<B, SLICES, 2, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
    return launch_q4_dot8_depth<B, SLICES, 3, PAIR>(w, w2, x, y, k, n, y_stride, stream, info);
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
    const int groups = groups_for(rowblocks, info.cus, 8);
    const hipError_t rc = kk::opt_in_lds(reinterpret_cast<const void *>(&dense_gemv<B, U, F16>), lds);
    if (rc != hipSuccess) return rc;
    hipLaunchKernelGGL((dense_gemv<B, U, F16>), dim3(groups), dim3(kThreads), lds, stream, w, x, y, k, n, y_stride);
    return hipGetLastError();
}

// One launch of dense_stream with WAVES waves per workgroup, about per_cu
// waves per CU (more when a wave would own more than kDot8MaxRowsPerWave rows).
template <bool F16, int WAVES, int DEPTH, int XPASSES, bool EARLY = false>
hipError_t launch_dense_stream_passes(const uint8_t *w, const float *x, float *y, int k, int n, hipStream_t stream,
                                      const DeviceInfo &info, int per_cu) {
    if (static_cast<long long>(XPASSES) * 64 * WAVES * 4 < k) return hipErrorInvalidValue;
    long long waves = std::min<long long>(n, static_cast<long long>(info.cus) * per_cu);
    waves = std::max<long long>(waves, (n + kDot8MaxRowsPerWave - 1) / kDot8MaxRowsPerWave);
    const int groups = static_cast<int>((waves + WAVES - 1) / WAVES);
    const size_t lds = static_cast<size_t>(k) * 4 + static_cast<size_t>(WAVES) * kDot8MaxRowsPerWave * 4;
    auto kernel = &dense_stream<F16, WAVES, DEPTH, XPASSES, EARLY>;
    // opted into the whole LDS once per device and kernel, so a later call
    // with a larger K on the same instance stays inside the grant
    const hipError_t rc = kk::opt_in_lds(reinterpret_cast<const void *>(kernel), lds);
    if (rc != hipSuccess) return rc;
    hipLaunchKernelGGL(kernel, dim3(groups), dim3(64 * WAVES), lds, stream, w, x, y, k, n);
    return hipGetLastError();
}

// dense_stream with the fewest X staging passes that cover K (K <= 16384).
template <bool F16, int WAVES, int DEPTH, bool EARLY = false>
hipError_t launch_dense_stream(const uint8_t *w, const float *x, float *y, int k, int n, hipStream_t stream,
                               const DeviceInfo &info, int per_cu) {
    const int passes = (k / 4 + 64 * WAVES - 1) / (64 * WAVES);
    if (passes <= 1) return launch_dense_stream_passes<F16, WAVES, DEPTH, 1, EARLY>(w, x, y, k, n, stream, info, per_cu);
    if (passes <= 2) return launch_dense_stream_passes<F16, WAVES, DEPTH, 2, EARLY>(w, x, y, k, n, stream, info, per_cu);
    if (passes <= 4) return launch_dense_stream_passes<F16, WAVES, DEPTH, 4, EARLY>(w, x, y, k, n, stream, info, per_cu);
    if (passes <= 8) return launch_dense_stream_passes<F16, WAVES, DEPTH, 8, EARLY>(w, x, y, k, n, stream, info, per_cu);
    if (passes <= 16) return launch_dense_stream_passes<F16, WAVES, DEPTH, 16, EARLY>(w, x, y, k, n, stream, info, per_cu);
    return hipErrorInvalidValue;
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
    const bool force_general = kk::tuning_or(kk::kGemvGeneral, 0) != 0;

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
    if (type == 2) {
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
    if (route) *route = type == 1 ? "f16_gemv" : "f32_gemv";
    for (int b0 = 0; b0 < batch; b0 += chunk) {
        const int bc = std::min(chunk, batch - b0);
        const float *xc = x + static_cast<size_t>(b0) * k;
        float *yc = y + static_cast<size_t>(b0) * n;
        hipError_t rc = hipSuccess;
        if (bc == 1) {
            // one column: the streamed kernel (8 waves per CU, 4 chunks in flight
            // per wave; K4096 x N4096: F16 8.9 against 11.1 us, F32 14.1 against
            // 19.0 us for dense_gemv<1>)
            // 3 chunks in flight, the refill issued before each chunk is waited
            // for (F16 8.4 against 8.85 us, F32 13.4 against 13.85 us)
            rc = type == 1 ? launch_dense_stream<true, 8, 3, true>(wb, xc, yc, k, n, stream, info, 8)
                           : launch_dense_stream<false, 8, 3, true>(wb, xc, yc, k, n, stream, info, 8);
        } else if (type == 1) {
            switch (bc) {
            case 2: rc = launch_dense<2, true>(wb, xc, yc, k, n, n, stream, info); break;
            case 3: rc = launch_dense<3, true>(wb, xc, yc, k, n, n, stream, info); break;
            default: rc = launch_dense<4, true>(wb, xc, yc, k, n, n, stream, info); break;
            }
        } else {
            switch (bc) {
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
           (reinterpret_cast<uintptr_t>(x) & 15) == 0 && kk::tuning_or(kk::kGemvGeneral, 0) == 0;
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
