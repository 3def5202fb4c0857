// Common Q4 ABI v1 kernels (reference src/q4-common.inc, src/q4-activation.inc,
// src/q4-pair.inc; persistent layout src/q4-common-pack.h:16-31) on gfx950.
//
// Weight layout (layout 1 "Micro32Bank", scale order 1 "KMajor"): for output
// column c and K32 block b the 16 bytes of signed nibble pairs (K 2p low,
// 2p + 1 high) of that column's block are contiguous at
// ((c/32) * (Kp/32) + b) * 512 + (c%16) * 32 + ((c%32)/16) * 16, so one 16-byte
// load gives a lane 32 K values of one column in natural order; the FP16
// scales are [b][Np] after the weights.
//
// Activations are quantized as the reference does (reference
// kernels/kunlun-common-{max,main,residual}-exact.xpu, quant-row-serial):
//   M = 1: per tensor, two int8 components: max0 = max|x| (1 if 0),
//          q0 = rnd(x * (127/max0)), r = x - q0 * (max0/127), q1 the same on r;
//   M > 1: per row, one component q = rnd(x * (127/max_row)).
// rnd rounds half away from zero and clamps to [-127, 127]. Products with the
// weights are exact int32 block sums (v_dot4_i32_i8 / v_mfma_i32_16x16x32_i8
// on weights widened to 16*q), then y = sum_b d_b * (S0 s0 + S1 s1) in F32.
#include "device_common.h"
#include "launch.h"

#include <algorithm>

namespace {

constexpr int kCqWaves = 8;
constexpr int kCqThreads = 64 * kCqWaves;
constexpr int kCqDepth = 4;            // GEMV items (block pairs) in flight per wave
constexpr int kQuantThreads = 1024;    // single-workgroup per-tensor quantization
constexpr int kRowThreads = 256;       // Row A8: one workgroup per row

typedef int int32x4 __attribute__((ext_vector_type(4)));

// Max of |x| bit patterns over the workgroup (NaN above Inf, as the
// reference's integer max); every thread gets the result.
template <int Threads>
__device__ uint32_t block_max_bits(uint32_t v, uint32_t *scratch) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), offset, kk::kWave)));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < Threads / 64; ++i) m = max(m, scratch[i]);
    return m;
}

// One row of X (k F16 or F32 values, the type a template parameter of the
// kernels: a runtime flag would put a branch around every load, and each
// load would be waited for before the next is issued) through a buffer
// resource whose extent is the row's bytes: value j outside [0, k) reads zero
// without a memory access, so the loads need no bounds branch either.
struct XRow {
    __amdgpu_buffer_rsrc_t rsrc;
    int k;
};
template <bool F16>
__device__ __forceinline__ XRow x_row(const void *x, size_t row, int k) {
    constexpr size_t kElem = F16 ? 2 : 4;
    const uint8_t *base = static_cast<const uint8_t *>(x) + row * static_cast<size_t>(k) * kElem;
    return {__builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, static_cast<int>(k * kElem), 0x00020000),
            k};
}
template <bool F16>
__device__ __forceinline__ float x_value(const XRow &r, int j) {
    const uint32_t jj = static_cast<uint32_t>(j) < static_cast<uint32_t>(r.k) ? static_cast<uint32_t>(j) : 0x20000000u;
    if (F16) return kk::half_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(r.rsrc, static_cast<int>(2u * jj), 0, 0));
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r.rsrc, static_cast<int>(4u * jj), 0, 0));
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (static_cast<uint32_t>(a) & 255u) | ((static_cast<uint32_t>(b) & 255u) << 8) |
           ((static_cast<uint32_t>(c) & 255u) << 16) | (static_cast<uint32_t>(d) << 24);
}

// Two-component per-tensor quantization of the values a workgroup holds
// (v[i][t] for its groups; values past k are zero): on return v holds the
// residuals' codes' inputs replaced by the codes themselves in q0/q1, and
// s[] = {max0/127, max1/127, max0, max1}. Every thread of the workgroup calls it.
template <int Threads, int Groups>
__device__ void quantize_pair(float (&v)[Groups][8], int (&q0)[Groups][8], int (&q1)[Groups][8], float (&s)[4],
                              uint32_t *scratch) {
#pragma clang fp contract(off)
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < Groups; ++i)
#pragma unroll
        for (int t = 0; t < 8; ++t) m = max(m, __float_as_uint(v[i][t]) & 0x7fffffffu);
    m = block_max_bits<Threads>(m, scratch);
    const float max0 = m ? __uint_as_float(m) : 1.0f;
    const float s0 = max0 / 127.0f, inv0 = 127.0f / max0;
    uint32_t m1 = 0;
#pragma unroll
    for (int i = 0; i < Groups; ++i)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float scaled = v[i][t] * inv0;
            q0[i][t] = kk::round_clamp(scaled, 127);
            const float back = static_cast<float>(q0[i][t]) * s0;
            v[i][t] = v[i][t] - back;                       // residual
            m1 = max(m1, __float_as_uint(v[i][t]) & 0x7fffffffu);
        }
    m1 = block_max_bits<Threads>(m1, scratch);
    const float max1 = m1 ? __uint_as_float(m1) : 1.0f;
    const float s1 = max1 / 127.0f, inv1 = 127.0f / max1;
#pragma unroll
    for (int i = 0; i < Groups; ++i)
#pragma unroll
        for (int t = 0; t < 8; ++t) q1[i][t] = kk::round_clamp(v[i][t] * inv1, 127);
    s[0] = s0;
    s[1] = s1;
    s[2] = max0;
    s[3] = max1;
}

// Writes group g's codes to the view (main at (g/4)*64 + (g%4)*8, residual
// 2kp further, the group's gap bytes zero).
__device__ __forceinline__ void write_view_group(int8_t *values, int kp, int g, const int (&a)[8], const int (&b)[8]) {
    const size_t at = static_cast<size_t>(g / 4) * 64 + (g % 4) * 8;
    uint32_t *main = reinterpret_cast<uint32_t *>(values + at);
    uint32_t *resid = reinterpret_cast<uint32_t *>(values + 2 * static_cast<size_t>(kp) + at);
    main[0] = pack4(a[0], a[1], a[2], a[3]);
    main[1] = pack4(a[4], a[5], a[6], a[7]);
    main[8] = 0;                          // bytes at + 32 .. + 40: the group's gap
    main[9] = 0;
    resid[0] = pack4(b[0], b[1], b[2], b[3]);
    resid[1] = pack4(b[4], b[5], b[6], b[7]);
    resid[8] = 0;
    resid[9] = 0;
}

__device__ __forceinline__ void write_view_tail(int8_t *values, int kp, float *params, const float (&s)[4]) {
    if (threadIdx.x < 256) reinterpret_cast<uint32_t *>(values + 4 * static_cast<size_t>(kp))[threadIdx.x] = 0;
    if (threadIdx.x < 16) params[threadIdx.x] = threadIdx.x < 4 ? s[threadIdx.x] : 0.0f;
}

// ---------------------------------------------------------------------------
// M = 1: two-component per-tensor quantization into the reference's view:
// main code of K j at values[(j/32)*64 + j%32], residual at values[2kp + ...],
// the other 32 bytes of each 64-byte group and values[4kp .. 4kp+1024) zero;
// params = {max0/127, max1/127, max0, max1, 0 ...} (16 floats).
// One workgroup; thread t owns groups of 8 values g = t + 1024 i.
template <bool F16>
__global__ __launch_bounds__(kQuantThreads) void common_quant_pair(const void *__restrict__ x, int x_f16, int k,
                                                                  int kp, int8_t *__restrict__ values,
                                                                  float *__restrict__ params) {
#pragma clang fp contract(off)
    __shared__ uint32_t scratch[kQuantThreads / 64];
    constexpr int kMaxGroups = 2;              // kp <= 16384 = 2 * 1024 * 8
    const int groups = kp / 8;
    float v[kMaxGroups][8];
    const XRow xr = x_row<F16>(x, 0, k);
#pragma unroll
    for (int i = 0; i < kMaxGroups; ++i) {
        const int g = threadIdx.x + kQuantThreads * i;
#pragma unroll
        for (int t = 0; t < 8; ++t) v[i][t] = x_value<F16>(xr, g < groups ? 8 * g + t : -1);
    }
    int q0[kMaxGroups][8], q1[kMaxGroups][8];
    float sc[4];
    quantize_pair<kQuantThreads, kMaxGroups>(v, q0, q1, sc, scratch);
#pragma unroll
    for (int i = 0; i < kMaxGroups; ++i) {
        const int g = threadIdx.x + kQuantThreads * i;
        if (g < groups) write_view_group(values, kp, g, q0[i], q1[i]);
    }
    write_view_tail(values, kp, params, sc);
}

// ---------------------------------------------------------------------------
// M > 1: Row A8. Workgroup r quantizes row r of X (rows >= `rows` are the
// zero padding rows: scale 1/127, codes 0) into values[r*kp ..] and writes the
// row scale to all 16 floats of params[r*16 ..]. The same codes also go to
// `tiled` in the GEMM's A-operand order, two blocks per lane: row r, K j at
// (((r/16) * (kp/64) + j/64) * 64 + r%16 + 16 * (j%32/8)) * 16 + (j/32 % 2) * 8 + j%8,
// so one wave reads a 16-row x 64-K operand pair as 1 KB contiguous.
__device__ __forceinline__ size_t tiled_offset(int r, int j, int blocks) {
    return ((static_cast<size_t>(r / 16) * (blocks / 2) + j / 64) * 64 + r % 16 + 16 * ((j % 32) / 8)) * 16 +
           ((j / 32) % 2) * 8 + j % 8;
}

template <bool F16>
__global__ __launch_bounds__(kRowThreads) void common_quant_rows(const void *__restrict__ x, int x_f16, int k,
                                                                int kp, int rows, int8_t *__restrict__ values,
                                                                float *__restrict__ params,
                                                                int8_t *__restrict__ tiled) {
#pragma clang fp contract(off)
    __shared__ uint32_t scratch[kRowThreads / 64];
    const int row = blockIdx.x;
    const bool real = row < rows;
    const XRow xr = x_row<F16>(x, real ? row : 0, real ? k : 0);   // a padding row reads zeros
    uint32_t m = 0;
    for (int j0 = 0; j0 < k; j0 += 8 * kRowThreads) {
        float v[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = x_value<F16>(xr, j0 + t * kRowThreads + static_cast<int>(threadIdx.x));
#pragma unroll
        for (int t = 0; t < 8; ++t) m = max(m, __float_as_uint(v[t]) & 0x7fffffffu);
    }
    m = block_max_bits<kRowThreads>(m, scratch);
    const float mx = m ? __uint_as_float(m) : 1.0f;
    const float scale = mx / 127.0f, inv = 127.0f / mx;
    // four values per thread per step, written as one dword
    uint32_t *out = reinterpret_cast<uint32_t *>(values + static_cast<size_t>(row) * kp);
    for (int d = threadIdx.x; d < kp / 4; d += kRowThreads) {
        int q[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int j = 4 * d + t;
            const float v = x_value<F16>(xr, j);
            q[t] = kk::round_clamp(v * inv, 127);
        }
        const uint32_t word = pack4(q[0], q[1], q[2], q[3]);
        out[d] = word;
        *reinterpret_cast<uint32_t *>(tiled + tiled_offset(row, 4 * d, kp / 32)) = word;
    }
    if (threadIdx.x < 16) params[row * 16 + threadIdx.x] = scale;
}

// ---------------------------------------------------------------------------
// M = 1 GEMV over one or two weights (the gate/up pair shares the
// activations). Workgroup = one N32 tile of one weight; its 8 waves take block
// pairs in turn. In an item (blocks 2i, 2i+1) lane l loads the 16 bytes of
// column 16 (c%2) + c/2 (c = l%32) of block 2i + l/32: the wave reads 1 KB
// contiguous. A8 (EXACT false): activation per block in LDS as 16 dwords
// [component][even K, odd K][4]; the weight dword w gives 16*q of the even K
// as (w << 4) & 0xf0f0f0f0 and of the odd K as w & 0xf0f0f0f0, so
// v_dot4_i32_i8 yields 16 * sum q x_q exactly. EXACT: the activations are
// 23-bit block fixed point digits (kk::fixed_point_digits) and v_dot8_i32_i4
// takes the weight dwords as they are (natural K order).
struct GemvMatrix {
    const uint8_t *w;
    float *y;
};

// MODE: kPrepared (act = the quantized view, params its scales), kQuantize
// (act = X: every workgroup quantizes X itself, workgroup 0 also writes the
// view to view_values / view_params), kExact (act = X).
constexpr int kPrepared = 0, kQuantize = 1, kExact = 2;

template <int MODE, bool F16>
__global__ __launch_bounds__(kCqThreads) void common_gemv(GemvMatrix m0, GemvMatrix m1, int tiles_per_matrix,
                                                         const void *__restrict__ act, int x_f16,
                                                         const float *__restrict__ params,
                                                         int8_t *__restrict__ view_values,
                                                         float *__restrict__ view_params, int k, int kp, int n,
                                                         int np) {
    constexpr bool EXACT = MODE == kExact;
    constexpr bool RAW_X = MODE != kPrepared;
    extern __shared__ uint4 lds4[];
    __shared__ uint32_t scratch[kCqWaves];
    const int which = blockIdx.x / tiles_per_matrix;
    const int tile = blockIdx.x - which * tiles_per_matrix;
    const GemvMatrix mat = which ? m1 : m0;
    const int blocks = kp >> 5;
    const int pairs = blocks >> 1;
    const uint16_t *scales = reinterpret_cast<const uint16_t *>(mat.w + static_cast<size_t>(np) * kp / 2);
    constexpr int kBlockWords = EXACT ? 24 : 16;
    uint32_t *act_lds = reinterpret_cast<uint32_t *>(lds4);                       // [blocks][kBlockWords]
    float *block_scale = reinterpret_cast<float *>(act_lds + static_cast<size_t>(blocks) * kBlockWords);  // EXACT
    float *partial = block_scale + (EXACT ? blocks : 0);                         // [waves][32]

    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int chunk = lane & 31;
    const int col = tile * 32 + 16 * (chunk & 1) + (chunk >> 1);
    const size_t tile_block0 = static_cast<size_t>(tile) * blocks;

    // 1. activation loads (before the weights: the memory counter is in order)
    constexpr int kMaxPasses = 4;              // kp / 8 <= 2048 groups = 4 x 512 threads
    const int groups = kp / 8;
    uint32_t raw[kMaxPasses][4];
    float xv[kMaxPasses][8];
    const XRow xr = x_row<F16>(act, 0, k);
#pragma unroll
    for (int pass = 0; pass < kMaxPasses; ++pass) {
        const int g = min(pass * kCqThreads + static_cast<int>(threadIdx.x), groups - 1);
        if (RAW_X) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                xv[pass][t] = x_value<F16>(xr, 8 * g + t);
            }
        } else {
            const int8_t *codes = static_cast<const int8_t *>(act);
            const size_t at = static_cast<size_t>(g / 4) * 64 + (g % 4) * 8;
            const uint2 a = *reinterpret_cast<const uint2 *>(codes + at);
            const uint2 b = *reinterpret_cast<const uint2 *>(codes + 2 * static_cast<size_t>(kp) + at);
            raw[pass][0] = a.x;
            raw[pass][1] = a.y;
            raw[pass][2] = b.x;
            raw[pass][3] = b.y;
        }
    }
    float s0 = 0.0f, s1 = 0.0f;
    if (MODE == kPrepared) {
        s0 = params[0] * 0.0625f;              // the weights enter as 16 * q
        s1 = params[1] * 0.0625f;
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. the first weight items
    auto load_item = [&](int s, uint32_t (&buf)[5]) {
        const int it = min(wid + kCqWaves * s, pairs - 1);
        const int blk = 2 * it + (lane >> 5);
        // 1 KB contiguous per wave, read once per call: non-temporal
        const kk::u32x4_a4 v = kk::load_u32x4_stream(
            reinterpret_cast<const uint32_t *>(mat.w + (tile_block0 + blk) * 512 + chunk * 16));
        buf[0] = v.x;
        buf[1] = v.y;
        buf[2] = v.z;
        buf[3] = v.w;
        buf[4] = scales[static_cast<size_t>(blk) * np + min(col, np - 1)];
    };
    // every wave runs the same count of items (the last ones may add zero);
    // loads are unconditional (past the end they re-read a valid item): here
    // that measures faster than skipping them with a branch
    const int iters = (pairs + kCqWaves - 1) / kCqWaves;
    const int iters_padded = (iters + kCqDepth - 1) / kCqDepth * kCqDepth;
    uint32_t ring[kCqDepth][5];
#pragma unroll
    for (int d = 0; d < kCqDepth; ++d) {
        load_item(d, ring[d]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // 3. activations -> LDS
    if (MODE == kQuantize) {
        // clamped duplicate groups hold copies of the last group: no effect on the maxima
        int q0[kMaxPasses][8], q1[kMaxPasses][8];
        float sc[4];
        quantize_pair<kCqThreads, kMaxPasses>(xv, q0, q1, sc, scratch);
        s0 = sc[0] * 0.0625f;
        s1 = sc[1] * 0.0625f;
#pragma unroll
        for (int pass = 0; pass < kMaxPasses; ++pass) {
            const int g = pass * kCqThreads + static_cast<int>(threadIdx.x);
            if (g < groups) {
                raw[pass][0] = pack4(q0[pass][0], q0[pass][1], q0[pass][2], q0[pass][3]);
                raw[pass][1] = pack4(q0[pass][4], q0[pass][5], q0[pass][6], q0[pass][7]);
                raw[pass][2] = pack4(q1[pass][0], q1[pass][1], q1[pass][2], q1[pass][3]);
                raw[pass][3] = pack4(q1[pass][4], q1[pass][5], q1[pass][6], q1[pass][7]);
                if (blockIdx.x == 0) write_view_group(view_values, kp, g, q0[pass], q1[pass]);
            }
        }
        if (blockIdx.x == 0) write_view_tail(view_values, kp, view_params, sc);
    }
#pragma unroll
    for (int pass = 0; pass < kMaxPasses; ++pass) {
        const int idx = pass * kCqThreads + static_cast<int>(threadIdx.x);
        const int g = min(idx, groups - 1);
        if (EXACT) {
            float m = 0.0f, bad = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const float a = fabsf(xv[pass][t]);
                bad = (a <= 3.402823466e38f) ? bad : 1.0f;
                m = fmaxf(m, a);
            }
            m = fmaxf(m, kk::dpp_move<0xb1>(m));        // the 4 groups of a block: one quad
            m = fmaxf(m, kk::dpp_move<0x4e>(m));
            bad = fmaxf(bad, kk::dpp_move<0xb1>(bad));
            bad = fmaxf(bad, kk::dpp_move<0x4e>(bad));
            const int e = max(__builtin_amdgcn_frexp_expf(m), -100);
            uint32_t dig[6];
            kk::fixed_point_digits(xv[pass], ldexpf(1.0f, 22 - e), dig);
            if (idx < groups) {
#pragma unroll
                for (int l = 0; l < 6; ++l) act_lds[(g / 4) * 24 + (g % 4) * 6 + l] = dig[l];
                if ((g & 3) == 0) block_scale[g / 4] = bad != 0.0f ? __builtin_nanf("") : ldexpf(1.0f, e - 22);
            }
        } else if (idx < groups) {
            // even K: bytes 0, 2 of each dword; odd K: bytes 1, 3
            uint32_t *dst = act_lds + (g / 4) * 16 + (g % 4);
            dst[0] = __builtin_amdgcn_perm(raw[pass][1], raw[pass][0], 0x06040200u);
            dst[4] = __builtin_amdgcn_perm(raw[pass][1], raw[pass][0], 0x07050301u);
            dst[8] = __builtin_amdgcn_perm(raw[pass][3], raw[pass][2], 0x06040200u);
            dst[12] = __builtin_amdgcn_perm(raw[pass][3], raw[pass][2], 0x07050301u);
        }
    }
    __syncthreads();

    // 4. items
    float acc = 0.0f;
    auto compute_item = [&](int s, const uint32_t (&buf)[5]) {
        const int it = wid + kCqWaves * s;
        const bool live = it < pairs && col < n;
        const int blk = 2 * min(it, pairs - 1) + (lane >> 5);
        const float d = live ? kk::half_bits_to_float(buf[4]) : 0.0f;
        if (EXACT) {
            const uint4 *src = reinterpret_cast<const uint4 *>(act_lds + static_cast<size_t>(blk) * 24);
            uint32_t dg[24];
#pragma unroll
            for (int g = 0; g < 6; ++g) {
                const uint4 v4 = src[g];
                dg[4 * g] = v4.x;
                dg[4 * g + 1] = v4.y;
                dg[4 * g + 2] = v4.z;
                dg[4 * g + 3] = v4.w;
            }
            int t[6];
#pragma unroll
            for (int l = 0; l < 6; ++l) {
                t[l] = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    t[l] = __builtin_amdgcn_sdot8(static_cast<int>(buf[i]), static_cast<int>(dg[i * 6 + l]), t[l], false);
            }
            int sum = t[5];
#pragma unroll
            for (int l = 4; l >= 0; --l) sum = (sum << 4) + t[l];
            acc = fmaf(static_cast<float>(sum), live ? d * block_scale[blk] : 0.0f, acc);
        } else {
            const uint4 *src = reinterpret_cast<const uint4 *>(act_lds + static_cast<size_t>(blk) * 16);
            const uint4 e0 = src[0], o0 = src[1], e1 = src[2], o1 = src[3];
            const uint32_t a0e[4] = {e0.x, e0.y, e0.z, e0.w}, a0o[4] = {o0.x, o0.y, o0.z, o0.w};
            const uint32_t a1e[4] = {e1.x, e1.y, e1.z, e1.w}, a1o[4] = {o1.x, o1.y, o1.z, o1.w};
            int p0 = 0, p1 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ev = static_cast<int>((buf[i] << 4) & 0xf0f0f0f0u);
                const int od = static_cast<int>(buf[i] & 0xf0f0f0f0u);
                p0 = __builtin_amdgcn_sdot4(ev, static_cast<int>(a0e[i]), p0, false);
                p0 = __builtin_amdgcn_sdot4(od, static_cast<int>(a0o[i]), p0, false);
                p1 = __builtin_amdgcn_sdot4(ev, static_cast<int>(a1e[i]), p1, false);
                p1 = __builtin_amdgcn_sdot4(od, static_cast<int>(a1o[i]), p1, false);
            }
            const float t = fmaf(static_cast<float>(p0), s0, static_cast<float>(p1) * s1);
            acc = fmaf(d, t, acc);
        }
    };
    for (int base = 0; base < iters_padded; base += kCqDepth) {
#pragma unroll
        for (int dpt = 0; dpt < kCqDepth; ++dpt) {
            if (base + dpt < iters) compute_item(base + dpt, ring[dpt]);   // uniform; no loads inside
            load_item(base + dpt + kCqDepth, ring[dpt]);     // past the end: a valid address
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // 5. column sums: the two block halves of the wave, then the waves in order
    acc += __shfl_xor(acc, 32, kk::kWave);
    if (lane < 32) partial[wid * 32 + chunk] = acc;
    __syncthreads();
    if (threadIdx.x < 32) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kCqWaves; ++w) v += partial[w * 32 + threadIdx.x];
        const int c = tile * 32 + 16 * (threadIdx.x & 1) + (threadIdx.x >> 1);
        if (c < n) mat.y[c] = v;
    }
}

// ---------------------------------------------------------------------------
// M > 1 GEMM on v_mfma_i32_16x16x32_i8 (one K32 block per MFMA, so each
// block's int32 sums get their own FP16 scale). A workgroup is one N32 tile x
// up to 128 rows: wave w owns rows 32w .. 32w+31 (two 16-row tiles).
//
// Data path (wide loads only; narrow per-lane loads cost one L1 tag access
// per few lanes and starve this kernel): per stage of 8 blocks the tile's 4 KB
// of weights and 512 B of scales are copied into LDS by the 4 waves
// (global_load_lds, 16 B per lane, 2 copies per wave), two stages ahead into
// a ring of 3 buffers; each wave loads its activation operands with one
// dwordx4 per lane per row tile and block pair (the tiled order of
// common_quant_rows), one stage ahead. MFMA operand layout (wave64):
// A[l%16][8(l/16) .. +8), B[8(l/16) .. +8)[l%16], D[4(l/16) + r][l%16]; B
// lane l: column 16g + l%16 of the tile, K dword l/16 of the block, widened
// to 8 int8 = 16 * q.
constexpr int kGemmChunk = 8;                    // blocks per stage
constexpr int kGemmBufs = 3;                     // LDS stage buffers
constexpr int kGemmStageBytes = kGemmChunk * 512 + kGemmChunk * 64;

__device__ __forceinline__ void gemm_lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

// KS = 2 doubles the waves: wave 4h + g takes row group g over K half h
// (its own staging ring); the halves' sums meet in LDS and are added in a
// fixed order.
template <int KS>
__global__ __launch_bounds__(256 * KS) void common_gemm(const uint8_t *__restrict__ w, const int8_t *__restrict__ tiled,
                                                       const float *__restrict__ row_scales, float *__restrict__ y,
                                                       int rows, int defined_rows, int kp, int n, int np) {
    __shared__ __attribute__((aligned(16))) uint8_t lds_all[KS * kGemmBufs * kGemmStageBytes];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int wid = wave & 3, half = wave >> 2;
    uint8_t *const stage_lds = lds_all + half * kGemmBufs * kGemmStageBytes;
    const int tile = blockIdx.x;
    const int row0 = 32 * wid;
    const bool active = row0 < defined_rows;
    const int blocks = kp >> 5;
    const int chunks = blocks / kGemmChunk / KS;   // per K half (kp % (256 * KS) == 0)
    const int chunk0 = half * chunks;
    const int pairs = blocks / 2;
    const uint8_t *scales = w + static_cast<size_t>(np) * kp / 2;
    const int q = lane >> 4, c16 = lane & 15;

    // copies of stage c into buffer c % 3: wave w takes blocks 2w, 2w+1 (1 KB
    // of weights) and their scales (lanes 0..7: block 2w + lane/4, 16 B each)
    auto copy_stage = [&](int c) {
        const int cc = chunk0 + min(c, chunks - 1);        // past the end: a copy nobody reads
        uint8_t *buf = stage_lds + (c % kGemmBufs) * kGemmStageBytes;
        const int b0 = cc * kGemmChunk + 2 * wid;
        __builtin_amdgcn_global_load_lds(w + (static_cast<size_t>(tile) * blocks + b0) * 512 + lane * 16,
                                         buf + wid * 1024, 16, 0, 0);
        const int sl = min(lane, 7);                       // lanes 8.. repeat lane 7's copy
        const uint8_t *ssrc = scales + (static_cast<size_t>(b0 + sl / 4) * np + tile * 32) * 2 + (sl % 4) * 16;
        if (lane < 8) __builtin_amdgcn_global_load_lds(ssrc, buf + kGemmChunk * 512 + wid * 128, 16, 0, 0);
    };
    // activation operands of stage c: [row tile][block pair] as uint4
    const int8_t *abase = tiled + (static_cast<size_t>(row0 / 16) * pairs * 64 + lane) * 16;
    auto load_a = [&](int c, uint4 (&a)[2][kGemmChunk / 2]) {
        const int cc = chunk0 + min(c, chunks - 1);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int p = 0; p < kGemmChunk / 2; ++p)
                a[i][p] = *reinterpret_cast<const uint4 *>(abase + (static_cast<size_t>(i) * pairs +
                                                                    cc * (kGemmChunk / 2) + p) * 64 * 16);
    };
    auto widen = [](uint32_t wd) -> long {
        const uint32_t ev = (wd << 4) & 0xf0f0f0f0u, od = wd & 0xf0f0f0f0u;
        const uint32_t lo = __builtin_amdgcn_perm(od, ev, 0x05010400u);   // K 0..3
        const uint32_t hi = __builtin_amdgcn_perm(od, ev, 0x07030602u);   // K 4..7
        return static_cast<long>((static_cast<unsigned long>(hi) << 32) | lo);
    };

    float acc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
    const int32x4 zero = {0, 0, 0, 0};

    uint4 a_cur[2][kGemmChunk / 2], a_next[2][kGemmChunk / 2];
    // issue order: copies 0, A 0, copies 1; then per step c: A c+1, copies c+2.
    // At the top of step c only copies c+1 (2 per wave) may still be in flight.
    copy_stage(0);
    if (active) load_a(0, a_next);
    copy_stage(1);
    for (int c = 0; c < chunks; ++c) {
        __builtin_amdgcn_s_waitcnt(0x0F70 | 2);            // vmcnt(2): all but copies c+1
        gemm_lds_barrier();                                // every wave's copies of c landed,
                                                           // and reads of buffer (c-1)%3 are done
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int p = 0; p < kGemmChunk / 2; ++p) a_cur[i][p] = a_next[i][p];
        if (active) load_a(c + 1, a_next);
        copy_stage(c + 2);
        if (!active) continue;
        const uint8_t *buf = stage_lds + (c % kGemmBufs) * kGemmStageBytes;
#pragma unroll
        for (int j = 0; j < kGemmChunk; ++j) {
            const uint32_t w0 = *reinterpret_cast<const uint32_t *>(buf + j * 512 + c16 * 32 + 4 * q);
            const uint32_t w1 = *reinterpret_cast<const uint32_t *>(buf + j * 512 + c16 * 32 + 16 + 4 * q);
            const uint16_t *sc = reinterpret_cast<const uint16_t *>(buf + kGemmChunk * 512 + j * 64);
            const float d0 = kk::half_bits_to_float(sc[c16]) * 0.0625f;
            const float d1 = kk::half_bits_to_float(sc[16 + c16]) * 0.0625f;
            const long b0 = widen(w0), b1 = widen(w1);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint4 v = a_cur[i][j / 2];
                const long a = (j & 1) ? static_cast<long>((static_cast<unsigned long>(v.w) << 32) | v.z)
                                       : static_cast<long>((static_cast<unsigned long>(v.y) << 32) | v.x);
                const int32x4 p0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b0, zero, 0, 0, 0);
                const int32x4 p1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, zero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc[i][0][r] = fmaf(static_cast<float>(p0[r]), d0, acc[i][0][r]);
                    acc[i][1][r] = fmaf(static_cast<float>(p1[r]), d1, acc[i][1][r]);
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);                         // the trailing copies land before exit
    if (KS > 1) {
        // half 1 hands its sums to half 0 through the (now idle) staging LDS
        gemm_lds_barrier();
        float4 *xfer = reinterpret_cast<float4 *>(lds_all);     // [group][i*2+j][lane]
        if (half == 1 && active) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    xfer[(wid * 4 + i * 2 + j) * 64 + lane] =
                        make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
        }
        __syncthreads();
        if (half == 1) return;
        if (active) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float4 v = xfer[(wid * 4 + i * 2 + j) * 64 + lane];
                    acc[i][j][0] += v.x;
                    acc[i][j][1] += v.y;
                    acc[i][j][2] += v.z;
                    acc[i][j][3] += v.w;
                }
        }
    }
    if (!active) return;
    const int col[2] = {tile * 32 + c16, tile * 32 + 16 + c16};
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + 16 * i + 4 * q + r;
            if (row >= rows) continue;
            const float s = row_scales[row * 16];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                if (col[j] < n) y[static_cast<size_t>(row) * n + col[j]] = acc[i][j][r] * s;
        }
}

} // namespace

extern "C" int kk_common_quant_pair(const void *x, int x_f16, int k, int kp, void *values, void *params,
                                    hipStream_t stream) {
    if (!x || !values || !params || k <= 0 || kp < k || kp % 256 != 0 || kp > 16384) return hipErrorInvalidValue;
    if (x_f16)
        hipLaunchKernelGGL(common_quant_pair<true>, dim3(1), dim3(kQuantThreads), 0, stream, x, x_f16, k, kp,
                           static_cast<int8_t *>(values), static_cast<float *>(params));
    else
        hipLaunchKernelGGL(common_quant_pair<false>, dim3(1), dim3(kQuantThreads), 0, stream, x, x_f16, k, kp,
                           static_cast<int8_t *>(values), static_cast<float *>(params));
    return hipGetLastError();
}

extern "C" int kk_common_quant_rows(const void *x, int x_f16, int k, int kp, int rows, int defined_rows,
                                    void *values, void *params, void *tiled, hipStream_t stream) {
    if (!x || !values || !params || !tiled || k <= 0 || kp < k || kp % 256 != 0 || rows <= 0 ||
        defined_rows < rows || defined_rows % 32 != 0)
        return hipErrorInvalidValue;
    if (x_f16)
        hipLaunchKernelGGL(common_quant_rows<true>, dim3(defined_rows), dim3(kRowThreads), 0, stream, x, x_f16, k, kp,
                           rows, static_cast<int8_t *>(values), static_cast<float *>(params),
                           static_cast<int8_t *>(tiled));
    else
        hipLaunchKernelGGL(common_quant_rows<false>, dim3(defined_rows), dim3(kRowThreads), 0, stream, x, x_f16, k,
                           kp, rows, static_cast<int8_t *>(values), static_cast<float *>(params),
                           static_cast<int8_t *>(tiled));
    return hipGetLastError();
}

extern "C" size_t kk_common_gemv_lds_bytes(int kp, int exact) {
    const size_t blocks = static_cast<size_t>(kp) / 32;
    return blocks * (exact ? 24 * 4 + 4 : 16 * 4) + static_cast<size_t>(kCqWaves) * 32 * 4;
}

extern "C" int kk_common_gemv(const void *w0, float *y0, const void *w1, float *y1, const void *act, int mode,
                              int x_f16, void *params, void *view_values, int k, int kp, int n, int np,
                              hipStream_t stream) {
    if (!w0 || !y0 || !act || mode < 0 || mode > 2 || (mode != kExact && !params) ||
        (mode == kQuantize && !view_values) || kp % 256 != 0 || kp > 16384 || np % 256 != 0 || n > np || k > kp ||
        (reinterpret_cast<uintptr_t>(w0) & 255) != 0 || (w1 && (reinterpret_cast<uintptr_t>(w1) & 255)))
        return hipErrorInvalidValue;
    const int tiles = (n + 31) / 32;
    const int count = w1 ? 2 : 1;
    const size_t lds = kk_common_gemv_lds_bytes(kp, mode == kExact);
    const GemvMatrix m0{static_cast<const uint8_t *>(w0), y0};
    const GemvMatrix m1{static_cast<const uint8_t *>(w1 ? w1 : w0), w1 ? y1 : y0};
    const dim3 grid(tiles * count), block(kCqThreads);
    int8_t *vv = static_cast<int8_t *>(view_values);
    float *pp = static_cast<float *>(params);
#define KK_COMMON_GEMV(M, F)                                                                                \
    hipLaunchKernelGGL((common_gemv<M, F>), grid, block, lds, stream, m0, m1, tiles, act, x_f16, pp, vv, pp, k, kp, n, \
                       np)
    if (mode == kExact) {
        if (x_f16) KK_COMMON_GEMV(kExact, true); else KK_COMMON_GEMV(kExact, false);
    } else if (mode == kQuantize) {
        if (x_f16) KK_COMMON_GEMV(kQuantize, true); else KK_COMMON_GEMV(kQuantize, false);
    } else {
        if (x_f16) KK_COMMON_GEMV(kPrepared, true); else KK_COMMON_GEMV(kPrepared, false);
    }
#undef KK_COMMON_GEMV
    return hipGetLastError();
}

extern "C" int kk_common_gemm(const void *w, const void *tiled, const void *row_scales, float *y, int rows,
                              int defined_rows, int kp, int n, int np, hipStream_t stream) {
    // kp % 256 == 0 also makes the block count a multiple of the GEMM's ring depth
    if (!w || !tiled || !row_scales || !y || rows <= 0 || rows > 128 || defined_rows < rows ||
        defined_rows % 32 != 0 || defined_rows > 128 || kp % 256 != 0 || np % 256 != 0 || n > np ||
        (reinterpret_cast<uintptr_t>(w) & 255) != 0 || (reinterpret_cast<uintptr_t>(tiled) & 15) != 0)
        return hipErrorInvalidValue;
    const int tiles = (n + 31) / 32;
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const int8_t *tb = static_cast<const int8_t *>(tiled);
    const float *rs = static_cast<const float *>(row_scales);
    // two K halves per tile when Kp splits into whole stages (and the tiles
    // alone would leave compute units idle)
    if (kp % 512 == 0 && tiles < 1024)
        hipLaunchKernelGGL(common_gemm<2>, dim3(tiles), dim3(512), 0, stream, wb, tb, rs, y, rows, defined_rows, kp,
                           n, np);
    else
        hipLaunchKernelGGL(common_gemm<1>, dim3(tiles), dim3(256), 0, stream, wb, tb, rs, y, rows, defined_rows, kp,
                           n, np);
    return hipGetLastError();
}
