// Small-batch (1..16) Q4_0 GEMV on gfx950 fp16 MFMA with block-diagonal
// activation operands: one pass over the weights for the whole batch, each
// lane streaming whole 36-byte block pairs of one weight row.
//
// Y[b, r] = sum_k X[b, k] * W[r, k]  (reference kernels/kunlun-matvec.xpu:24-79,
// which re-reads W once per batch column). HBM-bound by design.
//
// Lane layout. A compute wave owns a tile of 16 weight rows and all of K;
// lane (n, h) = (l % 16, l / 16) loads row n, block pair 4 * step + h (x4,
// x4, x1: 36 bytes), so one load instruction covers 16 rows x 144 contiguous
// bytes. For v_mfma_f32_16x16x32_f16 that lane is B[8h .. 8h+7][n]: the four
// k-groups of one MFMA carry four different block pairs. The activation
// operand A is block diagonal: row m = 4s + i (slot s, batch column i of a
// group of four) is non-zero only in k-group s, where it holds the
// activations of pair 4 * step + s. Then D[4h + i][n] sums the 8 values of
// k-group h only, a partial sum of one Q4_0 block of row n, which lane (n, h)
// holds together with that block's F16 scale: no data crosses lanes before
// the final sum. Per block, four nibble dwords x hi/lo fragments = 8 MFMAs
// accumulate the block's 32 products into D; then acc += D * (d * s_inv) in
// F32.
//
// Workgroup. 16 waves = T tiles x P K-parts (T * P = 16): each wave owns
// SPW consecutive steps of one tile and keeps the next step in flight while
// it computes one (deeper rings measured slower: every wave's data then
// arrives late and the MFMA work does not overlap the stream). The four
// slots of a row (lanes n, n+16, n+32, n+48) are added in registers, then the
// P parts of each tile through LDS, in part order, so results do not depend
// on timing.
//
// Activations. Every wave first requests its share of X, then its weights,
// and converts X into LDS fragments while the weights are in flight (the
// memory counter is in order, so the conversion waits for X only); one
// LDS-only barrier later the fragments of all of K are visible. Per 32-value
// block and batch column a
// power of two 2^(14-e) with max |x| < 2^e (e clamped to [-100, 126]) scales
// the block into fp16 range, hi = fp16(x * 2^(14-e)), lo = fp16(x * 2^(14-e)
// - hi), so |x - (hi + lo) 2^(e-14)| <= 2^-22 max|x| of the block;
// s_inv = 2^(e-14) is applied with the weight scale. A block holding an Inf or
// NaN gets s_inv = NaN: its batch column becomes NaN in every output row (the
// batch-1 GEMV's rule). Each A operand occupies 272 LDS bytes: the 16 active
// lanes' 16-byte fragments, then 16 zero bytes that the 48 inactive lanes
// read.
//
// Steps past K (the last part's tail) re-read the last step (in bounds) and
// contribute zero (weight scale 0, zero activations, activation scale 0).
#include "device_common.h"
#include "launch.h"
#include "lds_opt_in.h"

#include <algorithm>

namespace {

using kk::half8;
using kk::kWave;

typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kTileRows = 16;
constexpr int kWaves = 16;                   // waves per workgroup: tiles x K-parts
constexpr int kThreads = kWaves * kWave;
constexpr int kOperandBytes = 17 * 16;       // 16 active fragments + the zero slot
constexpr int kMaxLdsBytes = 160 * 1024;
constexpr int kMaxStepsPerWave = 4;

// LDS bytes per step and column group: 16 operands ([block][dword][hi|lo])
// and the 2 x 4 slot scales of the 4 columns.
constexpr int kStepGroupBytes = 16 * kOperandBytes + 2 * 4 * 16;

struct BdPlan {
    int tiles_per_group = 0;   // T
    int parts = 0;             // P = 16 / T
    int steps_per_wave = 0;    // SPW
    int steps = 0;             // P * SPW >= ceil(K / 256)
    size_t lds_bytes = 0;
    int items = 0;             // activation items per thread (1, 2 or 4)
};

// The plan for T tiles per workgroup: steps per wave, LDS bytes and
// activation items per thread; parts == 0 when it does not fit the per-wave
// step, LDS and item limits (column groups 3 and 4 keep one step per wave:
// more would not fit in 128 VGPRs) or a K-part would hold no pair.
BdPlan bdiag_candidate(int k, int batch, int t) {
    const int q = (batch + 3) / 4;
    const int need = (k + 255) / 256;
    BdPlan p;
    p.tiles_per_group = t;
    p.parts = kWaves / t;
    p.steps_per_wave = (need + p.parts - 1) / p.parts;
    p.steps = p.parts * p.steps_per_wave;
    p.lds_bytes = static_cast<size_t>(p.steps) * q * kStepGroupBytes + static_cast<size_t>(kThreads) * q * 4;
    p.items = (4 * q * p.steps * 32 + kThreads - 1) / kThreads;
    p.items = p.items <= 1 ? 1 : p.items <= 2 ? 2 : p.items <= 4 ? 4 : 0;
    if (p.steps_per_wave > (q > 2 ? 1 : kMaxStepsPerWave) || p.lds_bytes > static_cast<size_t>(kMaxLdsBytes) ||
        p.items == 0 || (p.parts > need && t < kWaves))   // no part may be padding only
        p.parts = 0;
    return p;
}

constexpr int kTileChoices[] = {1, 2, 4, 8, 16};

// Operand (step, block, dword, hi|lo, group) and scale quad (step, block, group, slot) offsets.
__device__ __forceinline__ int operand_offset(int q_groups, int step, int blk, int dw, int hl, int q) {
    return ((((step * 2 + blk) * 4 + dw) * 2 + hl) * q_groups + q) * kOperandBytes;
}
__device__ __forceinline__ int scale_offset(int q_groups, int steps, int step, int blk, int q, int slot) {
    return steps * q_groups * 16 * kOperandBytes + (((step * 2 + blk) * q_groups + q) * 4 + slot) * 16;
}

// Q = column groups of four (batch <= 4Q), SPW = steps per wave, ITEMS =
// activation items per thread (4Q * steps * 32 items over the workgroup).
// w2 (gate/up pair, else null): tile 2i holds rows 16i .. 16i + 15 of w (the
// gate matrix), tile 2i + 1 the same rows of w2 (the up matrix); n is the
// row count of each and the workgroup's tile count is even, so both tiles of
// a pair meet in one workgroup, whose epilogue writes y = SiLU(gate) * up
// ([batch][n], kk::swiglu_value).
template <int Q, int SPW, int ITEMS>
__global__ __launch_bounds__(kThreads) void q4_bdiag_gemv(const uint8_t *__restrict__ w,
                                                        const uint8_t *__restrict__ w2,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int k, int n, int batch, int steps,
                                                        int parts) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pairs = k >> 6;
    const size_t row_bytes = static_cast<size_t>(pairs) * 36;
    const int nl = lane & 15, h = lane >> 4;
    const int part = wid % parts;
    const int tile = blockIdx.x * (kWaves / parts) + wid / parts;
    const bool second = w2 && (tile & 1);                       // wave-uniform: an up tile of the pair
    const int row_tile = w2 ? tile >> 1 : tile;
    const int row = min(row_tile * kTileRows + nl, n - 1);
    const int s_first = part * SPW;

    // 1. this thread's activation items (column b, pair p, block blk, dword
    //    dw), dw fastest so a block's four items are one quad of lanes
    const int items = 4 * Q * steps * 32;
    float4 xlo[ITEMS], xhi[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int item = min(tid + it * kThreads, items - 1);
        const int dw = item & 3, blk = (item >> 2) & 1, pb = item >> 3;
        const int b = pb / (4 * steps), p = pb - b * (4 * steps);
        const float *src =
            x + static_cast<size_t>(min(b, batch - 1)) * k + (2 * min(p, pairs - 1) + blk) * 32 + 4 * dw;
        xlo[it] = *reinterpret_cast<const float4 *>(src);
        xhi[it] = *reinterpret_cast<const float4 *>(src + 16);
    }
    // 2. the wave's first step: step s_first + j holds pair 4(s_first+j) + h
    uint32_t ring[SPW][9];
    auto load_step = [&](int j) {
        const int p = min(4 * (s_first + j) + h, pairs - 1);
        const uint32_t *src = reinterpret_cast<const uint32_t *>((second ? w2 : w) + static_cast<size_t>(row) * row_bytes +
                                                                 static_cast<size_t>(p) * 36);
        const kk::u32x4_a4 a = kk::load_u32x4(src), c = kk::load_u32x4(src + 4);
        ring[j][0] = a.x; ring[j][1] = a.y; ring[j][2] = a.z; ring[j][3] = a.w;
        ring[j][4] = c.x; ring[j][5] = c.y; ring[j][6] = c.z; ring[j][7] = c.w;
        ring[j][8] = src[8];
    };
    __builtin_amdgcn_sched_barrier(0);
    load_step(0);
    __builtin_amdgcn_sched_barrier(0);

    // 3. activations -> hi/lo fragments in LDS (the weights stay in flight)
    for (int o = tid; o < steps * Q * 16; o += kThreads)
        *reinterpret_cast<uint4 *>(lds + o * kOperandBytes + 256) = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
        const int item = tid + it * kThreads;
        const int dw = item & 3, blk = (item >> 2) & 1, pb = item >> 3;
        const int b = pb / (4 * steps), p = pb - b * (4 * steps);
        const bool live = item < items && b < batch && p < pairs;
        // block positions (4dw, 4dw+2, 4dw+1, 4dw+3, 16+4dw, 16+4dw+2, 16+4dw+1, 16+4dw+3)
        float v[8] = {xlo[it].x, xlo[it].z, xlo[it].y, xlo[it].w, xhi[it].x, xhi[it].z, xhi[it].y, xhi[it].w};
        float m = 0.0f, bad = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            v[t] = live ? v[t] : 0.0f;
            const float a = fabsf(v[t]);
            bad = (a <= 3.402823466e38f) ? bad : 1.0f;
            m = fmaxf(m, a);
        }
        m = fmaxf(m, kk::dpp_move<0xb1>(m));
        m = fmaxf(m, kk::dpp_move<0x4e>(m));
        bad = fmaxf(bad, kk::dpp_move<0xb1>(bad));
        bad = fmaxf(bad, kk::dpp_move<0x4e>(bad));
        const int e = bad != 0.0f ? 0 : min(max(__builtin_amdgcn_frexp_expf(m), -100), 126);
        const float scale = ldexpf(1.0f, 14 - e);
        half8 hi, lo;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float a = bad != 0.0f ? 0.0f : v[t] * scale;
            const _Float16 hv = static_cast<_Float16>(a);
            hi[t] = hv;
            lo[t] = static_cast<_Float16>(a - static_cast<float>(hv));
        }
        if (item < items) {
            const int step = p >> 2, slot = p & 3, q = b >> 2, i = b & 3;
            const int frag = (slot * 4 + i) * 16;
            *reinterpret_cast<half8 *>(lds + operand_offset(Q, step, blk, dw, 0, q) + frag) = hi;
            *reinterpret_cast<half8 *>(lds + operand_offset(Q, step, blk, dw, 1, q) + frag) = lo;
            if (dw == 0) {
                const float s_inv = !live ? 0.0f : bad != 0.0f ? __builtin_nanf("") : ldexpf(1.0f, e - 14);
                *reinterpret_cast<float *>(lds + scale_offset(Q, steps, step, blk, q, slot) + 4 * i) = s_inv;
            }
        }
    }
    kk::lds_barrier();   // every fragment written; the weights may still be in flight

    // 4. per step and block: 8 MFMAs per column group, then the scaled sums
    const int am = lane & 15;
    const bool active = (am >> 2) == h;                         // A row 4s + i lives in k-group s
    const int a_base = active ? (h * 4 + (am & 3)) * 16 : 256;  // inactive lanes read the zero slot
    float4v acc[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) acc[q] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
        if (j + 1 < SPW) {   // the next step goes out before this one is used
            __builtin_amdgcn_sched_barrier(0);
            load_step(j + 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        const int s = s_first + j;
        const bool valid = 4 * s + h < pairs;
        // block 0 of the pair: scale bytes 0-1, nibbles 2-17 (dword dw = bytes
        // 2+4dw..5+4dw); block 1: scale bytes 18-19, nibbles 20-35
        const float d0 = valid ? kk::half_bits_to_float(ring[j][0] & 0xffffu) : 0.0f;
        const float d1 = valid ? kk::half_bits_to_float(ring[j][4] >> 16) : 0.0f;
        float4v t[2][Q];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int q = 0; q < Q; ++q) t[blk][q] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int dw = 0; dw < 4; ++dw) {
            const half8 bq[2] = {kk::q4_dword_halves(kk::align_bytes(ring[j][dw + 1], ring[j][dw], 2)),
                                 kk::q4_dword_halves(ring[j][5 + dw])};
#pragma unroll
            for (int hl = 0; hl < 2; ++hl)
#pragma unroll
                for (int blk = 0; blk < 2; ++blk)
#pragma unroll
                    for (int q = 0; q < Q; ++q) {
                        const half8 a =
                            *reinterpret_cast<const half8 *>(lds + operand_offset(Q, s, blk, dw, hl, q) + a_base);
                        t[blk][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq[blk], t[blk][q], 0, 0, 0);
                    }
        }
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            const float dd = blk == 0 ? d0 : d1;
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const float4 sv = *reinterpret_cast<const float4 *>(lds + scale_offset(Q, steps, s, blk, q, h));
                acc[q][0] = fmaf(t[blk][q][0], dd * sv.x, acc[q][0]);
                acc[q][1] = fmaf(t[blk][q][1], dd * sv.y, acc[q][1]);
                acc[q][2] = fmaf(t[blk][q][2], dd * sv.z, acc[q][2]);
                acc[q][3] = fmaf(t[blk][q][3], dd * sv.w, acc[q][3]);
            }
        }
    }

    // 5. the four slots of row n (lanes n, n+16, n+32, n+48): lane (n, h)
    //    keeps column 4q + h; then the parts of each tile through LDS
    float *red = reinterpret_cast<float *>(lds + static_cast<size_t>(steps) * Q * kStepGroupBytes);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[q][i] += __shfl_xor(acc[q][i], 16, kWave);
            acc[q][i] += __shfl_xor(acc[q][i], 32, kWave);
        }
        red[(q * kWaves + wid) * kWave + lane] = h == 0 ? acc[q][0] : h == 1 ? acc[q][1] : h == 2 ? acc[q][2] : acc[q][3];
    }
    __syncthreads();
    if (part != 0 || second) return;
    const int out_row = row_tile * kTileRows + nl;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        float sum = 0.0f;
        for (int pp = 0; pp < parts; ++pp) sum += red[(q * kWaves + wid + pp) * kWave + lane];
        if (w2) {
            // the up tile's waves follow this tile's in the workgroup
            float up = 0.0f;
            for (int pp = 0; pp < parts; ++pp) up += red[(q * kWaves + wid + parts + pp) * kWave + lane];
            sum = kk::swiglu_value(sum, up);
        }
        if (out_row < n && 4 * q + h < batch) y[static_cast<size_t>(4 * q + h) * n + out_row] = sum;
    }
}

template <int Q, int SPW, int ITEMS>
const void *bdiag_kernel() {
    return reinterpret_cast<const void *>(&q4_bdiag_gemv<Q, SPW, ITEMS>);
}

// The kernel instance of a plan.
template <int Q>
const void *bdiag_kernel_for(const BdPlan &p) {
    if constexpr (Q > 2) {
        return p.items == 1 ? bdiag_kernel<Q, 1, 1>() : p.items == 2 ? bdiag_kernel<Q, 1, 2>() : bdiag_kernel<Q, 1, 4>();
    } else {
#define KK_BDIAG_SPW(S) (p.items == 1 ? bdiag_kernel<Q, S, 1>() : p.items == 2 ? bdiag_kernel<Q, S, 2>() : bdiag_kernel<Q, S, 4>())
        switch (p.steps_per_wave) {
        case 1: return KK_BDIAG_SPW(1);
        case 2: return KK_BDIAG_SPW(2);
        case 3: return KK_BDIAG_SPW(3);
        default: return KK_BDIAG_SPW(4);
        }
#undef KK_BDIAG_SPW
    }
}

const void *bdiag_kernel_for(int q, const BdPlan &p) {
    switch (q) {
    case 1: return bdiag_kernel_for<1>(p);
    case 2: return bdiag_kernel_for<2>(p);
    case 3: return bdiag_kernel_for<3>(p);
    default: return bdiag_kernel_for<4>(p);
    }
}

// Workgroups of `kernel` one CU holds at once with `lds` bytes each (dynamic
// LDS above 64 KiB opted into once per device and kernel). 0 when the query
// fails.
int bdiag_per_cu(const void *kernel, size_t lds) {
    if (kk::opt_in_lds(kernel, lds) != hipSuccess) return 0;
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, kThreads, lds) != hipSuccess) return 0;
    return blocks;
}

} // namespace

extern "C" int kk_q4_bdiag_gemv_supported(const void *w, const float *x, int k, int n, int batch) {
    if (!(batch >= 1 && batch <= 16 && k >= 64 && k <= 16384 && k % 64 == 0 && n >= 1 &&
          (reinterpret_cast<uintptr_t>(w) & 3) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0))
        return 0;
    for (int t : kTileChoices)
        if (bdiag_candidate(k, batch, t).parts > 0) return 1;
    return 0;
}

// Tiles per workgroup: the fewest (1, 2, 4, 8, 16) with which the workgroups
// the CUs hold at once cover every tile (else the last candidate that fits).
namespace {
hipError_t launch_bdiag(const void *w, const void *w2, const float *x, float *y, int k, int n, int batch, int cus,
                        hipStream_t stream) {
    int device = 0;
    hipError_t rc = hipGetDevice(&device);
    if (rc != hipSuccess) return rc;
    const int q = (batch + 3) / 4;
    const int tiles = (w2 ? 2 : 1) * ((n + kTileRows - 1) / kTileRows);
    BdPlan plan;
    const void *kernel = nullptr;
    for (int t : kTileChoices) {
        if (w2 && t == 1) continue;                             // a pair's two tiles share a workgroup
        const BdPlan p = bdiag_candidate(k, batch, t);
        if (p.parts == 0) continue;
        const void *kp = bdiag_kernel_for(q, p);
        const int per_cu = bdiag_per_cu(kp, p.lds_bytes);
        if (per_cu == 0) continue;
        plan = p;
        kernel = kp;
        if ((tiles + t - 1) / t <= cus * per_cu) break;
    }
    if (!kernel) return hipErrorInvalidConfiguration;
    const int groups = (tiles + plan.tiles_per_group - 1) / plan.tiles_per_group;
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    const uint8_t *wb2 = static_cast<const uint8_t *>(w2);
    void *args[] = {&wb, &wb2, &x, &y, &k, &n, &batch, &plan.steps, &plan.parts};
    rc = hipLaunchKernel(kernel, dim3(groups), dim3(kThreads), args, plan.lds_bytes, stream);
    return rc != hipSuccess ? rc : hipGetLastError();
}
} // namespace

extern "C" int kk_q4_bdiag_gemv(const void *w, const float *x, float *y, int k, int n, int batch, int cus,
                                hipStream_t stream) {
    if (!kk_q4_bdiag_gemv_supported(w, x, k, n, batch) || !y || cus <= 0) return hipErrorInvalidValue;
    return launch_bdiag(w, nullptr, x, y, k, n, batch, cus, stream);
}

// Gate/up pair: both matrices in one launch (X staged once per workgroup),
// y = [batch][n] = SiLU(X w_gate^T) * (X w_up^T).
extern "C" int kk_q4_bdiag_gemv_pair_swiglu(const void *w_gate, const void *w_up, const float *x, float *y, int k,
                                            int n, int batch, int cus, hipStream_t stream) {
    if (!kk_q4_bdiag_gemv_supported(w_gate, x, k, n, batch) || !kk_q4_bdiag_gemv_supported(w_up, x, k, n, batch) ||
        !w_up || !y || cus <= 0 || n > (1 << 29))
        return hipErrorInvalidValue;
    return launch_bdiag(w_gate, w_up, x, y, k, n, batch, cus, stream);
}
