// rowwise_i8 matmul on gfx950: device-side two-pass activation quantization
// and int8 MFMA with exact int32 accumulation and a fused combine epilogue.
//
// Reference path (reference src/k200.cpp:189-240): X is copied to the host,
// quantized per tensor in two passes (k200.cpp:212-225), uploaded, multiplied
// by the int8 weight rows in a closed vendor FC (k200.cpp:231,234-235) and
// combined as (P*max0/127 + R*max1/127) * scale[r]
// (reference kernels/kunlun-combine.xpu:10-19). Here all of it stays on the
// GPU: three quantization passes (or one single-workgroup pass for small X)
// and one MFMA kernel.
//
// Workspace layout (device):
//   codes    [2*batch][k] int8, row 2b = q0 of batch row b, row 2b+1 = q1
//   partial0 [kMaxGroups] f32  per-workgroup max|x|
//   partial1 [kMaxGroups] f32  per-workgroup max|r|
//   final    [4] f32           max0, max1
#include "device_common.h"
#include "launch.h"
#include "lds_opt_in.h"
#include "tuning.h"

#include <algorithm>
#include <cstdlib>

namespace {

using kk::kWave;

constexpr int kMaxGroups = 1024;
constexpr int kQuantThreads = 256;
constexpr int kFusedThreads = 1024;

struct Workspace {
    int8_t *codes;
    float *partial0;
    float *partial1;
    float *final_max;
};

size_t align256(size_t bytes) { return (bytes + 255) & ~static_cast<size_t>(255); }

__host__ __device__ inline Workspace layout(void *base, int k, int batch) {
    char *p = static_cast<char *>(base);
    const size_t codes = ((static_cast<size_t>(2) * batch * k) + 255) & ~static_cast<size_t>(255);
    Workspace ws;
    ws.codes = reinterpret_cast<int8_t *>(p);
    ws.partial0 = reinterpret_cast<float *>(p + codes);
    ws.partial1 = ws.partial0 + kMaxGroups;
    ws.final_max = ws.partial1 + kMaxGroups;
    return ws;
}

__device__ __forceinline__ void flag_nonfinite(int *status) {
    __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide max over float values held by each thread; result on all threads.
// LDS_ONLY: the barriers wait for LDS operations only, so global loads issued
// before the call stay in flight.
template <int Threads, bool LDS_ONLY = false>
__device__ float block_max(float v, float *scratch) {
    v = kk::wave_max(v);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (LDS_ONLY) kk::lds_barrier(); else __syncthreads();
    if (lane == 0) scratch[wave] = v;
    if (LDS_ONLY) kk::lds_barrier(); else __syncthreads();
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < Threads / kWave; ++i) m = fmaxf(m, scratch[i]);
    return m;
}

// Activation quantization arithmetic, rounded exactly as the reference host
// code (reference src/k200.cpp:216-218,223-224): no contraction.
__device__ __forceinline__ int quant_primary(float value, float max0) {
#pragma clang fp contract(off)
    const float inv = 127.0f / max0;
    return kk::round_clamp(value * inv, 127);
}
__device__ __forceinline__ float residual_of(float value, int q0, float max0) {
#pragma clang fp contract(off)
    const float step = max0 / 127.0f;
    const float product = static_cast<float>(q0) * step;
    return value - product;
}
__device__ __forceinline__ int quant_residual(float residual, float max1) {
#pragma clang fp contract(off)
    const float inv = 127.0f / max1;
    return kk::round_clamp(residual * inv, 127);
}

// Values are handled in groups of 4 (flat index 4 q): K % 32 == 0, so a group
// never crosses a row and its 4 codes go out as one 32-bit store at row
// 2b + component.
__device__ __forceinline__ size_t group_code_offset(size_t flat4, int k, int component) {
    const size_t b = flat4 / static_cast<size_t>(k), j = flat4 - b * static_cast<size_t>(k);
    return (2 * b + component) * static_cast<size_t>(k) + j;
}
// The same offset in 32-bit arithmetic, for 2 * batch * k < 2^32 (a 64-bit
// division is a long instruction sequence; a 32-bit one a few).
__device__ __forceinline__ uint32_t group_code_offset32(uint32_t flat4, uint32_t k, int component) {
    const uint32_t b = flat4 / k, j = flat4 - b * k;
    return (2 * b + static_cast<uint32_t>(component)) * k + j;
}
__device__ __forceinline__ uint32_t pack_codes(int a, int b, int c, int d) {
    return (static_cast<uint32_t>(a) & 0xffu) | ((static_cast<uint32_t>(b) & 0xffu) << 8) |
           ((static_cast<uint32_t>(c) & 0xffu) << 16) | (static_cast<uint32_t>(d) << 24);
}
// four activations from a 4-byte aligned address (X needs only float alignment)
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ float4 load_x4(const float *x, size_t q) {
    const f32x4_a4 v = *reinterpret_cast<const f32x4_a4 *>(x + 4 * q);
    return float4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ bool finite4(const float4 &v) {
    return isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w);
}
__device__ __forceinline__ float absmax4(const float4 &v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// The grid passes below are latency-bound (X is read three times, 8 MB at
// batch 512 x K4096): a thread issues the LOADS groups of a round, and in
// passes 2 and 3 the partial maxima before them, ahead of the first wait; the
// partial maxima are reduced behind LDS-only barriers, so that the X loads
// stay in flight across them. The loads are unconditional (indices clamped
// into X, slots past X discarded afterwards), so that the compiler's wait
// counts stay exact.
constexpr int kPartialsPerThread = kMaxGroups / kQuantThreads;
static_assert(kPartialsPerThread * kQuantThreads == kMaxGroups, "whole partial slots per thread");

// One round of a thread's X groups q, q + stride, ... (groups4 >= 1).
template <int LOADS>
__device__ __forceinline__ void load_round(const float *x, size_t q, size_t stride, size_t groups4,
                                           float4 (&v)[LOADS]) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) v[u] = load_x4(x, min(q + static_cast<size_t>(u) * stride, groups4 - 1));
}

// A thread's slots of the per-workgroup partials (groups >= 1; slots past
// groups repeat the last partial, which leaves the maximum unchanged).
__device__ __forceinline__ void load_partials(const float *partial, int groups, float (&p)[kPartialsPerThread]) {
#pragma unroll
    for (int u = 0; u < kPartialsPerThread; ++u)
        p[u] = partial[min(static_cast<int>(threadIdx.x) + u * kQuantThreads, groups - 1)];
}
__device__ __forceinline__ float max_of(const float (&p)[kPartialsPerThread]) {
    float m = p[0];
#pragma unroll
    for (int u = 1; u < kPartialsPerThread; ++u) m = fmaxf(m, p[u]);
    return m;
}

// Pass 1: per-workgroup max|x| and non-finite detection.
template <int LOADS>
__global__ __launch_bounds__(kQuantThreads) void i8_pass_max(const float *__restrict__ x, size_t count,
                                                            float *__restrict__ partial0, int *status) {
    __shared__ float scratch[kQuantThreads / kWave];
    float m = 0.0f;
    bool bad = false;
    const size_t groups4 = count / 4, stride = static_cast<size_t>(gridDim.x) * kQuantThreads;
    for (size_t q = static_cast<size_t>(blockIdx.x) * kQuantThreads + threadIdx.x; q < groups4;
         q += stride * LOADS) {
        float4 v[LOADS];
        load_round<LOADS>(x, q, stride, groups4, v);
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
            // a clamped slot repeats the last group: the max and the finite test are unchanged
            bad |= !finite4(v[u]);
            m = fmaxf(m, absmax4(v[u]));
        }
    }
    if (bad) flag_nonfinite(status);
    m = block_max<kQuantThreads>(m, scratch);
    if (threadIdx.x == 0) partial0[blockIdx.x] = m;
}

// Pass 2: max0 from the partials, q0 codes, per-workgroup max|r|.
template <int LOADS>
__global__ __launch_bounds__(kQuantThreads) void i8_pass_primary(const float *__restrict__ x, size_t count, int k,
                                                                const float *__restrict__ partial0, int groups,
                                                                int8_t *__restrict__ codes,
                                                                float *__restrict__ partial1) {
    __shared__ float scratch[kQuantThreads / kWave];
    const size_t groups4 = count / 4, stride = static_cast<size_t>(gridDim.x) * kQuantThreads;
    size_t q = static_cast<size_t>(blockIdx.x) * kQuantThreads + threadIdx.x;
    float p0[kPartialsPerThread];
    load_partials(partial0, groups, p0);
    float4 v[LOADS];
    load_round<LOADS>(x, q, stride, groups4, v);
    float max0 = block_max<kQuantThreads, true>(max_of(p0), scratch);
    if (max0 == 0.0f) max0 = 1.0f;
    float m1 = 0.0f;
    for (; q < groups4; q += stride * LOADS) {
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
            const size_t g = q + static_cast<size_t>(u) * stride;
            if (g < groups4) {
                const int a = quant_primary(v[u].x, max0), b = quant_primary(v[u].y, max0);
                const int c = quant_primary(v[u].z, max0), d = quant_primary(v[u].w, max0);
                *reinterpret_cast<uint32_t *>(codes + group_code_offset(4 * g, k, 0)) = pack_codes(a, b, c, d);
                m1 = fmaxf(m1,
                           fmaxf(fmaxf(fabsf(residual_of(v[u].x, a, max0)), fabsf(residual_of(v[u].y, b, max0))),
                                 fmaxf(fabsf(residual_of(v[u].z, c, max0)), fabsf(residual_of(v[u].w, d, max0)))));
            }
        }
        if (q + stride * LOADS < groups4) load_round<LOADS>(x, q + stride * LOADS, stride, groups4, v);
    }
    m1 = block_max<kQuantThreads>(m1, scratch);
    if (threadIdx.x == 0) partial1[blockIdx.x] = m1;
}

// Pass 3: max1 from the partials, q1 codes; workgroup 0 publishes max0/max1.
template <int LOADS>
__global__ __launch_bounds__(kQuantThreads) void i8_pass_residual(const float *__restrict__ x, size_t count, int k,
                                                                 const float *__restrict__ partial0,
                                                                 const float *__restrict__ partial1, int groups,
                                                                 int8_t *__restrict__ codes,
                                                                 float *__restrict__ final_max) {
    __shared__ float scratch[kQuantThreads / kWave];
    const size_t groups4 = count / 4, stride = static_cast<size_t>(gridDim.x) * kQuantThreads;
    size_t q = static_cast<size_t>(blockIdx.x) * kQuantThreads + threadIdx.x;
    float p0[kPartialsPerThread], p1[kPartialsPerThread];
    load_partials(partial0, groups, p0);
    load_partials(partial1, groups, p1);
    float4 v[LOADS];
    load_round<LOADS>(x, q, stride, groups4, v);
    float max0 = block_max<kQuantThreads, true>(max_of(p0), scratch);
    float max1 = block_max<kQuantThreads, true>(max_of(p1), scratch);
    if (max0 == 0.0f) max0 = 1.0f;
    if (max1 == 0.0f) max1 = 1.0f;
    auto q1 = [&](float value) { return quant_residual(residual_of(value, quant_primary(value, max0), max0), max1); };
    for (; q < groups4; q += stride * LOADS) {
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
            const size_t g = q + static_cast<size_t>(u) * stride;
            if (g < groups4)
                *reinterpret_cast<uint32_t *>(codes + group_code_offset(4 * g, k, 1)) =
                    pack_codes(q1(v[u].x), q1(v[u].y), q1(v[u].z), q1(v[u].w));
        }
        if (q + stride * LOADS < groups4) load_round<LOADS>(x, q + stride * LOADS, stride, groups4, v);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        final_max[0] = max0;
        final_max[1] = max1;
    }
}

template <int LOADS>
void launch_passes(const float *x, size_t count, int k, int groups, const Workspace &ws, int *status,
                   hipStream_t stream) {
    hipLaunchKernelGGL(i8_pass_max<LOADS>, dim3(groups), dim3(kQuantThreads), 0, stream, x, count, ws.partial0,
                       status);
    hipLaunchKernelGGL(i8_pass_primary<LOADS>, dim3(groups), dim3(kQuantThreads), 0, stream, x, count, k,
                       ws.partial0, groups, ws.codes, ws.partial1);
    hipLaunchKernelGGL(i8_pass_residual<LOADS>, dim3(groups), dim3(kQuantThreads), 0, stream, x, count, k,
                       ws.partial0, ws.partial1, groups, ws.codes, ws.final_max);
}

// All three passes in one workgroup, for small X (count <= 4 * kFusedThreads *
// kFusedGroups = 65536, so code offsets fit 32 bits): each thread loads its
// groups once and keeps them in registers. The arithmetic runs on one CU (about
// 0.2 us per 1024 values), so by default it takes X only up to 16384 values,
// where it costs as much as the three grid passes (K4096: 8.8 us at 16384
// values, 12.5 at 32768, 18.9 at 65536; the passes about 9.7 together).
constexpr int kFusedGroups = 16;
constexpr int kFusedQuantDefault = 16384;
__global__ __launch_bounds__(kFusedThreads) void i8_quantize_fused(const float *__restrict__ x, size_t count, int k,
                                                                  int8_t *__restrict__ codes,
                                                                  float *__restrict__ final_max, int *status) {
    __shared__ float scratch[kFusedThreads / kWave];
    const int groups4 = static_cast<int>(count / 4);
    float4 v[kFusedGroups];
    float m = 0.0f;
    bool bad = false;
#pragma unroll
    for (int t = 0; t < kFusedGroups; ++t) {
        const int q = static_cast<int>(threadIdx.x) + kFusedThreads * t;
        v[t] = q < groups4 ? load_x4(x, q) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        bad |= !finite4(v[t]);
        m = fmaxf(m, absmax4(v[t]));
    }
    if (bad) flag_nonfinite(status);
    float max0 = block_max<kFusedThreads>(m, scratch);
    if (max0 == 0.0f) max0 = 1.0f;
    float m1 = 0.0f;
#pragma unroll
    for (int t = 0; t < kFusedGroups; ++t) {
        const int q = static_cast<int>(threadIdx.x) + kFusedThreads * t;
        if (q >= groups4) break;
        const int a = quant_primary(v[t].x, max0), b = quant_primary(v[t].y, max0);
        const int c = quant_primary(v[t].z, max0), d = quant_primary(v[t].w, max0);
        *reinterpret_cast<uint32_t *>(codes + group_code_offset32(4u * q, k, 0)) = pack_codes(a, b, c, d);
        m1 = fmaxf(m1, fmaxf(fmaxf(fabsf(residual_of(v[t].x, a, max0)), fabsf(residual_of(v[t].y, b, max0))),
                             fmaxf(fabsf(residual_of(v[t].z, c, max0)), fabsf(residual_of(v[t].w, d, max0)))));
    }
    float max1 = block_max<kFusedThreads>(m1, scratch);
    if (max1 == 0.0f) max1 = 1.0f;
#pragma unroll
    for (int t = 0; t < kFusedGroups; ++t) {
        const int q = static_cast<int>(threadIdx.x) + kFusedThreads * t;
        if (q >= groups4) break;
        auto q1 = [&](float value) { return quant_residual(residual_of(value, quant_primary(value, max0), max0), max1); };
        *reinterpret_cast<uint32_t *>(codes + group_code_offset32(4u * q, k, 1)) =
            pack_codes(q1(v[t].x), q1(v[t].y), q1(v[t].z), q1(v[t].w));
    }
    if (threadIdx.x == 0) {
        final_max[0] = max0;
        final_max[1] = max1;
    }
}

// ---------------------------------------------------------------------------
// int8 MFMA matmul. v_mfma_i32_16x16x64_i8 operand layout (wave64):
//   A (16 x 64): lane l holds A[l % 16][16*(l/16) .. +16)
//   B (64 x 16): lane l holds B[16*(l/16) .. +16)[l % 16]
//   D (16 x 16): lane l holds D[4*(l/16) + i][l % 16], i = 0..3
// The reduction index is permuted so that each lane reads 64 contiguous bytes
// per 256-value K step: in MFMA s (0..3) of a step at k0, lane group g = l/16
// covers k0 + 64*g + 16*s .. +16, for A and B alike, so the four MFMAs sum
// exactly the products of k0 .. k0+255.
//
// A = activation codes (rows: 2b -> q0, 2b+1 -> q1), B^T = weight rows. Lane
// l then holds D rows 4g..4g+3 = (q0, q1) of batch rows 2g' and 2g'+1 for one
// weight row, so the combine happens in registers.
typedef int int32x4 __attribute__((ext_vector_type(4)));

// (P*wmax*s0 + R*wmax*s1) * row_scale, rounded after every operation.
__device__ __forceinline__ float combine(int primary, int residual, float wmax, float scale0, float scale1,
                                         float row_scale) {
#pragma clang fp contract(off)
    const float p = static_cast<float>(primary) * wmax;
    const float q = static_cast<float>(residual) * wmax;
    const float t0 = p * scale0;
    const float t1 = q * scale1;
    return (t0 + t1) * row_scale;
}

template <int MT, int NT>
__global__ __launch_bounds__(256) void i8_mfma_matmul(const int8_t *__restrict__ codes,
                                                     const int8_t *__restrict__ w,
                                                     const float *__restrict__ scales,
                                                     const float *__restrict__ maxima,
                                                     const float *__restrict__ final_max,
                                                     float *__restrict__ y, int k, int n, int batch,
                                                     int m_tiles_total, int n_tiles_total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int m_groups = (m_tiles_total + MT - 1) / MT;
    const int n_groups = (n_tiles_total + NT - 1) / NT;
    if (wave >= m_groups * n_groups) return;
    const int mg = wave % m_groups, ng = wave / m_groups;
    const int rows = 2 * batch;
    const int g = lane >> 4, c = lane & 15;

    int32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = int32x4{0, 0, 0, 0};

    const int8_t *arow[MT];
    bool avalid[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int r = (mg * MT + i) * 16 + c;
        avalid[i] = r < rows;
        arow[i] = codes + static_cast<size_t>(avalid[i] ? r : 0) * k;
    }
    const int8_t *brow[NT];
    bool bvalid[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int r = (ng * NT + j) * 16 + c;
        bvalid[j] = r < n;
        brow[j] = w + static_cast<size_t>(bvalid[j] ? r : 0) * k;
    }

    for (int k0 = 0; k0 < k; k0 += 256) {
        const int kb = k0 + 64 * g;
        int32x4 af[MT][4], bf[NT][4];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int kk0 = kb + 16 * s;
                if (avalid[i] && kk0 < k) {
                    const kk::u32x4_a4 v = kk::load_u32x4(reinterpret_cast<const uint32_t *>(arow[i] + kk0));
                    af[i][s] = int32x4{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
                } else {
                    af[i][s] = int32x4{0, 0, 0, 0};
                }
            }
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int kk0 = kb + 16 * s;
                if (bvalid[j] && kk0 < k) {
                    const kk::u32x4_a4 v = kk::load_u32x4(reinterpret_cast<const uint32_t *>(brow[j] + kk0));
                    bf[j][s] = int32x4{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
                } else {
                    bf[j][s] = int32x4{0, 0, 0, 0};
                }
            }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
    }

    // Epilogue: y[b, r] = (P*(max0/127) + R*(max1/127)) * scale[r], where the
    // raw products are first scaled by the weight maximum / 127 as the FC's
    // max-pointer convention does (the uploaded maxima are 127: exact no-op).
    const float scale0 = final_max[0] / 127.0f;
    const float scale1 = final_max[1] / 127.0f;
    const float wmax = maxima[0] / 127.0f;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int r = (ng * NT + j) * 16 + c;
        if (r >= n) continue;
        const float rs = scales[r];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int b = (mg * MT + i) * 8 + 2 * g + h;
                if (b >= batch) continue;
                y[static_cast<size_t>(b) * n + r] =
                    combine(acc[i][j][2 * h], acc[i][j][2 * h + 1], wmax, scale0, scale1, rs);
            }
        }
    }
}

// Batch 1..64 (2*batch <= 16 MT code rows: MT MFMA row tiles): one
// workgroup per 16 weight rows, its GW waves (8, or 16 at MT = 4) splitting K
// into contiguous ranges of 64-value steps; a chunk of steps is loaded before
// its MFMAs. The MFMA
// wants row l % 16 at k0 + 16 (l / 16) in lane l; the loads read row l / 4
// at k0 + 16 (l % 4) instead (a group of 4 lanes in one row: a load whose
// lanes read 16 rows costs several times more), and ds_bpermute moves lane
// 4 (l % 16) + l / 16's 16 bytes to lane l. The waves' int32 sums meet in LDS
// (exact in any order), then the combine.
constexpr int kGemvWaves = 8;
template <int MT, int GW = kGemvWaves>
__global__ __launch_bounds__(GW * kWave) void i8_gemv_ksplit(const int8_t *__restrict__ codes,
                                                                    const int8_t *__restrict__ w,
                                                                    const float *__restrict__ scales,
                                                                    const float *__restrict__ maxima,
                                                                    const float *__restrict__ final_max,
                                                                    float *__restrict__ y, int k, int n, int batch) {
    constexpr int kChunk = MT <= 1 ? 8 : MT <= 2 ? 6 : MT <= 4 && GW <= 8 ? 4 : 2;   // steps loaded before their MFMAs
    __shared__ int32x4 part[GW - 1][MT][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int n0 = blockIdx.x * 16;
    const int rows = 2 * batch;
    const int steps = (k + 63) / 64;
    const int per = (steps + GW - 1) / GW;
    const int s0 = wid * per, s1 = min(steps, s0 + per);
    const int lr = lane >> 2, lp = lane & 3;                   // loader row and 16-byte piece
    const int src = (4 * c + g) * 4;                           // lane (c, g) takes loader lane 4c + g
    const int8_t *arow[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) arow[i] = codes + static_cast<size_t>(16 * i + lr < rows ? 16 * i + lr : 0) * k;
    const int8_t *brow = w + static_cast<size_t>(min(n0 + lr, n - 1)) * k;
    auto to_mfma_lane = [&](const int32x4 &v) {
        return int32x4{__builtin_amdgcn_ds_bpermute(src, v[0]), __builtin_amdgcn_ds_bpermute(src, v[1]),
                       __builtin_amdgcn_ds_bpermute(src, v[2]), __builtin_amdgcn_ds_bpermute(src, v[3])};
    };

    int32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = int32x4{0, 0, 0, 0};
    for (int sc = s0; sc < s1; sc += kChunk) {
        int32x4 af[kChunk][MT], bf[kChunk];
#pragma unroll
        for (int t = 0; t < kChunk; ++t) {
            const int kk0 = (sc + t) * 64 + 16 * lp;
            const bool ok = sc + t < s1 && kk0 < k;             // K % 32 == 0: a 16-byte chunk is all in or out
            if (ok) {
                const kk::u32x4_a4 b = kk::load_u32x4(reinterpret_cast<const uint32_t *>(brow + kk0));
                bf[t] = int32x4{static_cast<int>(b.x), static_cast<int>(b.y), static_cast<int>(b.z), static_cast<int>(b.w)};
            } else {
                bf[t] = int32x4{0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                if (ok && 16 * i + lr < rows) {
                    const kk::u32x4_a4 a = kk::load_u32x4(reinterpret_cast<const uint32_t *>(arow[i] + kk0));
                    af[t][i] = int32x4{static_cast<int>(a.x), static_cast<int>(a.y), static_cast<int>(a.z), static_cast<int>(a.w)};
                } else {
                    af[t][i] = int32x4{0, 0, 0, 0};
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kChunk; ++t) {
            const int32x4 b = to_mfma_lane(bf[t]);
#pragma unroll
            for (int i = 0; i < MT; ++i)
                acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(to_mfma_lane(af[t][i]), b, acc[i], 0, 0, 0);
        }
    }
    if (wid > 0) {
#pragma unroll
        for (int i = 0; i < MT; ++i) part[wid - 1][i][lane] = acc[i];
    }
    __syncthreads();
    if (wid > 0) return;
#pragma unroll 3
    for (int v = 0; v < GW - 1; ++v)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[i] += part[v][i][lane];

    // D rows 4g + j of row tile i, weight row n0 + c: (q0, q1) of batch rows
    // 8i + 2g and 8i + 2g + 1
    const int r = n0 + c;
    if (r >= n) return;
    const float scale0 = final_max[0] / 127.0f;
    const float scale1 = final_max[1] / 127.0f;
    const float wmax = maxima[0] / 127.0f;
    const float rs = scales[r];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int b = 8 * i + 2 * g + h;
            if (b < batch)
                y[static_cast<size_t>(b) * n + r] = combine(acc[i][2 * h], acc[i][2 * h + 1], wmax, scale0, scale1, rs);
        }
}

// Batch 1..8 with batch * K <= 16384: the quantization and the product in one
// launch. Every workgroup quantizes X itself (the single-workgroup pass's
// arithmetic, X in registers) into an LDS code table, rows padded by 16 bytes
// so the 16 MFMA rows read distinct banks, then runs the K-split product of
// i8_gemv_ksplit<1> with A read from LDS.
constexpr int kFusedGemvCount = 16384;
template <int WAVES>
__global__ __launch_bounds__(WAVES * kWave) void i8_gemv_fused(const float *__restrict__ x,
                                                                   const int8_t *__restrict__ w,
                                                                   const float *__restrict__ scales,
                                                                   const float *__restrict__ maxima,
                                                                   float *__restrict__ y, int k, int n, int batch,
                                                                   int *status) {
    constexpr int kThreadsF = WAVES * kWave;
    constexpr int kFusedGemvGroups = kFusedGemvCount / 4 / kThreadsF;   // float4 per thread
    __shared__ float scratch[WAVES];
    __shared__ __align__(16) int8_t table[2 * kFusedGemvCount + 16 * 16];   // [2 batch][k + 16]
    __shared__ int32x4 part[WAVES - 1][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int rows = 2 * batch;
    const int stride = k + 16;
    const int groups4 = batch * k / 4;
    const int n0 = blockIdx.x * 16;
    const int steps = (k + 63) / 64;
    const int per = (steps + WAVES - 1) / WAVES;
    const int s0 = wid * per, s1 = min(steps, s0 + per);
    const int8_t *brow = w + static_cast<size_t>(min(n0 + c, n - 1)) * k;
    constexpr int kChunk = 8;
    // branch-free (clamped address, zeroed after the load), so that the
    // memory-counter waits stay exact and the chunk stays in flight across the
    // quantization below
    auto load_b = [&](int sc, int32x4 (&bf)[kChunk]) {
#pragma unroll
        for (int t = 0; t < kChunk; ++t) {
            const int kk0 = (sc + t) * 64 + 16 * g;
            const bool live = sc + t < s1 && kk0 < k;
            const kk::u32x4_a4 b = kk::load_u32x4(reinterpret_cast<const uint32_t *>(brow + min(kk0, k - 16)));
            bf[t] = live ? int32x4{static_cast<int>(b.x), static_cast<int>(b.y), static_cast<int>(b.z), static_cast<int>(b.w)}
                         : int32x4{0, 0, 0, 0};
        }
    };

    // 1. two-pass quantization (reference src/k200.cpp:212-225); the X loads
    // go first, then the wave's first weight chunk, which stays in flight
    // while X is quantized (the memory counter is in order)
    float4 v[kFusedGemvGroups];
#pragma unroll
    for (int t = 0; t < kFusedGemvGroups; ++t) {
        const int q = static_cast<int>(threadIdx.x) + kThreadsF * t;
        v[t] = load_x4(x, min(q, groups4 - 1));   // branch-free, as the weight loads; slots past X unused
    }
    __builtin_amdgcn_sched_barrier(0);
    int32x4 bf[kChunk];
    load_b(s0, bf);
    __builtin_amdgcn_sched_barrier(0);
    float m = 0.0f;
    bool bad = false;
#pragma unroll
    for (int t = 0; t < kFusedGemvGroups; ++t) {
        const bool in_x = static_cast<int>(threadIdx.x) + kThreadsF * t < groups4;
        bad |= in_x && !finite4(v[t]);
        m = fmaxf(m, in_x ? absmax4(v[t]) : 0.0f);
    }
    if (bad) flag_nonfinite(status);
    // the barriers of the quantization wait for LDS only: the weight chunk
    // stays in flight until its MFMAs
    float max0 = block_max<kThreadsF, true>(m, scratch);
    if (max0 == 0.0f) max0 = 1.0f;
    float m1 = 0.0f;
#pragma unroll
    for (int t = 0; t < kFusedGemvGroups; ++t) {
        const int q = static_cast<int>(threadIdx.x) + kThreadsF * t;
        if (q >= groups4) break;
        const int a = quant_primary(v[t].x, max0), b = quant_primary(v[t].y, max0);
        const int cc = quant_primary(v[t].z, max0), d = quant_primary(v[t].w, max0);
        const int row = 4 * q / k, j = 4 * q - row * k;
        *reinterpret_cast<uint32_t *>(table + (2 * row) * stride + j) = pack_codes(a, b, cc, d);
        m1 = fmaxf(m1, fmaxf(fmaxf(fabsf(residual_of(v[t].x, a, max0)), fabsf(residual_of(v[t].y, b, max0))),
                             fmaxf(fabsf(residual_of(v[t].z, cc, max0)), fabsf(residual_of(v[t].w, d, max0)))));
    }
    float max1 = block_max<kThreadsF, true>(m1, scratch);
    if (max1 == 0.0f) max1 = 1.0f;
#pragma unroll
    for (int t = 0; t < kFusedGemvGroups; ++t) {
        const int q = static_cast<int>(threadIdx.x) + kThreadsF * t;
        if (q >= groups4) break;
        auto q1 = [&](float value) { return quant_residual(residual_of(value, quant_primary(value, max0), max0), max1); };
        const int row = 4 * q / k, j = 4 * q - row * k;
        *reinterpret_cast<uint32_t *>(table + (2 * row + 1) * stride + j) =
            pack_codes(q1(v[t].x), q1(v[t].y), q1(v[t].z), q1(v[t].w));
    }
    kk::lds_barrier();

    // 2. K-split int8 MFMA product (A from the table)
    const int8_t *arow = table + (c < rows ? c : 0) * stride;
    int32x4 acc = {0, 0, 0, 0};
    for (int sc = s0; sc < s1; sc += kChunk) {
        if (sc != s0) load_b(sc, bf);
#pragma unroll
        for (int t = 0; t < kChunk; ++t) {
            const int kk0 = (sc + t) * 64 + 16 * g;
            const int32x4 af = sc + t < s1 && kk0 < k && c < rows ? *reinterpret_cast<const int32x4 *>(arow + kk0)
                                                                  : int32x4{0, 0, 0, 0};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[t], acc, 0, 0, 0);
        }
    }
    if (wid > 0) part[wid - 1][lane] = acc;
    __syncthreads();
    if (wid > 0) return;
#pragma unroll
    for (int vv = 0; vv < WAVES - 1; ++vv) acc += part[vv][lane];
    const int r = n0 + c;
    if (r >= n) return;
    const float scale0 = max0 / 127.0f;
    const float scale1 = max1 / 127.0f;
    const float wmax = maxima[0] / 127.0f;
    const float rs = scales[r];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int b = 2 * g + h;
        if (b < batch) y[static_cast<size_t>(b) * n + r] = combine(acc[2 * h], acc[2 * h + 1], wmax, scale0, scale1, rs);
    }
}

// ---------------------------------------------------------------------------
// Batch-1 rowwise_i8 GEMV for K <= 1024 * CH (K % 32 == 0). A workgroup of 8
// waves
//  1. issues the loads of X (8 values per thread), then those of each
//     wave's R weight rows at most (a row is CH fully coalesced 1 KB loads:
//     lane l reads bytes 1024 i + 16 l);
//  2. quantizes X in the reference's two passes (reference
//     src/k200.cpp:212-225) with workgroup maxima into an LDS code table;
//     its barriers wait for LDS only, so the weights stay in flight;
//  3. per wave and row: int32 dot products of the row's bytes with the
//     lane's codes (read once from the table, v_dot4_i32_i8), wave sums and
//     the combine (reference kernels/kunlun-combine.xpu:10-19). The int32
//     sums are exact in any order, so Y equals the MFMA routes' bit for bit.
// All global loads are branch-free (clamped addresses; code slots past K are
// zero, rows past the wave's own are dropped).
__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, kWave);
    return v;
}

constexpr int kRowsThreads = 512;
constexpr int kRowsWaves = kRowsThreads / kWave;

template <int CH, int R>
__global__ __launch_bounds__(kRowsThreads) void i8_gemv_rows(const float *__restrict__ x,
                                                             const int8_t *__restrict__ w,
                                                             const float *__restrict__ scales,
                                                             const float *__restrict__ maxima,
                                                             float *__restrict__ y, int k, int n, int rows_base,
                                                             int rows_rem, int *status) {
    static_assert(CH * 1024 <= 8 * kRowsThreads, "X: 8 values per thread");
    __shared__ float scratch[kRowsWaves];
    __shared__ __align__(16) uint32_t codes[2][CH * 256];   // q0, q1 rows of CH KiB
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = blockIdx.x * kRowsWaves + (threadIdx.x >> 6);
    const int r_begin = wave * rows_base + min(wave, rows_rem);
    const int rows = rows_base + (wave < rows_rem ? 1 : 0);     // 0 .. R
    // 1. activations (thread t: values 8t .. 8t+7), then the weight rows: loads
    //    return in issue order, so X arrives first and is quantized while the
    //    rows are still in flight
    const int x0 = min(8 * static_cast<int>(threadIdx.x), k - 8);
    const float4 xa = load_x4(x + x0, 0), xb = load_x4(x + x0, 1);
    __builtin_amdgcn_sched_barrier(0);
    kk::u32x4_a4 wv[R][CH];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int r = max(0, min(r_begin + min(j, rows - 1), n - 1));
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int off = min(1024 * i + 16 * lane, k - 16);
            wv[j][i] = kk::load_u32x4_stream(reinterpret_cast<const uint32_t *>(w + static_cast<size_t>(r) * k + off));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const bool in_k = 8 * static_cast<int>(threadIdx.x) < k;
    float v[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    // 2. two-pass quantization, workgroup maxima over LDS-only barriers
    float m = 0.0f;
    bool bad = false;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        v[t] = in_k ? v[t] : 0.0f;
        bad |= !isfinite(v[t]);
        m = fmaxf(m, fabsf(v[t]));
    }
    if (bad) flag_nonfinite(status);
    float max0 = block_max<kRowsThreads, true>(m, scratch);
    if (max0 == 0.0f) max0 = 1.0f;
    int q0[8];
    float m1 = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        q0[t] = quant_primary(v[t], max0);
        v[t] = residual_of(v[t], q0[t], max0);
        m1 = fmaxf(m1, fabsf(v[t]));
    }
    float max1 = block_max<kRowsThreads, true>(m1, scratch);
    if (max1 == 0.0f) max1 = 1.0f;
    if (2 * static_cast<int>(threadIdx.x) < CH * 256) {           // code dwords 2t, 2t+1 (zero past K)
        codes[0][2 * threadIdx.x] = pack_codes(q0[0], q0[1], q0[2], q0[3]);
        codes[0][2 * threadIdx.x + 1] = pack_codes(q0[4], q0[5], q0[6], q0[7]);
        codes[1][2 * threadIdx.x] = pack_codes(quant_residual(v[0], max1), quant_residual(v[1], max1),
                                               quant_residual(v[2], max1), quant_residual(v[3], max1));
        codes[1][2 * threadIdx.x + 1] = pack_codes(quant_residual(v[4], max1), quant_residual(v[5], max1),
                                                   quant_residual(v[6], max1), quant_residual(v[7], max1));
    }
    kk::lds_barrier();
    // 3. the lane's codes (16 per chunk and component), then the rows
    uint4 c0[CH], c1[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        c0[i] = *reinterpret_cast<const uint4 *>(&codes[0][256 * i + 4 * lane]);
        c1[i] = *reinterpret_cast<const uint4 *>(&codes[1][256 * i + 4 * lane]);
    }
    const float scale0 = max0 / 127.0f;
    const float scale1 = max1 / 127.0f;
    const float wmax = maxima[0] / 127.0f;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        int p = 0, q = 0;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const bool live = 1024 * i + 16 * lane < k;         // clamped slots: zero codes already, weights not
            const uint32_t a0 = live ? c0[i].x : 0u, a1 = live ? c0[i].y : 0u, a2 = live ? c0[i].z : 0u,
                           a3 = live ? c0[i].w : 0u;
            const uint32_t b0 = live ? c1[i].x : 0u, b1 = live ? c1[i].y : 0u, b2 = live ? c1[i].z : 0u,
                           b3 = live ? c1[i].w : 0u;
            p = __builtin_amdgcn_sdot4(static_cast<int>(wv[j][i][0]), static_cast<int>(a0), p, false);
            p = __builtin_amdgcn_sdot4(static_cast<int>(wv[j][i][1]), static_cast<int>(a1), p, false);
            p = __builtin_amdgcn_sdot4(static_cast<int>(wv[j][i][2]), static_cast<int>(a2), p, false);
            p = __builtin_amdgcn_sdot4(static_cast<int>(wv[j][i][3]), static_cast<int>(a3), p, false);
            q = __builtin_amdgcn_sdot4(static_cast<int>(wv[j][i][0]), static_cast<int>(b0), q, false);
            q = __builtin_amdgcn_sdot4(static_cast<int>(wv[j][i][1]), static_cast<int>(b1), q, false);
            q = __builtin_amdgcn_sdot4(static_cast<int>(wv[j][i][2]), static_cast<int>(b2), q, false);
            q = __builtin_amdgcn_sdot4(static_cast<int>(wv[j][i][3]), static_cast<int>(b3), q, false);
        }
        p = wave_sum_int(p);
        q = wave_sum_int(q);
        const int r = r_begin + j;
        if (lane == 0 && j < rows && r < n) y[r] = combine(p, q, wmax, scale0, scale1, scales[r]);
    }
}

template <int CH, int R>
hipError_t launch_i8_rows(const float *x, const int8_t *w, const float *scales, const float *maxima, float *y, int k,
                          int n, int waves, int *status, hipStream_t stream) {
    const int groups = (waves + kRowsWaves - 1) / kRowsWaves;
    const int all = groups * kRowsWaves;                        // every wave of the grid takes rows
    const int rows_base = n / all, rows_rem = n % all;
    if (rows_base + (rows_rem ? 1 : 0) > R) return hipErrorInvalidValue;
    hipLaunchKernelGGL((i8_gemv_rows<CH, R>), dim3(groups), dim3(kRowsThreads), 0, stream, x, w, scales, maxima, y, k,
                       n, rows_base, rows_rem, status);
    return hipGetLastError();
}

// Batch > 64, K % 128 == 0: LDS-staged int8 GEMM. Workgroup tile: 128 code
// rows (64 batch rows) x 128 weight rows; 16 waves = 2 k-groups x (2 x 4)
// wave tiles of 64 x 32 (four waves per SIMD: at 2 x 2 tiles of 64 x 64,
// two per SIMD, K4096 x N4096 at batch 512 took 43.0-44.9 us per call
// against 40.9-41.2). A stage is 128 K: k-group h takes the stage's 64-K
// step h. Both operands arrive by buffer_load_dwordx4 ... lds (1 KB of LDS per
// wave instruction, no registers), three stages ahead into a ring of four.
// LDS rows are 128 B (8 chunks of 16 B); chunk ch of row r sits at position
// ch ^ ((r >> 1) & 7), so the 16 rows of an MFMA operand (row pairs share a
// 256-byte bank period) read 16 distinct bank groups.
constexpr int kIgRows = 128;                  // code rows and weight rows per tile
constexpr int kIgK = 128;                     // K per stage
constexpr int kIgSlots = 4;
constexpr int kIgOpBytes = kIgRows * kIgK;    // 16 KiB per operand and stage
constexpr int kIgStageBytes = 2 * kIgOpBytes;
constexpr int kIgLdsBytes = kIgSlots * kIgStageBytes;   // 128 KiB
static_assert(kIgLdsBytes >= 4 * 64 * 64 * 4 && kIgLdsBytes <= 160 * 1024, "ring also holds the k-group sums");

// vmcnt(copies per stage * stages_after), stages_after 0..2
template <int CPW>
__device__ __forceinline__ void ig_wait(int stages_after) {
    if (stages_after <= 0) __builtin_amdgcn_s_waitcnt(0x0F70);
    else if (stages_after == 1) __builtin_amdgcn_s_waitcnt(0x0F70 | CPW);
    else __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * CPW));
}

// Stage s's copies of wave `wid` of W waves: A copies wid + W t and B copies
// wid + W t (copy i: rows 8i .. 8i+7 of the tile, lane -> row 8i + l/8,
// position l % 8). (A separate function: the host pass rejects a kernel-local
// lambda that hands captured values to these builtins.)
template <int W>
__device__ __forceinline__ void ig_copy_stage(const int8_t *a_tile, int a_extent, const int8_t *b_tile, int b_extent,
                                              const uint32_t (&a_off)[16 / W], const uint32_t (&b_off)[16 / W], int wid,
                                              int s) {
    extern __shared__ __align__(16) uint8_t ig_lds[];
    const __amdgpu_buffer_rsrc_t a_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(a_tile), 0, a_extent, 0x00020000);
    const __amdgpu_buffer_rsrc_t b_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(b_tile), 0, b_extent, 0x00020000);
    __attribute__((address_space(3))) uint8_t *buf =
        (__attribute__((address_space(3))) uint8_t *)ig_lds + (s % kIgSlots) * kIgStageBytes;
#pragma unroll
    for (int t = 0; t < 16 / W; ++t) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, buf + (wid + W * t) * 1024, 16, a_off[t], s * kIgK, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, buf + kIgOpBytes + (wid + W * t) * 1024, 16, b_off[t],
                                                 s * kIgK, 0, 0);
    }
}

// CW column waves per k-group and row half: wave tiles of 64 x (128 / CW)
// (CW = 2: 8 waves of 64 x 64; CW = 4: 16 waves of 64 x 32, four per SIMD).
template <int CW>
__global__ __launch_bounds__(256 * CW) void i8_lds_gemm(const int8_t *__restrict__ codes, const int8_t *__restrict__ w,
                                                   const float *__restrict__ scales, const float *__restrict__ maxima,
                                                   const float *__restrict__ final_max, float *__restrict__ y,
                                                   int k, int n, int batch, int m_tiles, int tiles, int tiles_per_xcd) {
    extern __shared__ __align__(16) uint8_t ig_lds[];
    const int bid = blockIdx.x;
    const int tile = (bid % 8) * tiles_per_xcd + bid / 8;       // weight-tile major, contiguous per XCD
    if (tile >= tiles) return;                                  // whole workgroup, before any barrier
    const int nt = tile / m_tiles, mt = tile - nt * m_tiles;
    const int rows = 2 * batch;
    const int m0 = mt * kIgRows, n0 = nt * kIgRows;
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    constexpr int kWaves = 4 * CW, kCopies = 16 / kWaves;      // copies per operand, wave and stage
    constexpr int kWn = 128 / CW, kNt = kWn / 16;              // wave tile columns, 16-column MFMA tiles
    const int kg = wid / (2 * CW), wm = (wid / CW) & 1, wn = wid % CW;
    const int g = lane >> 4, c = lane & 15;

    // copy offsets: lane l of copy i -> tile row 8i + l/8 (clamped to the last
    // real row), chunk (l % 8) ^ ((row >> 1) & 7) of the stage's 128 bytes
    const int a_rows = min(kIgRows, rows - m0), b_rows = min(kIgRows, n - n0);
    const int8_t *a_tile = codes + static_cast<size_t>(m0) * k;
    const int8_t *b_tile = w + static_cast<size_t>(n0) * k;
    uint32_t a_off[kCopies], b_off[kCopies];
#pragma unroll
    for (int t = 0; t < kCopies; ++t) {
        const int row = 8 * (wid + kWaves * t) + (lane >> 3);
        const int chunk = (lane & 7) ^ ((row >> 1) & 7);
        a_off[t] = static_cast<uint32_t>(min(row, a_rows - 1)) * k + 16 * chunk;
        b_off[t] = static_cast<uint32_t>(min(row, b_rows - 1)) * k + 16 * chunk;
    }
    const int a_extent = a_rows * k, b_extent = b_rows * k;
    const int stages = k / kIgK;

    int32x4 acc[4][kNt];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kNt; ++j) acc[i][j] = int32x4{0, 0, 0, 0};

    const int ahead0 = min(kIgSlots - 1, stages);
    for (int s = 0; s < ahead0; ++s) ig_copy_stage<kWaves>(a_tile, a_extent, b_tile, b_extent, a_off, b_off, wid, s);
    for (int s = 0; s < stages; ++s) {
        ig_wait<2 * kCopies>(min(kIgSlots - 2, stages - 1 - s));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        if (s + kIgSlots - 1 < stages)
            ig_copy_stage<kWaves>(a_tile, a_extent, b_tile, b_extent, a_off, b_off, wid, s + kIgSlots - 1);
        const uint8_t *abuf = ig_lds + (s % kIgSlots) * kIgStageBytes;
        const uint8_t *bbuf = abuf + kIgOpBytes;
        // k-group kg: step kg of the stage, chunks 4 kg + g of each row
        int32x4 af[4], bf[kNt];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ra = wm * 64 + i * 16 + c;
            af[i] = *reinterpret_cast<const int32x4 *>(abuf + ra * kIgK + (((4 * kg + g) ^ ((ra >> 1) & 7)) * 16));
        }
#pragma unroll
        for (int j = 0; j < kNt; ++j) {
            const int rb = wn * kWn + j * 16 + c;
            bf[j] = *reinterpret_cast<const int32x4 *>(bbuf + rb * kIgK + (((4 * kg + g) ^ ((rb >> 1) & 7)) * 16));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < kNt; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }

    // k-group 1 hands its sums to k-group 0 (exact int32 adds), which combines
    __syncthreads();                                            // every copy landed (last wait: all), ring idle
    int32x4 *xfer = reinterpret_cast<int32x4 *>(ig_lds) + (wid % (2 * CW)) * 4 * kNt * kWave;
    if (kg == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < kNt; ++j) xfer[(i * kNt + j) * kWave + lane] = acc[i][j];
    }
    __syncthreads();
    if (kg == 1) return;
    const float scale0 = final_max[0] / 127.0f;
    const float scale1 = final_max[1] / 127.0f;
    const float wmax = maxima[0] / 127.0f;
#pragma unroll
    for (int j = 0; j < kNt; ++j) {
        const int r = n0 + wn * kWn + j * 16 + c;
        if (r >= n) continue;
        const float rs = scales[r];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int32x4 d = acc[i][j] + xfer[(i * kNt + j) * kWave + lane];
            // D rows 4g .. 4g+3 of row tile i: (q0, q1) of two batch rows
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int b = (m0 + wm * 64 + i * 16 + 4 * g) / 2 + h;
                if (b < batch) y[static_cast<size_t>(b) * n + r] = combine(d[2 * h], d[2 * h + 1], wmax, scale0, scale1, rs);
            }
        }
    }
}

template <int MT, int NT>
hipError_t launch_i8(const int8_t *codes, const int8_t *w, const float *scales, const float *maxima,
                     const float *final_max, float *y, int k, int n, int batch, hipStream_t stream) {
    const int m_tiles = (2 * batch + 15) / 16;
    const int n_tiles = (n + 15) / 16;
    const long long waves = static_cast<long long>((m_tiles + MT - 1) / MT) * ((n_tiles + NT - 1) / NT);
    const int groups = static_cast<int>((waves + 3) / 4);
    hipLaunchKernelGGL((i8_mfma_matmul<MT, NT>), dim3(groups), dim3(256), 0, stream, codes, w, scales, maxima,
                       final_max, y, k, n, batch, m_tiles, n_tiles);
    return hipGetLastError();
}

} // namespace

extern "C" size_t kk_i8_workspace_bytes(int k, int batch) {
    return align256(static_cast<size_t>(2) * batch * k) + (2 * kMaxGroups + 64) * sizeof(float);
}

extern "C" int kk_i8_quantize(const float *x, int k, int batch, void *workspace, int *status, hipStream_t stream) {
    if (!x || !workspace || !status || k <= 0 || batch <= 0) return hipErrorInvalidValue;
    const Workspace ws = layout(workspace, k, batch);
    const size_t count = static_cast<size_t>(k) * batch;
    const size_t fused_limit = std::min<size_t>(static_cast<size_t>(kk::tuning_or(kk::kI8FusedQuantLimit, kFusedQuantDefault)),
                                                4 * kFusedThreads * kFusedGroups);
    if (count <= fused_limit) {
        hipLaunchKernelGGL(i8_quantize_fused, dim3(1), dim3(kFusedThreads), 0, stream, x, count, k, ws.codes,
                           ws.final_max, status);
        return hipGetLastError();
    }
    // one group of 4 values per thread where X allows; past kMaxGroups
    // workgroups, 2 or 4 groups per thread and round
    const size_t groups4 = count / 4;
    const int groups = static_cast<int>(std::min<size_t>(kMaxGroups, (groups4 + kQuantThreads - 1) / kQuantThreads));
    const size_t per_thread = (groups4 + static_cast<size_t>(groups) * kQuantThreads - 1) /
                              (static_cast<size_t>(groups) * kQuantThreads);
    if (per_thread <= 1) launch_passes<1>(x, count, k, groups, ws, status, stream);
    else if (per_thread <= 2) launch_passes<2>(x, count, k, groups, ws, status, stream);
    else launch_passes<4>(x, count, k, groups, ws, status, stream);
    return hipGetLastError();
}

extern "C" int kk_i8_matmul(const void *workspace, const int8_t *w, const float *scales, const float *maxima,
                            float *y, int k, int n, int batch, hipStream_t stream, const char **route) {
    if (!workspace || !w || !scales || !maxima || !y || k <= 0 || (k & 31) || n <= 0 || batch <= 0)
        return hipErrorInvalidValue;
    const Workspace ws = layout(const_cast<void *>(workspace), k, batch);
    if (batch <= 64) {
        if (route) *route = batch <= 8 ? "i8_mfma_gemv" : "i8_mfma_gemm";
        const dim3 grid((n + 15) / 16), block(kGemvWaves * kWave);
        if (batch <= 8)
            hipLaunchKernelGGL(i8_gemv_ksplit<1>, grid, block, 0, stream, ws.codes, w, scales, maxima, ws.final_max, y,
                               k, n, batch);
        else if (batch <= 16)
            hipLaunchKernelGGL(i8_gemv_ksplit<2>, grid, block, 0, stream, ws.codes, w, scales, maxima, ws.final_max, y,
                               k, n, batch);
        else if (batch <= 32)   // 16 waves (K4096 x N4096 at batch 32: 22.5-23.0 us per call against 24.1-24.4 with 8)
            hipLaunchKernelGGL((i8_gemv_ksplit<4, 16>), grid, dim3(16 * kWave), 0, stream, ws.codes, w, scales, maxima,
                               ws.final_max, y, k, n, batch);
        else
            hipLaunchKernelGGL(i8_gemv_ksplit<8>, grid, block, 0, stream, ws.codes, w, scales, maxima, ws.final_max, y,
                               k, n, batch);
        return hipGetLastError();
    }
    if (route) *route = "i8_mfma_gemm";
    if (k % kIgK == 0 && static_cast<long long>(2 * batch) * k <= 0x7fffffffLL &&
        static_cast<long long>(n) * k <= 0x7fffffffLL) {
        const int m_tiles = (2 * batch + kIgRows - 1) / kIgRows;
        const int tiles = m_tiles * ((n + kIgRows - 1) / kIgRows);
        const int tiles_per_xcd = (tiles + 7) / 8;
        const hipError_t rc = kk::opt_in_lds(reinterpret_cast<const void *>(&i8_lds_gemm<4>), kIgLdsBytes);
        if (rc != hipSuccess) return rc;
        hipLaunchKernelGGL(i8_lds_gemm<4>, dim3(tiles_per_xcd * 8), dim3(1024), kIgLdsBytes, stream, ws.codes, w,
                           scales, maxima, ws.final_max, y, k, n, batch, m_tiles, tiles, tiles_per_xcd);
        return hipGetLastError();
    }
    return launch_i8<4, 4>(ws.codes, w, scales, maxima, ws.final_max, y, k, n, batch, stream);
}

extern "C" int kk_i8_gemv_rows_supported(int k, int batch) {
    return batch == 1 && k >= 32 && (k % 32) == 0 && k <= 4096;
}

// Waves: 8 per CU (measured at K4096 x N4096: 6.3 us; 16 and 32 per CU with
// one row each: 6.8 and 6.9 us), more when a wave would own more than 4 rows;
// 2 rows in flight per wave where that covers them.
extern "C" int kk_i8_gemv_rows(const float *x, const int8_t *w, const float *scales, const float *maxima, float *y,
                               int k, int n, int cus, int *status, hipStream_t stream) {
    if (!x || !w || !scales || !maxima || !y || !status || n <= 0 || cus <= 0 || !kk_i8_gemv_rows_supported(k, 1))
        return hipErrorInvalidValue;
    const int waves = static_cast<int>(std::min<long long>(n, std::max<long long>(static_cast<long long>(cus) * 8,
                                                                                  (n + 3) / 4)));
    const int per_wave = (n + waves - 1) / waves;
    const int ch = (k + 1023) / 1024;
#define KK_I8_ROWS(CH)                                                                                   \
    if (ch <= CH) return per_wave <= 2 ? launch_i8_rows<CH, 2>(x, w, scales, maxima, y, k, n, waves, status, stream) \
                                       : launch_i8_rows<CH, 4>(x, w, scales, maxima, y, k, n, waves, status, stream);
    KK_I8_ROWS(1)
    KK_I8_ROWS(2)
    KK_I8_ROWS(4)
#undef KK_I8_ROWS
    return hipErrorInvalidValue;
}

extern "C" int kk_i8_gemv_fused_supported(int k, int batch) {
    return k > 0 && (k % 32) == 0 && batch >= 1 && batch <= 8 && static_cast<long long>(batch) * k <= kFusedGemvCount;
}

extern "C" int kk_i8_gemv_fused(const float *x, const int8_t *w, const float *scales, const float *maxima, float *y,
                                int k, int n, int batch, int *status, hipStream_t stream) {
    if (!x || !w || !scales || !maxima || !y || !status || n <= 0 || !kk_i8_gemv_fused_supported(k, batch))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(i8_gemv_fused<kGemvWaves>, dim3((n + 15) / 16), dim3(kGemvWaves * kWave), 0, stream, x, w,
                       scales, maxima, y, k, n, batch, status);
    return hipGetLastError();
}
