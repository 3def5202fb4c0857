// Small-batch (2..16) Q4_0 GEMV on gfx950 fp16 MFMA, one pass over the
// weights for the whole batch.
//
// Y[b, r] = sum_k X[b, k] * W[r, k]  (reference kernels/kunlun-matvec.xpu:24-79,
// which re-reads W once per batch column). HBM-bound: every weight byte is
// read once per call, like the batch-1 GEMV.
//
// Per 32-value Q4_0 block, one v_mfma_f32_16x16x32_f16 pair computes the
// block sums S[m][r] = sum_k X[m][k] * (q[r][k] - 8) for 16 batch rows (A) by
// 16 weight rows (B); the block's F16 scale d[r] then scales them in F32:
// acc += d * S. The weights enter as exact fp16 (q - 8) (magic-number
// decode), and each activation row as fp16 hi + lo of x * 2^s_m, a per-row
// power of two with max |x * 2^s_m| < 2^14: |x*2^s - hi - lo| <= 2^-22
// |x*2^s| (about the F32 input precision), so the only other rounding is the
// F32 accumulation.
//
// Data flow: a prepass (x_to_frag) writes the activations as MFMA A
// fragments [block][hi|lo][lane][8 halves] in the weight nibble order (block
// position 8g + t of lane group g holds value (4g, 4g+2, 4g+1, 4g+3, 16+4g,
// 16+4g+2, 16+4g+1, 16+4g+3)[t], the order a nibble dword decodes to). The
// GEMV workgroup (4 waves, one 16-row weight tile per wave) walks K in
// chunks of 16 blocks: the chunk's A fragments (32 KiB, shared by the four
// waves, from L2) arrive one chunk ahead and each wave's raw 18-byte weight
// blocks (16 rows x 288 B, padded rows, from HBM) three chunks ahead, by
// direct global -> LDS copies; each lane then reads its nibble dword and
// scale.
#include "device_common.h"
#include "launch.h"
#include "lds_opt_in.h"
#include "tuning.h"

#include <algorithm>

namespace {

using kk::kWave;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBatchRows = 16;                      // MFMA M (batch rows >= batch are zero)
constexpr int kTileRows = 16;                       // MFMA N: weight rows per wave task
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kChunkBlocks = 16;                    // K chunk of 512 values
constexpr int kChunkRowBytes = kChunkBlocks * 18;   // 288 bytes of one weight row per chunk
constexpr int kStageStride = 304;                   // staged row stride: lane reads hit 64 distinct banks
constexpr int kStageBytes = 5 * 1024;               // per wave and buffer: 16 x 304 B rounded to whole 1 KiB copies
constexpr int kFragBlockBytes = 2 * kWave * 16;     // hi and lo A fragments of one block: 2 KiB
constexpr int kChunkFragBytes = kChunkBlocks * kFragBlockBytes;           // 32 KiB
constexpr int kXBuffers = 2;                        // A fragments: one chunk ahead (from L2)
constexpr int kWBuffers = 4;                        // weights: three chunks ahead (from HBM)
constexpr int kWAhead = kWBuffers - 1;
constexpr int kStageSetBytes = kWaves * kStageBytes;                      // one chunk of all four tiles
constexpr int kLdsBytes = kXBuffers * kChunkFragBytes + kWBuffers * kStageSetBytes;   // 144 KiB
constexpr int kWCopies = kStageBytes / 1024;        // 16-byte copies of a full weight chunk per lane
// s_waitcnt with vmcnt = kWCopies (expcnt, lgkmcnt not waited on): the copy
// issued last (weights, kWCopies instructions) may stay in flight
constexpr int kWaitAllButWeights = 0x0F70 | kWCopies;
constexpr int kPrepassThreads = 1024;
static_assert(kTileRows * kStageStride <= kStageBytes, "staged tile fits its copies");
static_assert(kStageStride % 16 == 0 && kChunkRowBytes % 16 == 0, "16-byte copies never straddle a row");

// ---------------------------------------------------------------------------
// Prepass: one workgroup per A row m (16); each thread holds its items' values
// between the max reduction and the stores (one pass over X). Row scale
// s_m = 2^(14 - e), 2^(e-1) <= max|x_m| < 2^e (non-finite or zero rows keep
// s = 1); frag holds blocks_pad blocks (zero beyond k and for rows >= batch).
// PACKED (batch <= 8, 8 workgroups): one fragment per block, A row m holding
// the hi part of batch row m and A row m + 8 its lo part, so one MFMA per
// block computes both and the two halves of D are added at the end.
template <bool PACKED>
__global__ __launch_bounds__(kPrepassThreads) void x_to_frag(const float *__restrict__ x, int batch, int k,
                                                             int blocks_pad, _Float16 *__restrict__ frag,
                                                             float *__restrict__ row_inv) {
    __shared__ float partial[kPrepassThreads / kWave];
    constexpr int kMaxItems = 16384 / 32 * 4 / kPrepassThreads;   // 2: (block, lane group) items per thread
    const int m = blockIdx.x;
    const bool real = m < batch;
    const float *row = x + static_cast<size_t>(real ? m : 0) * k;
    const int blocks = k >> 5;
    float v[kMaxItems][8];
    float mx = 0.0f;
#pragma unroll
    for (int it = 0; it < kMaxItems; ++it) {
        const int item = threadIdx.x + kPrepassThreads * it;
        const int j = item >> 2, g = item & 3;
        if (real && j < blocks) {
            // block positions (4g, 4g+2, 4g+1, 4g+3, 16+4g, 16+4g+2, 16+4g+1, 16+4g+3)
            const float4 lo = *reinterpret_cast<const float4 *>(row + j * 32 + 4 * g);
            const float4 hi = *reinterpret_cast<const float4 *>(row + j * 32 + 16 + 4 * g);
            v[it][0] = lo.x; v[it][1] = lo.z; v[it][2] = lo.y; v[it][3] = lo.w;
            v[it][4] = hi.x; v[it][5] = hi.z; v[it][6] = hi.y; v[it][7] = hi.w;
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) v[it][t] = 0.0f;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) mx = fmaxf(mx, fabsf(v[it][t]));
    }
    mx = kk::wave_max(mx);
    if ((threadIdx.x & (kWave - 1)) == 0) partial[threadIdx.x / kWave] = mx;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPrepassThreads / kWave; ++i) mx = fmaxf(mx, partial[i]);
    int e = __builtin_amdgcn_frexp_expf(mx);
    const bool finite = mx <= 3.402823466e38f && mx > 0.0f;
    e = finite ? max(min(e, 126), -100) : 14;
    const float s = ldexpf(1.0f, 14 - e);
    if (threadIdx.x == 0) row_inv[m] = ldexpf(1.0f, e - 14);
#pragma unroll
    for (int it = 0; it < kMaxItems; ++it) {
        const int item = threadIdx.x + kPrepassThreads * it;
        if (item >= blocks_pad * 4) break;
        const int j = item >> 2, g = item & 3;
        half8 hi, lo;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float a = v[it][t] * s;
            const _Float16 h = static_cast<_Float16>(a);
            hi[t] = h;
            lo[t] = static_cast<_Float16>(a - static_cast<float>(h));
        }
        const int lane = g * kBatchRows + m;
        if constexpr (PACKED) {
            *reinterpret_cast<half8 *>(frag + (static_cast<size_t>(j) * kWave + lane) * 8) = hi;
            *reinterpret_cast<half8 *>(frag + (static_cast<size_t>(j) * kWave + lane + 8) * 8) = lo;
        } else {
            *reinterpret_cast<half8 *>(frag + (static_cast<size_t>(j * 2 + 0) * kWave + lane) * 8) = hi;
            *reinterpret_cast<half8 *>(frag + (static_cast<size_t>(j * 2 + 1) * kWave + lane) * 8) = lo;
        }
    }
}

// ---------------------------------------------------------------------------
// B fragment of lane (row n, group g) from nibble dword g of a block:
// positions (4g, 4g+2, 4g+1, 4g+3, 16+4g, 16+4g+2, 16+4g+1, 16+4g+3), each
// the exact fp16 q - 8.
__device__ __forceinline__ half8 decode_nibbles(uint32_t qs) { return kk::q4_dword_halves(qs); }

// Workgroup barrier without a memory fence. The LDS reads of a wave are
// complete when it reaches the barrier (their values feed the MFMAs before
// it), and the copies a step reads were waited for with s_waitcnt; the asm
// statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

// One block: lane (n, g) reads its scale and nibble dword from the staged row
// (`srow` = row n, `qrow` = row n + 4 g + 2 bytes) and its A fragments.
__device__ __forceinline__ void block_mma(const uint8_t *srow, const uint8_t *qrow, const uint8_t *frow, int j,
                                          float4v &acc) {
    const uint32_t d16 = *reinterpret_cast<const uint16_t *>(srow + 18 * j);
    const uint32_t qs = *reinterpret_cast<const uint16_t *>(qrow + 18 * j) |
                        (static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(qrow + 18 * j + 2)) << 16);
    const half8 bf = decode_nibbles(qs);
    const half8 ahi = *reinterpret_cast<const half8 *>(frow + j * kFragBlockBytes);
    const half8 alo = *reinterpret_cast<const half8 *>(frow + j * kFragBlockBytes + kWave * 16);
    float4v t = {0.0f, 0.0f, 0.0f, 0.0f};
    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bf, t, 0, 0, 0);
    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bf, t, 0, 0, 0);
    const float d = kk::half_bits_to_float(d16);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = fmaf(d, t[r], acc[r]);
}

// kGroup consecutive blocks: all LDS reads first, then the MFMA pairs (one
// independent chain per block), then the scaled accumulation, so the reads'
// latency and the MFMA latency overlap across blocks.
constexpr int kGroup = 8;
__device__ __forceinline__ void block_group(const uint8_t *srow, const uint8_t *qrow, const uint8_t *frow, int j0,
                                            float4v &acc) {
    uint32_t d16[kGroup], qlo[kGroup], qhi[kGroup];
    half8 ahi[kGroup], alo[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
        const int j = j0 + i;
        d16[i] = *reinterpret_cast<const uint16_t *>(srow + 18 * j);
        qlo[i] = *reinterpret_cast<const uint16_t *>(qrow + 18 * j);
        qhi[i] = *reinterpret_cast<const uint16_t *>(qrow + 18 * j + 2);
        ahi[i] = *reinterpret_cast<const half8 *>(frow + j * kFragBlockBytes);
        alo[i] = *reinterpret_cast<const half8 *>(frow + j * kFragBlockBytes + kWave * 16);
    }
    __builtin_amdgcn_sched_barrier(0);   // reads issued in block order, consumed in block order
    float4v t[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
        const half8 bf = decode_nibbles(qlo[i] | (qhi[i] << 16));
        t[i] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
        t[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[i], bf, t[i], 0, 0, 0);
        t[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[i], bf, t[i], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
        const float d = kk::half_bits_to_float(d16[i]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(d, t[i][r], acc[r]);
    }
}

// Workgroup: 4 waves, wave w owns weight tile (base + w) of 16 rows; every
// wave runs every chunk (tiles past the end read a valid tile and store
// nothing), so the barriers are uniform. Chunk c + 1 is copied global -> LDS
// (global_load_lds, no registers) while chunk c is computed.
__global__ __launch_bounds__(kThreads) void q4_mfma_gemv(const uint8_t *__restrict__ w,
                                                        const _Float16 *__restrict__ frag,
                                                        const float *__restrict__ row_inv, float *__restrict__ y,
                                                        int k, int n, int batch, int tiles) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int blocks = k >> 5;
    const size_t row_bytes = static_cast<size_t>(blocks) * 18;      // multiple of 4 (K % 64 == 0)
    const int chunks = (blocks + kChunkBlocks - 1) / kChunkBlocks;
    const int nl = lane & 15, g = lane >> 4;
    const uint8_t *fbytes = reinterpret_cast<const uint8_t *>(frag);
    // the scales of the lane's batch rows 4g .. 4g+3, requested first and first
    // used in the epilogue (unconditional loads: no wait for them before)
    float inv_rows[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) inv_rows[r] = row_inv[min(4 * g + r, batch - 1)];

    for (int base = blockIdx.x * kWaves; base < tiles; base += gridDim.x * kWaves) {
        const int tile = base + wid;
        const int r0 = min(tile, tiles - 1) * kTileRows;
        uint8_t *const xbase = lds;
        uint8_t *const wbase = lds + kXBuffers * kChunkFragBytes;

        // This wave's quarter of chunk c's A fragments (8 x 1 KiB) into X buffer c % 2.
        auto copy_x = [&](int c) {
            c = min(c, chunks - 1);                         // past the end: a copy nobody reads
            uint8_t *xb = xbase + (c & 1) * kChunkFragBytes;
            const uint8_t *fsrc = fbytes + static_cast<size_t>(c) * kChunkFragBytes;
#pragma unroll
            for (int i = 0; i < kChunkFragBytes / (kWaves * 1024); ++i) {
                const int block_kib = i * kWaves + wid;
                __builtin_amdgcn_global_load_lds(fsrc + block_kib * 1024 + lane * 16, xb + block_kib * 1024, 16, 0, 0);
            }
        };
        // This wave's tile rows of chunk c into stage buffer `slot`: the staged
        // [row][304 B] image as 5 x 1 KiB copies (padding lanes and bytes past
        // a row's end copy a dummy in-bounds source and are never read). A
        // partial last chunk copies dwords so that no copy crosses a row's end.
        auto copy_w = [&](int c, int slot) {
            c = min(c, chunks - 1);
            uint8_t *sb = wbase + slot * kStageSetBytes + wid * kStageBytes;
            const int valid = min(kChunkBlocks, blocks - c * kChunkBlocks) * 18;
            const size_t chunk_off = static_cast<size_t>(c) * kChunkRowBytes;
            if (valid == kChunkRowBytes) {
#pragma unroll
                for (int i = 0; i < kWCopies; ++i) {
                    const int p = i * 1024 + lane * 16;
                    const int row = p / kStageStride, col = p - row * kStageStride;
                    const bool in = row < kTileRows && col < kChunkRowBytes;
                    const size_t off = in ? static_cast<size_t>(min(r0 + row, n - 1)) * row_bytes + chunk_off + col : 0;
                    __builtin_amdgcn_global_load_lds(w + off, sb + i * 1024, 16, 0, 0);
                }
            } else {
#pragma unroll
                for (int i = 0; i < kStageBytes / 256; ++i) {
                    const int p = i * 256 + lane * 4;
                    const int row = p / kStageStride, col = p - row * kStageStride;
                    const bool in = row < kTileRows && col + 4 <= valid;
                    const size_t off = in ? static_cast<size_t>(min(r0 + row, n - 1)) * row_bytes + chunk_off + col : 0;
                    __builtin_amdgcn_global_load_lds(w + off, sb + i * 256, 4, 0, 0);
                }
            }
        };

        float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
        // Issue order per step: X (c + 1), then W (c + 3). At the top of step c
        // everything but the last weight copy (chunk c + 2) must have landed,
        // which includes X (c) and W (c); a partial-chunk copy has more
        // instructions, so the wait is then stricter than needed, never looser.
        copy_x(0);
        for (int a = 0; a < kWAhead; ++a) copy_w(a, a);
        for (int c = 0; c < chunks; ++c) {
            if (c == 0) __builtin_amdgcn_s_waitcnt(0);
            else __builtin_amdgcn_s_waitcnt(kWaitAllButWeights);
            // every wave's copies of chunk c landed and its reads of step c - 1
            // are done. A bare s_barrier: a fenced __syncthreads would also wait
            // for the copies still meant to be in flight.
            lds_barrier();
            copy_x(c + 1);
            copy_w(c + kWAhead, (c + kWAhead) % kWBuffers);
            const uint8_t *xb = xbase + (c & 1) * kChunkFragBytes;
            const uint8_t *srow = wbase + (c % kWBuffers) * kStageSetBytes + wid * kStageBytes + nl * kStageStride;
            const uint8_t *qrow = srow + 2 + 4 * g;
            const uint8_t *frow = xb + lane * 16;
            const int nb = min(kChunkBlocks, blocks - c * kChunkBlocks);
            if (nb == kChunkBlocks) {
#pragma unroll
                for (int j0 = 0; j0 < kChunkBlocks; j0 += kGroup) block_group(srow, qrow, frow, j0, acc);
            } else {
                for (int j = 0; j < nb; ++j) block_mma(srow, qrow, frow, j, acc);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);                      // the trailing copies land before
        __syncthreads();                                    // the next tile group reuses the buffers
        // D reg r of lane (n, g): batch row 4g + r, weight row r0 + n
        const int rr = r0 + nl;
        if (tile < tiles && rr < n) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * g + r;
                if (m < batch) y[static_cast<size_t>(m) * n + rr] = acc[r] * inv_rows[r];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// q4_lds_gemv<SB>: the same products, streamed (K % (32 SB) == 0, 16-byte
// aligned weights). A workgroup owns 64 weight rows (four 16-row MFMA tiles);
// its 4 KG waves are KG k-groups x 4 tiles (KG = 4 for 16-block stages: 16
// waves, four per SIMD, so more of each wave's LDS read -> decode -> MFMA
// latency is hidden; KG = 2 for 8-block stages): wave w computes tile w & 3
// over blocks SB/KG (w >> 2) .. +SB/KG-1 of every SB-block stage, and the
// k-groups' sums meet in LDS at the end in a fixed order. Per stage the waves copy the
// stage's A fragments (SB blocks x (hi, lo) = 2 SB KiB, from L2) and the 64
// rows' raw bytes (18 SB B per row as 16-byte chunks, from HBM; consecutive
// lanes take consecutive chunks, so one copy touches a few rows) straight
// into LDS (buffer_load_dwordx4 ... lds; per-lane offsets fixed over stages,
// the stage offset in the SGPR soffset), into a ring of Slots stages, all but
// one ahead. One barrier per stage: SB = 16 halves the barriers of SB = 8 for
// the same LDS (3 x 51 KiB against 6 x 26 KiB). PAD: weight rows sit 18 SB +
// 16 bytes apart in LDS, one empty 16-byte chunk after each row (its copy
// lane reads past the extent: zeros, no memory access; a pair's halves are
// rounded up to whole copies the same way), so the 16 rows a wave reads at
// once spread over the banks (at 18 SB bytes, 288 = 72 dwords for SB = 16,
// bank conflicts took 53% of the LDS-active cycles; K4096 x N14336 at batch
// 16 went from 18.1-18.5 to 17.3-17.4 us per call, the batch-16 gate/up pair
// from 30.0-30.7 to 28.1-28.8 us). A fragments are lane-contiguous.
constexpr int kLgRows = 64;                                  // weight rows per workgroup

template <int SB, bool PACKED, int KG = 2, bool PAD = false, bool PAIR = false>
struct LgShape {
    static_assert(SB == 8 || SB == 16, "stage of 8 or 16 blocks");
    static_assert(KG == 2 || (KG == 4 && SB == 16), "k-groups");
    static constexpr int Waves = 4 * KG;                               // 4 row tiles x KG k-groups
    static constexpr int Threads = 64 * Waves;
    static constexpr int RowStage = SB * 18;                           // bytes of a row per stage
    static constexpr int Slots = SB == 8 ? 6 : PACKED ? 4 : 3;         // ring stages
    static constexpr int ABlockBytes = PACKED ? kFragBlockBytes / 2 : kFragBlockBytes;
    static constexpr int AStageBytes = SB * ABlockBytes;               // 8 / 16 / 32 KiB
    static constexpr int RowStride = PAD ? RowStage + 16 : RowStage;   // bytes of a row in LDS (PAD: one empty chunk)
    // a pair's gate rows (0 .. 31) and up rows (32 .. 63) each fill whole
    // 1 KiB copies: with PAD the halves are rounded up to HalfChunks
    static constexpr int HalfChunks = PAIR && PAD ? ((kLgRows / 2) * (RowStride / 16) + 63) / 64 * 64
                                                  : (kLgRows / 2) * (RowStride / 16);
    static constexpr int BStageBytes = 2 * HalfChunks * 16;            // 9 / 18 KiB (PAD: 10 / 19, pair 20)
    static constexpr int StageBytes = AStageBytes + BStageBytes;
    static constexpr int ACopies = AStageBytes / 1024, BCopies = BStageBytes / 1024;
    static constexpr int ACopiesPerWave = ACopies / Waves;
    static constexpr int BCopiesPerWave = (BCopies + Waves - 1) / Waves;   // waves below BCopies % Waves
    static constexpr int BCopiesRem = BCopies % Waves;                     // issue them all
    static constexpr int WaveBlocks = SB / KG;                         // blocks per wave and stage
    static constexpr int LdsBytes = Slots * StageBytes;                // 102 .. 150 KiB
    static_assert(BCopies * 1024 == BStageBytes && ACopies % Waves == 0 && BCopiesRem != 0, "whole copies");
    static_assert(WaveBlocks % 2 == 0, "block parity follows the wave's block index");
    static_assert(LdsBytes <= 160 * 1024, "LDS");
};

// s_waitcnt vmcnt(n), any n <= 63 (gfx9 keeps vmcnt[5:4] in bits 15:14)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}
__device__ __forceinline__ void wait_vmcnt_dyn(int n) {     // n wave-uniform, 0 .. 16
    switch (n) {
    case 0: wait_vmcnt<0>(); break;   case 1: wait_vmcnt<1>(); break;   case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;   case 4: wait_vmcnt<4>(); break;   case 5: wait_vmcnt<5>(); break;
    case 6: wait_vmcnt<6>(); break;   case 7: wait_vmcnt<7>(); break;   case 8: wait_vmcnt<8>(); break;
    case 9: wait_vmcnt<9>(); break;   case 10: wait_vmcnt<10>(); break; case 11: wait_vmcnt<11>(); break;
    case 12: wait_vmcnt<12>(); break; case 13: wait_vmcnt<13>(); break; case 14: wait_vmcnt<14>(); break;
    case 15: wait_vmcnt<15>(); break; default: wait_vmcnt<16>(); break;
    }
}

// v_and_or_b32 with all operands in VGPRs (a VOP3 takes no literal here)
__device__ __forceinline__ uint32_t lg_and_or(uint32_t a, uint32_t mask, uint32_t bits) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(mask), "v"(bits));
    return r;
}

// One stage's copies of wave `wid`: A copies wid + 8t, weight copies wid + 8t
// (those below BCopies). (A separate function: the host pass rejects a
// kernel-local lambda that hands captured values to these builtins, and then
// drops the launch stub.)
// PAIR: copies below BCopies / 2 come from w_tile (the gate rows), the rest
// from w2_tile (the up rows; b_off relative to it).
template <int SB, bool PACKED, bool PAIR, int KG, bool PAD>
__device__ __forceinline__ void lg_copy_stage(const uint8_t *frag, int frag_bytes, uint8_t *w_tile, int w_extent,
                                              uint8_t *w2_tile, int w2_extent,
                                              const uint32_t (&b_off)[LgShape<SB, PACKED, KG, PAD, PAIR>::BCopiesPerWave],
                                              int wid, int lane, int s) {
    using L = LgShape<SB, PACKED, KG, PAD, PAIR>;
    extern __shared__ __align__(16) uint8_t lg_lds[];
    const __amdgpu_buffer_rsrc_t a_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(frag), 0, frag_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(w_tile, 0, w_extent, 0x00020000);
    __attribute__((address_space(3))) uint8_t *buf =
        (__attribute__((address_space(3))) uint8_t *)lg_lds + (s % L::Slots) * L::StageBytes;
#pragma unroll
    for (int t = 0; t < L::ACopiesPerWave; ++t)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, buf + (wid + L::Waves * t) * 1024, 16,
                                                 (wid + L::Waves * t) * 1024 + lane * 16, s * L::AStageBytes, 0, 0);
#pragma unroll
    for (int t = 0; t < L::BCopiesPerWave; ++t) {
        const int copy = wid + L::Waves * t;                    // wave-uniform
        if (copy >= L::BCopies) continue;
        if (PAIR && copy >= L::BCopies / 2) {
            const __amdgpu_buffer_rsrc_t b2_rsrc = __builtin_amdgcn_make_buffer_rsrc(w2_tile, 0, w2_extent, 0x00020000);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(b2_rsrc, buf + L::AStageBytes + copy * 1024, 16, b_off[t],
                                                     s * L::RowStage, 0, 2);
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, buf + L::AStageBytes + copy * 1024, 16, b_off[t],
                                                     s * L::RowStage, 0, 2);   // non-temporal: read once
        }
    }
}

// PAIR (w2 the up matrix; SB = 16, so each weight copy lies in one half):
// the workgroup's rows 0..31 are rows 32i .. 32i + 31 of w (the gate
// matrix), rows 32..63 the same rows of w2, and y = SiLU(gate) * up
// ([batch][n], kk::swiglu_value) from the gate tiles' waves.
template <int SB, bool PACKED, bool PAIR = false, int KG = 2, bool PAD = false>
__global__ __launch_bounds__(256 * KG) void q4_lds_gemv(const uint8_t *__restrict__ w,
                                                         const uint8_t *__restrict__ w2,
                                                         const _Float16 *__restrict__ frag,
                                                         const float *__restrict__ row_inv, float *__restrict__ y,
                                                         int n, int batch, int stages, uint32_t row_bytes,
                                                         int tiles, int tiles_per_xcd) {
    using L = LgShape<SB, PACKED, KG, PAD, PAIR>;
    static_assert(!PAIR || (L::BCopies % 2 == 0 && (L::BCopies / 2) * 64 == L::HalfChunks),
                  "a pair's weight copies split at the half");
    extern __shared__ __align__(16) uint8_t lg_lds[];
    const int bid = blockIdx.x;
    const int tile = (bid % 8) * tiles_per_xcd + bid / 8;       // contiguous row ranges per XCD
    if (tile >= tiles) return;                                  // whole workgroup, before any barrier
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int kh = wid >> 2, wt = wid & 3;
    const int g = lane >> 4, c16 = lane & 15;
    constexpr int kOutRows = PAIR ? kLgRows / 2 : kLgRows;      // output rows per workgroup
    // the scales of the lane's batch rows 4g .. 4g+3, requested first and first
    // used in the epilogue (unconditional loads: no wait for them before)
    float inv_rows[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) inv_rows[r] = row_inv[min(4 * g + r, batch - 1)];
    const int n0 = tile * kOutRows;

    // weight copy i: 16-byte chunks 64i .. 64i+63 of the stage's [row][RowStage]
    // bytes; rows past n repeat row n - 1 and are never stored
    constexpr int kChunks = L::RowStride / 16;                  // per row: 9 / 18 (PAD: + 1 empty)
    const int w_extent = min(kOutRows, n - n0) * static_cast<int>(row_bytes);
    uint8_t *const w_tile = const_cast<uint8_t *>(w + static_cast<size_t>(n0) * row_bytes);
    uint8_t *const w2_tile = PAIR ? const_cast<uint8_t *>(w2 + static_cast<size_t>(n0) * row_bytes) : nullptr;
    uint32_t b_off[L::BCopiesPerWave];
#pragma unroll
    for (int t = 0; t < L::BCopiesPerWave; ++t) {
        const int q = min(wid + L::Waves * t, L::BCopies - 1) * 64 + lane;
        const int ql = PAIR && q >= L::HalfChunks ? q - L::HalfChunks : q;   // chunk within its matrix's rows
        const int mrow = ql / kChunks, chunk = ql - (ql / kChunks) * kChunks;   // row of its own matrix's tile
        // an empty chunk (PAD), or a pair half's rounding past its 32 rows:
        // past the extent, so zeros without a memory access
        const bool pad = (PAD && chunk == kChunks - 1) || (PAIR && mrow >= kOutRows);
        b_off[t] = pad ? 0x80000000u : static_cast<uint32_t>(min(n0 + mrow, n - 1) - n0) * row_bytes + 16 * chunk;
    }
    const int frag_bytes = stages * L::AStageBytes;
    const uint8_t *fbytes = reinterpret_cast<const uint8_t *>(frag);
    const int my_copies = L::ACopiesPerWave + (wid < L::BCopiesRem ? L::BCopiesPerWave : L::BCopiesPerWave - 1);

    float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t mask_lo = 0x000f000fu, mask_hi = 0x00f000f0u, magic = 0x64006400u;
    asm volatile("" : "+v"(mask_lo), "+v"(mask_hi), "+v"(magic));   // keep them in VGPRs
    const half2v off = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const half2v off72 = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};

    // Stage t's copies are issued at stage t - (Slots - 1) (the prologue
    // issues the first Slots - 1), after that stage's barrier, into buffer
    // t % Slots (stage t - Slots's, which every wave finished before the
    // barrier). At the top of stage s this wave's copies of stages
    // s+1 .. min(s+Slots-2, stages-1) may still be in flight.
    const int ahead0 = min(L::Slots - 1, stages);
    for (int s = 0; s < ahead0; ++s)
        lg_copy_stage<SB, PACKED, PAIR, KG, PAD>(fbytes, frag_bytes, w_tile, w_extent, w2_tile, w_extent, b_off, wid, lane, s);
    for (int s = 0; s < stages; ++s) {
        wait_vmcnt_dyn(my_copies * min(L::Slots - 2, stages - 1 - s));
        lds_barrier();
        if (s + L::Slots - 1 < stages)
            lg_copy_stage<SB, PACKED, PAIR, KG, PAD>(fbytes, frag_bytes, w_tile, w_extent, w2_tile, w_extent, b_off, wid, lane,
                                            s + L::Slots - 1);
        const uint8_t *abuf = lg_lds + (s % L::Slots) * L::StageBytes;
        const int trow = wt * 16 + c16;                         // tile row (PAIR: 0 .. 31 gate, 32 .. 63 up)
        const uint8_t *brow = abuf + L::AStageBytes +
                              (PAIR ? (trow / 32) * L::HalfChunks * 16 + (trow % 32) * L::RowStride : trow * L::RowStride);
        uint32_t qs[L::WaveBlocks], d16[L::WaveBlocks];
        half8 ahi[L::WaveBlocks], alo[L::WaveBlocks];
#pragma unroll
        for (int i = 0; i < L::WaveBlocks; ++i) {
            const int j = L::WaveBlocks * kh + i;               // block of the stage (parity of i)
            d16[i] = *reinterpret_cast<const uint16_t *>(brow + 18 * j);
            if ((i & 1) == 0) {                                 // even block: nibble dword g at +2 + 4g
                const uint32_t *p = reinterpret_cast<const uint32_t *>(brow + 18 * j + 4 * g);
                qs[i] = __builtin_amdgcn_alignbyte(p[1], p[0], 2);
            } else {                                            // odd block: on a dword
                qs[i] = *reinterpret_cast<const uint32_t *>(brow + 18 * j + 2 + 4 * g);
            }
            ahi[i] = *reinterpret_cast<const half8 *>(abuf + j * L::ABlockBytes + lane * 16);
            if (!PACKED) alo[i] = *reinterpret_cast<const half8 *>(abuf + j * L::ABlockBytes + kWave * 16 + lane * 16);
        }
        float4v t[L::WaveBlocks];
#pragma unroll
        for (int i = 0; i < L::WaveBlocks; ++i) {
            // exact fp16 q - 8 of positions (4g, 4g+2, 4g+1, 4g+3, 16+4g, ...):
            // 1024 + q less 1032, and (1024 + 16 q) / 16 less 72
            union { uint32_t u; half2v h; } p0, p1, p2, p3;
            const uint32_t qh = qs[i] >> 8;
            p0.u = lg_and_or(qs[i], mask_lo, magic);
            p1.u = lg_and_or(qh, mask_lo, magic);
            p2.u = lg_and_or(qs[i], mask_hi, magic);
            p3.u = lg_and_or(qh, mask_hi, magic);
            const half2v e0 = p0.h + off, e1 = p1.h + off;
            const half2v e2 = p2.h * sixteenth + off72, e3 = p3.h * sixteenth + off72;
            half8 bf;
            bf[0] = e0[0]; bf[1] = e0[1]; bf[2] = e1[0]; bf[3] = e1[1];
            bf[4] = e2[0]; bf[5] = e2[1]; bf[6] = e3[0]; bf[7] = e3[1];
            t[i] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
            t[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[i], bf, t[i], 0, 0, 0);
            if (!PACKED) t[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[i], bf, t[i], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < L::WaveBlocks; ++i) {
            const float d = kk::half_bits_to_float(d16[i]);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = fmaf(d, t[i][r], acc[r]);
        }
    }

    // k-groups 1 .. KG-1 hand their sums to k-group 0 through LDS (every
    // copy has landed: the last wait was for all of them), which adds them
    // in k-group order
    __syncthreads();
    float4v *xfer = reinterpret_cast<float4v *>(lg_lds);
    if (kh >= 1) xfer[((kh - 1) * 4 + wt) * kWave + lane] = acc;
    __syncthreads();
    if (!PAIR && kh >= 1) return;
#pragma unroll
    for (int h = 1; h < KG; ++h) acc += xfer[((h - 1) * 4 + wt) * kWave + lane];
    if constexpr (PACKED) {
        // D rows 8..15 (lanes 32..63) are the lo parts of batch rows 0..7
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] += __shfl_down(acc[r], 32);
    }
    if constexpr (PAIR) {
        // the up tiles (waves 2, 3 of k-group 0) hand their sums to the gate
        // tiles (waves 0, 1) through LDS; every wave takes part in the barrier
        float4v *upx = xfer + (KG - 1) * 4 * kWave;
        if (kh == 0 && wt >= 2) upx[(wt - 2) * kWave + lane] = acc;
        __syncthreads();
        if (kh >= 1 || wt >= 2 || (PACKED && g >= 2)) return;
        const float4v up = upx[wt * kWave + lane];
        const int rr = n0 + wt * 16 + c16;
        if (rr < n) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 4 * g + r;
                if (m < batch)
                    y[static_cast<size_t>(m) * n + rr] = kk::swiglu_value(acc[r] * inv_rows[r], up[r] * inv_rows[r]);
            }
        }
        return;
    }
    if (PACKED && g >= 2) return;
    // D reg r of lane (c16, g): batch row 4g + r, weight row n0 + 16 wt + c16
    const int rr = n0 + wt * 16 + c16;
    if (rr < n) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            if (m < batch) y[static_cast<size_t>(m) * n + rr] = acc[r] * inv_rows[r];
        }
    }
}

// Launch q4_lds_gemv<SB> (dynamic LDS above 64 KiB opted into once per
// device).
template <int SB, bool PACKED, bool PAIR = false, int KG = 2, bool PAD = false>
hipError_t launch_lds_gemv_kg(const uint8_t *w, const uint8_t *w2, const _Float16 *frag, const float *row_inv, float *y,
                              int k, int n, int batch, hipStream_t stream) {
    using L = LgShape<SB, PACKED, KG, PAD, PAIR>;
    const hipError_t rc =
        kk::opt_in_lds(reinterpret_cast<const void *>(&q4_lds_gemv<SB, PACKED, PAIR, KG, PAD>), L::LdsBytes);
    if (rc != hipSuccess) return rc;
    const int out_rows = PAIR ? kLgRows / 2 : kLgRows;
    const int tiles = (n + out_rows - 1) / out_rows;
    const int tiles_per_xcd = (tiles + 7) / 8;
    hipLaunchKernelGGL((q4_lds_gemv<SB, PACKED, PAIR, KG, PAD>), dim3(tiles_per_xcd * 8), dim3(L::Threads), L::LdsBytes, stream,
                       w, w2, frag, row_inv, y, n, batch, k / (SB * 32), static_cast<uint32_t>(k / 32 * 18), tiles,
                       tiles_per_xcd);
    return hipGetLastError();
}

template <int SB, bool PACKED, bool PAIR = false>
hipError_t launch_lds_gemv(const uint8_t *w, const uint8_t *w2, const _Float16 *frag, const float *row_inv, float *y,
                           int k, int n, int batch, hipStream_t stream) {
    return launch_lds_gemv_kg<SB, PACKED, PAIR, SB == 16 ? 4 : 2, true>(w, w2, frag, row_inv, y, k, n, batch, stream);
}

} // namespace

extern "C" size_t kk_q4_mfma_gemv_workspace_bytes(int k) {
    const int blocks_pad = ((k >> 5) + kChunkBlocks - 1) / kChunkBlocks * kChunkBlocks;
    return static_cast<size_t>(blocks_pad) * kFragBlockBytes + 256;
}

extern "C" int kk_q4_mfma_gemv(const void *w, const float *x, float *y, int k, int n, int batch, void *workspace,
                               int cus, hipStream_t stream) {
    if (!w || !x || !y || !workspace || k <= 0 || (k & 63) || k > 16384 || n <= 0 || batch < 1 ||
        batch > kBatchRows || cus <= 0 || (reinterpret_cast<uintptr_t>(w) & 3))
        return hipErrorInvalidValue;
    const int blocks_pad = ((k >> 5) + kChunkBlocks - 1) / kChunkBlocks * kChunkBlocks;
    _Float16 *frag = static_cast<_Float16 *>(workspace);
    float *row_inv = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                               static_cast<size_t>(blocks_pad) * kFragBlockBytes);
    // streamed kernels: K % 256 == 0 and 16-byte aligned weights; batch <= 8
    // packs hi and lo into one fragment (one MFMA per block)
    const bool streamed = k % 256 == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
    const bool packed = streamed && batch <= kBatchRows / 2;
    if (packed)
        hipLaunchKernelGGL(x_to_frag<true>, dim3(kBatchRows / 2), dim3(kPrepassThreads), 0, stream, x, batch, k,
                           blocks_pad, frag, row_inv);
    else
        hipLaunchKernelGGL(x_to_frag<false>, dim3(kBatchRows), dim3(kPrepassThreads), 0, stream, x, batch, k,
                           blocks_pad, frag, row_inv);
    hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) return rc;
    rc = kk::opt_in_lds(reinterpret_cast<const void *>(&q4_mfma_gemv), kLdsBytes);
    if (rc != hipSuccess) return rc;
    if (streamed) {
        const uint8_t *wb = static_cast<const uint8_t *>(w);
        if (k % 512 == 0)
            return packed ? launch_lds_gemv<16, true>(wb, nullptr, frag, row_inv, y, k, n, batch, stream)
                          : launch_lds_gemv<16, false>(wb, nullptr, frag, row_inv, y, k, n, batch, stream);
        return packed ? launch_lds_gemv<8, true>(wb, nullptr, frag, row_inv, y, k, n, batch, stream)
                      : launch_lds_gemv<8, false>(wb, nullptr, frag, row_inv, y, k, n, batch, stream);
    }
    const int tiles = (n + kTileRows - 1) / kTileRows;
    const int groups = std::max(1, std::min((tiles + kWaves - 1) / kWaves, cus));
    hipLaunchKernelGGL(q4_mfma_gemv, dim3(groups), dim3(kThreads), kLdsBytes, stream, static_cast<const uint8_t *>(w),
                       frag, row_inv, y, k, n, batch, tiles);
    return hipGetLastError();
}

// Gate/up pair on the streamed kernel at K % 512 == 0 (16-byte aligned weights
// and X): one prepass, then both products and SwiGLU in one launch.
extern "C" int kk_q4_mfma_pair_swiglu_supported(const void *w_gate, const void *w_up, const float *x, int k, int n,
                                                int batch) {
    return w_gate && w_up && x && k > 0 && k % 512 == 0 && k <= 16384 && n >= 1 && batch >= 1 &&
           batch <= kBatchRows && (reinterpret_cast<uintptr_t>(w_gate) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(w_up) & 15) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

extern "C" int kk_q4_mfma_gemv_pair_swiglu(const void *w_gate, const void *w_up, const float *x, float *y, int k,
                                           int n, int batch, void *workspace, hipStream_t stream) {
    if (!kk_q4_mfma_pair_swiglu_supported(w_gate, w_up, x, k, n, batch) || !y || !workspace)
        return hipErrorInvalidValue;
    const int blocks_pad = ((k >> 5) + kChunkBlocks - 1) / kChunkBlocks * kChunkBlocks;
    _Float16 *frag = static_cast<_Float16 *>(workspace);
    float *row_inv = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                               static_cast<size_t>(blocks_pad) * kFragBlockBytes);
    const bool packed = batch <= kBatchRows / 2;
    if (packed)
        hipLaunchKernelGGL(x_to_frag<true>, dim3(kBatchRows / 2), dim3(kPrepassThreads), 0, stream, x, batch, k,
                           blocks_pad, frag, row_inv);
    else
        hipLaunchKernelGGL(x_to_frag<false>, dim3(kBatchRows), dim3(kPrepassThreads), 0, stream, x, batch, k,
                           blocks_pad, frag, row_inv);
    const hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) return rc;
    const uint8_t *wg = static_cast<const uint8_t *>(w_gate), *wu = static_cast<const uint8_t *>(w_up);
    return packed ? launch_lds_gemv<16, true, true>(wg, wu, frag, row_inv, y, k, n, batch, stream)
                  : launch_lds_gemv<16, false, true>(wg, wu, frag, row_inv, y, k, n, batch, stream);
}

// ---------------------------------------------------------------------------
// Small-batch (1..16) F32 / F16 GEMV on fp32 MFMA (v_mfma_f32_16x16x4_f32):
// exact F32 products (an F16 weight widens exactly), F32 accumulation, one
// pass over the weights for the whole batch.
//
// Workgroup = one 16-row weight tile; its 8 waves take K eighths (32-value
// steps, 2 in flight per wave) and meet in LDS at the end in wave order.
// Two steps in flight measured fastest (4096 x 4096, F32 batch 8: 15.7 us
// at 2 steps, 17.1 at 3, 18.4 at 4, 21.7 at 1); there a launch is one
// workgroup per CU, each wave with 64 KiB of loads to issue.
// MFMA t (0..7) of a step takes k0 + 8g + t from lane group g (A[m][k] in
// lane m + 16 k, B[k][n] in lane n + 16 k, D[4g + i][n] in lane n + 16 g), so
// lane (n, g) needs weights and activations k0 + 8g .. k0 + 8g + 7 of row n.
// The loads are laid out for the cache instead: lane l reads row l / 4 (and
// batch row l / 4), 16-byte piece 2 (l % 4) of the step in one load and piece
// 2 (l % 4) + 1 in the other (F16: piece l % 4), so each group of 4 lanes
// stays in one cache line (a load whose lanes read 16 different rows costs
// several times more), and ds_bpermute moves lane 4n + g's values to lane
// (n, g): the same values in the same MFMA order.
namespace {

constexpr int kDenseWaves = 8;     // K split over the workgroup's waves (two per SIMD)
constexpr int kDenseDepth = 2;     // 32-value steps of loads in flight per wave

template <bool F16W>
__global__ __launch_bounds__(kWave * kDenseWaves) void dense_mfma_gemv(const uint8_t *__restrict__ w,
                                                                      const float *__restrict__ x,
                                                                      float *__restrict__ y, int k, int n,
                                                                      int batch) {
    __shared__ float4v partial[kDenseWaves][kWave];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int q = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nl = lane & 15, g = lane >> 4;
    const int lr = lane >> 2, lp = lane & 3;                   // loader row and piece pair
    const int r = min(static_cast<int>(blockIdx.x) * 16 + lr, n - 1);
    const bool live_m = lr < batch;
    const float *xrow = x + static_cast<size_t>(min(lr, batch - 1)) * k + 8 * lp;
    const uint8_t *wrow = w + static_cast<size_t>(r) * k * (F16W ? 2 : 4) + (F16W ? 16 : 32) * lp;
    const int src = (4 * nl + g) * 4;                          // lane (n, g) takes loader lane 4n + g
    const int steps = k >> 5;
    const int s0 = steps * q / kDenseWaves, s1 = steps * (q + 1) / kDenseWaves;

    // one step: 8 activations and 8 weights of this lane (a past-the-end step
    // reloads the wave's last step; its MFMAs are skipped)
    // b holds 8 F32 weights, or (F16) 4 dwords of raw halves widened after the move
    auto load = [&](int s, float (&a)[8], float (&b)[8]) {
        s = min(s, max(s1 - 1, s0));
        const float4 *xs = reinterpret_cast<const float4 *>(xrow + static_cast<size_t>(s) * 32);
        const float4 x0 = xs[0], x1 = xs[1];
        a[0] = x0.x; a[1] = x0.y; a[2] = x0.z; a[3] = x0.w; a[4] = x1.x; a[5] = x1.y; a[6] = x1.z; a[7] = x1.w;
#pragma unroll
        for (int t = 0; t < 8; ++t) a[t] = live_m ? a[t] : 0.0f;
        if constexpr (F16W) {
            const uint4 h = *reinterpret_cast<const uint4 *>(wrow + static_cast<size_t>(s) * 64);
            b[0] = __uint_as_float(h.x); b[1] = __uint_as_float(h.y); b[2] = __uint_as_float(h.z); b[3] = __uint_as_float(h.w);
        } else {
            const uint8_t *ws = wrow + static_cast<size_t>(s) * 128;
            const float4 w0 = *reinterpret_cast<const float4 *>(ws), w1 = *reinterpret_cast<const float4 *>(ws + 16);
            b[0] = w0.x; b[1] = w0.y; b[2] = w0.z; b[3] = w0.w; b[4] = w1.x; b[5] = w1.y; b[6] = w1.z; b[7] = w1.w;
        }
    };
    auto to_mfma_layout = [&](float (&a)[8], float (&b)[8]) {
#pragma unroll
        for (int t = 0; t < 8; ++t) a[t] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(a[t])));
        if constexpr (F16W) {
            float wide[8];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t u = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, __float_as_int(b[t])));
                wide[2 * t] = kk::half_bits_to_float(u & 0xffffu);
                wide[2 * t + 1] = kk::half_bits_to_float(u >> 16);
            }
#pragma unroll
            for (int t = 0; t < 8; ++t) b[t] = wide[t];
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) b[t] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(b[t])));
        }
    };

    float4v acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
    float a[kDenseDepth][8], b[kDenseDepth][8];
#pragma unroll
    for (int d = 0; d < kDenseDepth; ++d) load(s0 + d, a[d], b[d]);
    for (int s = s0; s < s1; s += kDenseDepth) {
#pragma unroll
        for (int d = 0; d < kDenseDepth; ++d) {
            if (s + d < s1) {                               // uniform: every lane of the wave agrees
                float ca[8], cb[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) { ca[t] = a[d][t]; cb[t] = b[d][t]; }
                load(s + d + kDenseDepth, a[d], b[d]);
                to_mfma_layout(ca, cb);
#pragma unroll
                for (int t = 0; t < 8; t += 2) {
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(ca[t], cb[t], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(ca[t + 1], cb[t + 1], acc1, 0, 0, 0);
                }
            }
        }
    }
    partial[q][lane] = acc0 + acc1;
    __syncthreads();
    if (q != 0) return;
    float4v sum = partial[0][lane];
#pragma unroll
    for (int i = 1; i < kDenseWaves; ++i) sum += partial[i][lane];
    // D reg i of lane (n, g): batch row 4g + i, weight row tile*16 + n
    const int row = static_cast<int>(blockIdx.x) * 16 + nl;
    if (row < n) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * g + i;
            if (m < batch) y[static_cast<size_t>(m) * n + row] = sum[i];
        }
    }
}

// F16 weights, batch 2..8, K <= 4096: the weights streamed as the batch-1
// GEMV reads them. An item is one 1 KiB chunk (512 values) of one row, so
// every load instruction covers 1 KiB of contiguous row bytes. A workgroup
// owns T 16-row tiles and wave w takes chunk w of every tile row, keeping
// kF16sDepth items in flight. Each arrived item goes into the wave's own LDS
// area (lane l: bytes 16 l .. 16 l + 15, zero past the row end; row stride
// 1040 B), and when a tile's 16 rows are there, lane (n, g) reads 16-byte
// piece 4j + g of row n (conflict-free at that stride): the B operand of
// v_mfma_f32_16x16x32_f16 for K32 slice j of the chunk.
// The A operand, held in registers for the whole launch: row r of it is
// column r of X (r < 8) as the fp16 hi part, and column r - 8 as the lo
// part, of x * 2^s. The power of two 2^s, per column and chunk, brings the
// chunk's max |x| below 2^14, and |x 2^s - hi - lo| <= 2^-22 |x 2^s| + 2^-25
// (the lo part may be an fp16 subnormal).
// fp16 x fp16 products are exact in F32, so D[r][n] are exact products
// summed in F32; the hi and lo rows of a column are added and the sum
// multiplied by 2^-s.
// X is read lane-contiguously (lane l: column l / 8, 16 B at 16 (l % 8)
// within each 128 B of the chunk; lanes that read different rows of X in one
// instruction cost one cache-tag lookup each) and moved into the A layout
// with ds_bpermute: lane (r, g) takes values 8g + 4h .. 8g + 4h + 3 (h = r / 8)
// of column r % 8, converts them to hi and lo, keeps its own half (hi for
// r < 8, lo otherwise) and trades the other with lane r ^ 8 by DPP.
// An F16 weight that is Inf or NaN times a lo part of 0 would give NaN
// where the F32 product gives +-Inf. With finite X the split products stay
// below 2^39 in magnitude, so a tile's sums are all finite exactly when its
// weights are; a tile with a non-finite sum, or whose chunk of X holds a
// non-finite value, is recomputed on an exact path: v_mfma_f32_16x16x4_f32
// on the F32 activations (reloaded) and the widened staged weights, the
// products of dense_mfma_gemv.
// The waves' tile sums meet in LDS and are added in wave order.
constexpr int kF16sWaves = 8;
constexpr int kF16sDepth = 16;
constexpr int kF16sRowStride = 1040;
constexpr int kF16sStageBytes = 16 * kF16sRowStride;
constexpr int kF16sMaxTiles = 4;
constexpr int kF16sLdsBytes = kF16sWaves * kF16sStageBytes + kF16sMaxTiles * kF16sWaves * 32 * 16;

__global__ __launch_bounds__(kWave * kF16sWaves) void f16_stream_gemv(const uint8_t *__restrict__ w,
                                                                     const float *__restrict__ x,
                                                                     float *__restrict__ y, int k, int n, int batch,
                                                                     int tiles_per_group) {
    extern __shared__ __align__(16) uint8_t fs_lds[];
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    constexpr int kXor8 = 0x128;                                  // DPP row_ror:8, lane r ^ 8 within 16
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const bool hi_row = r16 < 8;
    const uint32_t row_bytes = static_cast<uint32_t>(k) * 2;
    const int tiles = (n + 15) / 16;
    const int tile0 = blockIdx.x * tiles_per_group;
    const int items = tiles_per_group * 16;
    const int c = wid;                                           // this wave's chunk
    const int jlive = __builtin_amdgcn_readfirstlane(max(0, min(16, (k - c * 512) / 32)));   // K32 slices in K
    uint8_t *stage = fs_lds + wid * kF16sStageBytes;
    float4v *partial = reinterpret_cast<float4v *>(fs_lds + kF16sWaves * kF16sStageBytes);   // [T][waves][32]

    // 1. X, lane-contiguous: lane l holds values c*512 + 32 j + 4 (l % 8) .. + 3 of column l / 8
    float xv[16][4];
    {
        const int lc = lane >> 3, q = lane & 7;
        const bool lc_live = lc < batch;
        const float *xl = x + static_cast<size_t>(min(lc, batch - 1)) * k;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int k0 = c * 512 + 32 * j + 4 * q;
            const bool live = lc_live && k0 < k;
            const float4 a = *reinterpret_cast<const float4 *>(xl + (live ? k0 : 0));
            xv[j][0] = live ? a.x : 0.0f; xv[j][1] = live ? a.y : 0.0f;
            xv[j][2] = live ? a.z : 0.0f; xv[j][3] = live ? a.w : 0.0f;
        }
    }
    // 2. the first items (issued after X: the memory counter is in order)
    __builtin_amdgcn_sched_barrier(0);
    auto load_item = [&](int item, u32x4 &v) {
        const int it = min(item, items - 1);
        const int i = it & 15, t = it >> 4;
        const int tile = min(tile0 + t, tiles - 1);
        const int r = min(tile * 16 + i, n - 1);
        const uint32_t off = min(static_cast<uint32_t>(c) * 1024u + 16u * lane, row_bytes - 16u);
        v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(w + static_cast<size_t>(r) * row_bytes + off));
    };
    u32x4 ring[kF16sDepth];
#pragma unroll
    for (int d = 0; d < kF16sDepth; ++d) {
        load_item(d, ring[d]);
        __builtin_amdgcn_sched_barrier(0);
    }
    // 3. X into the A layout; the chunk's scale per column; hi/lo fragments
    {
        const int src = ((r16 & 7) * 8 + 2 * g + (r16 >> 3)) * 4;
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
            for (int t = 0; t < 4; ++t)
                xv[j][t] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(xv[j][t])));
    }
    float m = 0.0f, bad = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float a = fabsf(xv[j][t]);
            bad = (a <= 3.402823466e38f) ? bad : 1.0f;
            m = fmaxf(m, a);
        }
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), kXor8, 0xf, 0xf, false)));
    m = fmaxf(m, __shfl_xor(m, 16, kWave));
    m = fmaxf(m, __shfl_xor(m, 32, kWave));
    const bool x_bad = __builtin_amdgcn_ballot_w64(bad != 0.0f) != 0;   // wave-uniform
    const int e = max(min(__builtin_amdgcn_frexp_expf(m), 128), -110);   // m < 2^e; 2^(14-e) and 2^(e-14) stay normal
    const float to_f16 = ldexpf(1.0f, 14 - e);
    const float inv_self = ldexpf(1.0f, e - 14);
    float inv[8];
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) inv[cc] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv_self), cc));
    half8 af[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        half4 hh, ll;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float v = xv[j][t] * to_f16;
            const _Float16 h = static_cast<_Float16>(v);
            hh[t] = h;
            ll[t] = static_cast<_Float16>(v - static_cast<float>(h));
        }
        // hi lanes keep their hi parts and take the partner's (values 4..7); lo lanes the reverse
        const u32x2 send = hi_row ? __builtin_bit_cast(u32x2, ll) : __builtin_bit_cast(u32x2, hh);
        u32x2 recv;
        recv[0] = __builtin_amdgcn_update_dpp(0, static_cast<int>(send[0]), kXor8, 0xf, 0xf, false);
        recv[1] = __builtin_amdgcn_update_dpp(0, static_cast<int>(send[1]), kXor8, 0xf, 0xf, false);
        const half4 other = __builtin_bit_cast(half4, recv);
        const half4 first = hi_row ? hh : other, last = hi_row ? other : ll;   // values 0..3, 4..7
        af[j][0] = first[0]; af[j][1] = first[1]; af[j][2] = first[2]; af[j][3] = first[3];
        af[j][4] = last[0]; af[j][5] = last[1]; af[j][6] = last[2]; af[j][7] = last[3];
    }

    auto tile_compute = [&](int t) {
        float4v d = {0.0f, 0.0f, 0.0f, 0.0f};
        bool tile_bad = x_bad;
        if (!tile_bad) {
            float4v acc[4] = {};
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j < jlive) {
                    const half8 b = *reinterpret_cast<const half8 *>(stage + r16 * kF16sRowStride + (4 * j + g) * 16);
                    acc[j & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[j], b, acc[j & 3], 0, 0, 0);
                }
            const float4v sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            const bool nf = !(fabsf(sum[0]) <= 3.402823466e38f && fabsf(sum[1]) <= 3.402823466e38f &&
                              fabsf(sum[2]) <= 3.402823466e38f && fabsf(sum[3]) <= 3.402823466e38f);
            tile_bad = __builtin_amdgcn_ballot_w64(nf) != 0;               // wave-uniform
            // lane (n, g): g < 2 hold the hi rows of columns 4g .. 4g+3, lane + 32 their lo rows
            float4v lo;
#pragma unroll
            for (int r = 0; r < 4; ++r) lo[r] = __shfl_xor(sum[r], 32, kWave);
#pragma unroll
            for (int r = 0; r < 4; ++r) d[r] = (sum[r] + lo[r]) * inv[(4 * g + r) & 7];
        }
        if (tile_bad) {
            // exact path: F32 activations of column r16 (< 8; rows 8..15 zero)
            const bool live_row = r16 < batch && r16 < 8;
            const float *xr = x + static_cast<size_t>(min(r16, batch - 1)) * k;
            float4v a32[4] = {};
            for (int j = 0; j < jlive; ++j) {
                const int k0 = c * 512 + 32 * j + 8 * g;
                const float4 xa = *reinterpret_cast<const float4 *>(xr + (live_row ? k0 : 0));
                const float4 xb = *reinterpret_cast<const float4 *>(xr + (live_row ? k0 : 0) + 4);
                const float xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                const u32x4 p = *reinterpret_cast<const u32x4 *>(stage + r16 * kF16sRowStride + (4 * j + g) * 16);
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) {
                    a32[(2 * e2) & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        live_row ? xs[2 * e2] : 0.0f, kk::half_bits_to_float(p[e2] & 0xffffu), a32[(2 * e2) & 3], 0, 0, 0);
                    a32[(2 * e2 + 1) & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        live_row ? xs[2 * e2 + 1] : 0.0f, kk::half_bits_to_float(p[e2] >> 16), a32[(2 * e2 + 1) & 3],
                        0, 0, 0);
                }
            }
            d = (a32[0] + a32[1]) + (a32[2] + a32[3]);
        }
        if (lane < 32) partial[(t * kF16sWaves + wid) * 32 + lane] = d;
    };
    auto stage_item = [&](int item, const u32x4 &v) {
        const int i = item & 15;
        const bool live = (static_cast<uint32_t>(c) * 1024u + 16u * lane) < row_bytes;
        *reinterpret_cast<u32x4 *>(stage + i * kF16sRowStride + 16 * lane) = live ? v : u32x4{0u, 0u, 0u, 0u};
        if (i == 15) tile_compute(item >> 4);
    };
    if (items <= kF16sDepth) {
#pragma unroll
        for (int dd = 0; dd < kF16sDepth; ++dd) stage_item(dd, ring[dd]);
    } else {
        for (int base = 0; base < items; base += kF16sDepth) {
#pragma unroll
            for (int dd = 0; dd < kF16sDepth; ++dd) {
                const int item = base + dd;
                if (item < items) stage_item(item, ring[dd]);
                load_item(item + kF16sDepth, ring[dd]);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): the clamped refills end here
    }
    __syncthreads();
    // 4. D[4g + r][n] of lane (n, g < 2): column 4g + r, weight row 16 tile + n
    for (int idx = threadIdx.x; idx < tiles_per_group * 128; idx += kWave * kF16sWaves) {
        const int t = idx >> 7, mm = (idx >> 4) & 7, nn = idx & 15;
        const int row = (tile0 + t) * 16 + nn;
        if (mm >= batch || tile0 + t >= tiles || row >= n) continue;
        const int src_lane = (mm >> 2) * 16 + nn, r = mm & 3;
        float sum = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kF16sWaves; ++ww) sum += partial[(t * kF16sWaves + ww) * 32 + src_lane][r];
        y[static_cast<size_t>(mm) * n + row] = sum;
    }
}

} // namespace

extern "C" int kk_dense_mfma_gemv(int type, const void *w, const float *x, float *y, int k, int n, int batch,
                                  hipStream_t stream) {
    if ((type != 0 && type != 1) || !w || !x || !y || k <= 0 || (k & 31) || n <= 0 || batch < 1 ||
        batch > 16 || (reinterpret_cast<uintptr_t>(w) & 15) || (reinterpret_cast<uintptr_t>(x) & 15))
        return hipErrorInvalidValue;
    if (type == 1 && batch <= 8 && k <= 4096 && kk::tuning_or(kk::kDenseStream, 1) != 0) {
        int device = 0;
        hipError_t rc = hipGetDevice(&device);
        if (rc != hipSuccess) return rc;
        rc = kk::opt_in_lds(reinterpret_cast<const void *>(&f16_stream_gemv), kF16sLdsBytes);
        if (rc != hipSuccess) return rc;
        const int cus = kk::cu_count(device);
        const int tiles = (n + 15) / 16;
        const int t = std::max(1, std::min(kF16sMaxTiles, (tiles + cus - 1) / cus));
        hipLaunchKernelGGL(f16_stream_gemv, dim3((tiles + t - 1) / t), dim3(kWave * kF16sWaves), kF16sLdsBytes, stream,
                           static_cast<const uint8_t *>(w), x, y, k, n, batch, t);
        return hipGetLastError();
    }
    const int tiles = (n + 15) / 16;
    if (type == 1)
        hipLaunchKernelGGL(dense_mfma_gemv<true>, dim3(tiles), dim3(kWave * kDenseWaves), 0, stream,
                           static_cast<const uint8_t *>(w), x, y, k, n, batch);
    else
        hipLaunchKernelGGL(dense_mfma_gemv<false>, dim3(tiles), dim3(kWave * kDenseWaves), 0, stream,
                           static_cast<const uint8_t *>(w), x, y, k, n, batch);
    return hipGetLastError();
}
