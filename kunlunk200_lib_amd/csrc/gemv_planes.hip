// Batch-1 Q4_0 GEMV on int8 MFMA with activation digit planes (gfx950).
//
// Y[r] = sum_k X[k] * W[r, k] for raw 18-byte Q4_0 rows (reference
// kernels/kunlun-matvec.xpu:24-79: per 32-value block, d * sum_j (q_j - 8) x_j).
//
// Arithmetic. Each 32-value activation block b with 2^(e-1) <= max|x| < 2^e
// (e = frexp exponent) becomes fixed point: the high half (values 16..31) as
// X_j = rint(x_j * 2^(18-e)), |X_j| <= 2^18, and the low half (values 0..15)
// as X'_j = rint(x_j * 2^(22-e)) = 16 X_j up to rounding, |X'_j| <= 2^22.
// Each is written as three balanced base-256 digits in [-128, 127]
// (V = D0 + 256 D1 + 65536 D2): Z = (V + 0x808080) ^ 0x808080 holds them
// as int8 in its low three bytes. The weight nibbles become int8 without a
// shift: low nibbles as q (0..15, one AND), high nibbles as 16 (q - 8)
// ((byte & 0xF0) ^ 0x80); one v_bitop3 each. v_mfma_i32_16x16x64_i8 then
// gives, per weight row and digit plane l, the exact plane sum
//   D_l = sum_{j<16} q_j D_l(X'_j) + sum_{j>=16} 16 (q_j - 8) D_l(X_j),
// and S = D_0 + 256 D_1 + 65536 D_2 - 8 sum_{j<16} X'_j
//       = sum_{j<16} (q_j - 8) X'_j + sum_{j>=16} (q_j - 8) 16 X_j
// exactly in int32 (|S| <= 2^30), so y += float(S) * d * 2^(e-22).
// Error: per element at most 2^(e-19) <= max|x| 2^-18, so
// |sum_j w_j e_j| <= ||w|| ||e|| <= 2^-18 sqrt(32) ||x|| ||w|| = 2.2e-5 ||x|| ||w||,
// inside the 1e-4 ||x|| ||w|| bound of the F32-accumulate GEMV.
//
// MFMA mapping (16x16x64 i8: lane l holds A[l%16][16(l/16)..+16),
// B[16(l/16)..+16)[l%16], D[4(l/16)+i][l%16]). An "octet" is eight
// consecutive blocks (256 values, 144 bytes of a row). Lane (n = l%16,
// g = l/16) owns block pair g of the octet of weight row n: blocks 2g and
// 2g+1, 36 bytes. Four MFMAs cover an octet: for each of its two blocks, one
// for nibble bytes 0..7 and one for bytes 8..15; the lane's 16 B-operand
// bytes are the low nibbles of bytes 0..3, their high nibbles, the low
// nibbles of bytes 4..7 and their high nibbles (values 0-3, 16-19, 4-7,
// 20-23; then 8-11, 24-27, 12-15, 28-31), and the activation planes are
// stored in that order. The A operand puts block c's three planes in rows
// 4c'..4c'+2 for the lanes of group c' = c >> 1 and is zero elsewhere, so
// the first (last) two MFMAs leave in lane (n, g) the plane sums of block 2g
// (2g + 1) of row n, whose F16 scales that lane holds. Per octet and lane:
// 4 v_alignbyte (block 2g's nibbles start 2 bytes into the pair), 16
// v_bitop3, four MFMAs and two 7-op epilogues.
//
// Memory. Weight bytes never reach a register straight from memory: each
// wave streams "stages" (16 rows x 2 octets = 288 bytes per row) into its own
// ring of R LDS slots with five buffer_load_dwordx4 ... lds copies per stage
// (1 KB each, consecutive lanes on consecutive 16 bytes of a row), so every
// copy touches the fewest cache lines a 1 KB load can. Rows sit 19 pieces of
// 16 bytes apart in a slot (one piece of padding; 9 pieces for a one-octet
// stage), an odd number of 16-byte units, so the 16 rows a ds_read of the
// lanes touches fall in distinct banks. Each stage's buffer resource starts
// at the stage, and the copy offsets of rows past the matrix or of unused
// copies lie past its extent: those lanes read zeros and nothing out of
// bounds. A wave issues the copy of stage s + R - 1 before it waits for
// stage s (every stage issues exactly five copies, so the memory-counter
// wait is a constant).
//
// Work split. One workgroup per CU (8 waves) takes a contiguous range of
// 16-row tiles (of both matrices in PAIR mode). Each tile's K is cut into 8
// chunks of an even number of octets (a chunk length depends on K only);
// the workgroup's chunks, tile-major, are dealt to its waves in equal
// numbers, so each wave owns whole chunks. A wave writes one sum per chunk
// and lane to LDS slots [tile][chunk][lane] (zeroed first), and after the
// last barrier the workgroup adds each output row's 32 slots in a fixed
// order: the result depends on the data and K only, not on the grid or the
// wave split, and the PAIR mode's gate and up sums equal the single-matrix
// kernel's bit for bit. PAIR mode writes SiLU(gate) * up (the swiglu
// kernel's element function). The activation planes are built once per
// workgroup into LDS while the first copies are in flight.
#include "device_common.h"
#include "launch.h"

#include <algorithm>

namespace {

using kk::kWave;
typedef int int32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t lds_byte;

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileRows = 16;
constexpr int kMaxTilesPerGroup = 16;
constexpr int kChunks = 8;                         // K chunks per tile (one LDS slot each)
constexpr int kBlockPlaneBytes = 96;               // 3 planes x 2 halves x 16 bytes
constexpr int kOctetBytes = 144;                   // 8 blocks of one row
constexpr int kOctetPlaneBytes = 8 * kBlockPlaneBytes;
constexpr int kCopies = 5;                         // 1 KB copies per stage
constexpr int kSlotBytes = kCopies * 1024;
constexpr int kPieces2 = 19, kPieces1 = 9;         // 16-byte pieces per row and stage of 2 / 1 octets
constexpr int kZeroBytes = 128;                    // zero A operand for lanes outside the plane rows
constexpr int kLdsLimit = 160 * 1024;
constexpr uint32_t kOutOfRange = 0x80000000u;      // copy offset past any extent: the lane reads zeros

struct PlanesLayout {
    uint32_t scale_corr, zero, partial, ring, total;
};

// LDS: [planes: blocks x 96][scale, correction: blocks x 8][zero 128]
//      [partials: tiles x mats x 8 chunks x 64 lanes x 4][ring: 8 waves x R x 5 KB]
__host__ __device__ inline PlanesLayout planes_layout(int k, int tiles_per_group, int mats, int ring_slots) {
    PlanesLayout l;
    const uint32_t blocks = static_cast<uint32_t>(k) / 32;
    l.scale_corr = blocks * kBlockPlaneBytes;
    l.zero = l.scale_corr + blocks * 8;
    l.partial = l.zero + kZeroBytes;
    l.ring = l.partial + static_cast<uint32_t>(tiles_per_group * mats * kChunks * kWave * 4);
    l.total = l.ring + static_cast<uint32_t>(kWaves * ring_slots * kSlotBytes);
    return l;
}

// One stage's five copies into LDS offset `slot`: copy j moves lane l's 16
// bytes at voff[j] past `base` to slot + 1024 j + 16 l. Offsets at or past
// `extent` read zeros. (A device function, not a lambda of the kernel: the
// host pass drops the launch stub of a kernel whose lambda hands captured
// values to this builtin.)
__device__ __forceinline__ void copy_stage(const uint8_t *base, uint32_t extent, uint32_t slot,
                                           const uint32_t (&voff)[kCopies]) {
    extern __shared__ __align__(16) uint8_t lds[];
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, static_cast<int>(extent), 0x00020000);
#pragma unroll
    for (int j = 0; j < kCopies; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_byte *)lds + slot + j * 1024, 16, voff[j], 0, 0, 0);
}

// LDS accesses issued after a wave's first LDS DMA copy are inline assembly:
// the compiler cannot tell the ring slot being read from the slots the
// copies in flight write, and would wait for every copy in flight before
// any LDS access it can see. The assembly accesses are ordered by explicit
// lgkmcnt waits. Addresses are byte offsets in the workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr(uint8_t *p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_byte *)p));
}
__device__ __forceinline__ void lds_store(uint32_t addr, uint32_t v) {
    asm volatile("ds_write_b32 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// PASSES: activation staging passes, k / 8 <= PASSES * kThreads. R: LDS
// ring slots per wave. PAIR: w is the gate matrix, w2 the up matrix,
// y = SiLU(X w^T) * (X w2^T).
template <int R, int PASSES, bool PAIR>
__global__ __launch_bounds__(kThreads) void q4_gemv_planes(const uint8_t *__restrict__ w,
                                                          const uint8_t *__restrict__ w2,
                                                          const float *__restrict__ x, float *__restrict__ y,
                                                          int k, int n, int tiles, int tiles_per_group) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int kMats = PAIR ? 2 : 1;
    const int blocks = k >> 5;
    const int octets = k >> 8;
    const uint32_t row_bytes = static_cast<uint32_t>(blocks) * 18;
    const uint32_t mat_bytes = static_cast<uint32_t>(n) * row_bytes;     // <= INT_MAX (matmul's limit)
    const PlanesLayout L = planes_layout(k, tiles_per_group, kMats, R);
    float *partial = reinterpret_cast<float *>(lds + L.partial);
    const uint32_t lds_base = lds_addr(lds);

    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int nn = lane & 15, g = lane >> 4;

    // this workgroup's tiles [t0, t1) (of each matrix) and this wave's units [v0, v1)
    const int groups = gridDim.x;
    const int t0 = static_cast<int>((static_cast<long long>(blockIdx.x) * tiles) / groups);
    const int t1 = static_cast<int>((static_cast<long long>(blockIdx.x + 1) * tiles) / groups);
    const int tw = t1 - t0;
    const int chunk = 2 * ((octets + 2 * kChunks - 1) / (2 * kChunks));   // octets per chunk, even
    const int units = kMats * tw * kChunks;
    const int v0 = (wid * units) / kWaves, v1 = ((wid + 1) * units) / kWaves;
    auto unit_begin = [&](int v) { return min((v % kChunks) * chunk, octets); };
    auto unit_end = [&](int v) { return min((v % kChunks + 1) * chunk, octets); };
    // Stage descriptors, one per lane: lane i describes this wave's stage i
    // (at most 64 per wave, which the host's plan ensures): its byte offset
    // in its matrix, and packed fields: unit v (bits 16..; the partial slot,
    // and through v / 8 the matrix and tile), first octet (bits 8..15), last
    // stage of its unit (bit 1), two octets rather than one (bit 0). The loop
    // reads them with v_readlane.
    uint32_t desc_start = 0, desc_info = 0;
    int stages = 0;
    for (int v = v0; v < v1; ++v) {
        const int ob = unit_begin(v), oe = unit_end(v);
        const int ns = (oe - ob + 1) >> 1;
        const int i = lane - stages;                          // this lane's stage within unit v
        if (i >= 0 && i < ns) {
            const int mt = v / kChunks, mtx = PAIR && mt >= tw ? 1 : 0;
            const int o = ob + 2 * i;
            desc_start = static_cast<uint32_t>((t0 + mt - mtx * tw) * kTileRows) * row_bytes +
                         static_cast<uint32_t>(o) * kOctetBytes;
            desc_info = (static_cast<uint32_t>(v) << 16) | (static_cast<uint32_t>(o) << 8) |
                        (i == ns - 1 ? 2u : 0u) | (oe - o >= 2 ? 1u : 0u);
        }
        stages += ns;
    }

    // lane copy offsets from a stage's first byte (row 0 of the tile, first octet)
    uint32_t voff2[kCopies], voff1[kCopies];
#pragma unroll
    for (int j = 0; j < kCopies; ++j) {
        const int p = 64 * j + lane;
        voff2[j] = static_cast<uint32_t>(p / kPieces2) * row_bytes + 16u * static_cast<uint32_t>(p % kPieces2);
        voff1[j] = p < 3 * 64 ? static_cast<uint32_t>(p / kPieces1) * row_bytes +
                                    16u * static_cast<uint32_t>(p % kPieces1)
                              : kOutOfRange;
    }
    // Copies of stage st into ring slot `slot`: five copies, no branch (so
    // the compiler counts them exactly); past the wave's last stage the
    // extent is 0 and every lane reads zeros. The tile's first row exists, so
    // start < mat_bytes.
    const uint32_t ring = L.ring + static_cast<uint32_t>(wid * R * kSlotBytes);
    auto issue_copies = [&](int st, int slot) {
        const bool live = st < stages;
        const int sl = min(st, kWave - 1);
        const uint32_t start =
            live ? static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(desc_start), sl)) : 0u;
        const uint32_t info = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(desc_info), sl));
        const bool mtx = PAIR && static_cast<int>(info >> 19) >= tw;   // v / 8 >= tw: the up matrix
        const uint32_t extent = live ? mat_bytes - start : 0u;
        const bool two = info & 1u;
        uint32_t vo[kCopies];
#pragma unroll
        for (int j = 0; j < kCopies; ++j) vo[j] = two ? voff2[j] : voff1[j];
        copy_stage((mtx ? w2 : w) + start, extent, ring + static_cast<uint32_t>(slot * kSlotBytes), vo);
    };

    // 1. activation loads: thread t owns values [8t, 8t + 8)
    const int groups8 = k >> 3;
    float4 xa[PASSES], xb[PASSES];
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const int t = min(pass * kThreads + static_cast<int>(threadIdx.x), groups8 - 1);
        xa[pass] = *reinterpret_cast<const float4 *>(x + 8 * t);
        xb[pass] = *reinterpret_cast<const float4 *>(x + 8 * t + 4);
    }
    // 2. the copies of the first R - 1 stages, after the activation loads
#pragma unroll
    for (int st = 0; st < R - 1; ++st) issue_copies(st, st);
    // 3. activation planes (in the MFMA k order), block scales and corrections;
    //    zero area and partials
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const int t = pass * kThreads + static_cast<int>(threadIdx.x);
        const float v[8] = {xa[pass].x, xa[pass].y, xa[pass].z, xa[pass].w,
                            xb[pass].x, xb[pass].y, xb[pass].z, xb[pass].w};
        float m = 0.0f, bad = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float a = fabsf(v[j]);
            bad = (a <= 3.402823466e38f) ? bad : 1.0f;
            m = fmaxf(m, a);
        }
        // the four threads of a block are one quad of lanes
        m = fmaxf(m, kk::dpp_move<0xb1>(m));
        m = fmaxf(m, kk::dpp_move<0x4e>(m));
        bad = fmaxf(bad, kk::dpp_move<0xb1>(bad));
        bad = fmaxf(bad, kk::dpp_move<0x4e>(bad));
        const int e = max(__builtin_amdgcn_frexp_expf(m), -100);
        const int part = t & 3;                     // values 8 part .. 8 part + 7 of the block
        const int high = part >> 1;                 // values 16..31
        const float to_fixed = ldexpf(1.0f, (high ? 18 : 22) - e);
        uint32_t z[8];
        int sum = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t f = __float_as_uint(fmaf(v[j], to_fixed, 12582912.0f));   // 0x4b400000 + V
            sum += static_cast<int>(f - 0x4b400000u);
            z[j] = (f + 0xb5408080u) ^ 0x808080u;      // bytes 0..2: balanced digits of V
        }
        // the low half's two threads are lanes 4j and 4j + 1
        sum += __builtin_amdgcn_update_dpp(0, sum, 0xb1, 0xf, 0xf, false);
        // planes: byte l of z[j] -> plane l, value j (dwords of values 0-3, 4-7)
        uint32_t pl[3][2];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const uint32_t ab = __builtin_amdgcn_perm(z[4 * s2 + 1], z[4 * s2 + 0], 0x05010400u);   // a0 b0 a1 b1
            const uint32_t cd = __builtin_amdgcn_perm(z[4 * s2 + 3], z[4 * s2 + 2], 0x05010400u);
            const uint32_t ab2 = __builtin_amdgcn_perm(z[4 * s2 + 1], z[4 * s2 + 0], 0x0c0c0602u);  // a2 b2 0 0
            const uint32_t cd2 = __builtin_amdgcn_perm(z[4 * s2 + 3], z[4 * s2 + 2], 0x0c0c0602u);
            pl[0][s2] = __builtin_amdgcn_perm(cd, ab, 0x05040100u);     // a0 b0 c0 d0
            pl[1][s2] = __builtin_amdgcn_perm(cd, ab, 0x07060302u);     // a1 b1 c1 d1
            pl[2][s2] = __builtin_amdgcn_perm(cd2, ab2, 0x05040100u);   // a2 b2 c2 d2
        }
        if (t < groups8) {
            const int blk = t >> 2;
            // 16-byte group (part & 1) holds values {0-3, 16-19, 4-7, 20-23} (+8 for group 1):
            // this thread's values 0-3 go to dword `high`, values 4-7 to dword high + 2
            const uint32_t dst = lds_base + static_cast<uint32_t>(blk * kBlockPlaneBytes + (part & 1) * 16 + high * 4);
#pragma unroll
            for (int l = 0; l < 3; ++l) {
                lds_store(dst + l * 32, pl[l][0]);
                lds_store(dst + l * 32 + 8, pl[l][1]);
            }
            if (part == 0) {
                const float s = bad != 0.0f ? __builtin_nanf("") : ldexpf(1.0f, e - 22);
                lds_store(lds_base + L.scale_corr + blk * 8, __float_as_uint(s));
                lds_store(lds_base + L.scale_corr + blk * 8 + 4, static_cast<uint32_t>(8 * sum));
            }
        }
    }
    if (threadIdx.x < kZeroBytes / 4) lds_store(lds_base + L.zero + 4 * threadIdx.x, 0u);
    for (int i = threadIdx.x; i < kMats * tw * kChunks * kWave; i += kThreads) lds_store(lds_base + L.partial + 4 * i, 0u);
    // LDS writes done, then a plain barrier: __syncthreads() would also wait
    // for the weight copies in flight
    lds_wait();
    __builtin_amdgcn_s_barrier();

    // 4. per-lane constants
    // A operand: lanes (m, c') with m in {4c', 4c'+1, 4c'+2} read plane m & 3 of
    // block 2c' (+1 for the last two MFMAs) of the octet; the others read zeros
    const bool a_active = (nn >> 2) == g && (nn & 3) < 3;
    const uint32_t a_base = a_active ? static_cast<uint32_t>(2 * g * kBlockPlaneBytes + (nn & 3) * 32) : L.zero;
    const uint32_t a_step = a_active ? static_cast<uint32_t>(kOctetPlaneBytes) : 0u;
    const uint32_t b_off2 = static_cast<uint32_t>(nn * kPieces2 * 16 + 36 * g);
    const uint32_t b_off1 = static_cast<uint32_t>(nn * kPieces1 * 16 + 36 * g);
    float acc = 0.0f;

    // the two nibble dwords (bytes 4i .. 4i+7 of a block's nibbles) -> B:
    // low nibbles as q, high nibbles as 16 (q - 8)
    auto b_operand = [](uint32_t n0, uint32_t n1) {
        int32x4 b;
        b.x = static_cast<int>(n0 & 0x0f0f0f0fu);
        b.y = static_cast<int>((n0 & 0xf0f0f0f0u) ^ 0x80808080u);
        b.z = static_cast<int>(n1 & 0x0f0f0f0fu);
        b.w = static_cast<int>((n1 & 0xf0f0f0f0u) ^ 0x80808080u);
        return b;
    };
    auto epilogue = [&](const int32x4 &dsum, uint32_t d_bits, uint32_t scale_bits, uint32_t corr) {
        const int s = dsum.x + (dsum.y << 8) + (dsum.z << 16) - static_cast<int>(corr);
        acc = fmaf(static_cast<float>(s), kk::half_bits_to_float(d_bits) * __uint_as_float(scale_bits), acc);
    };
    // one octet: the pair's 36 bytes at LDS offset `src`, global octet index og
    auto compute_octet = [&](uint32_t src, int og) {
        uint32_t wv[9];
        int32x4 a0, a1, a2, a3, sc;
        const uint32_t a_off = lds_base + a_base + static_cast<uint32_t>(og) * a_step;
        const uint32_t sc_off = lds_base + L.scale_corr + static_cast<uint32_t>(og * 64 + g * 16);
        const uint32_t b_off = lds_base + src;
        asm volatile(
            "ds_read_b32 %0, %14\n"
            "ds_read_b32 %1, %14 offset:4\n"
            "ds_read_b32 %2, %14 offset:8\n"
            "ds_read_b32 %3, %14 offset:12\n"
            "ds_read_b32 %4, %14 offset:16\n"
            "ds_read_b32 %5, %14 offset:20\n"
            "ds_read_b32 %6, %14 offset:24\n"
            "ds_read_b32 %7, %14 offset:28\n"
            "ds_read_b32 %8, %14 offset:32\n"
            "ds_read_b128 %9, %15\n"
            "ds_read_b128 %10, %15 offset:16\n"
            "ds_read_b128 %11, %15 offset:96\n"
            "ds_read_b128 %12, %15 offset:112\n"
            "ds_read_b128 %13, %16\n"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(wv[0]), "=&v"(wv[1]), "=&v"(wv[2]), "=&v"(wv[3]), "=&v"(wv[4]), "=&v"(wv[5]), "=&v"(wv[6]),
              "=&v"(wv[7]), "=&v"(wv[8]), "=&v"(a0), "=&v"(a1), "=&v"(a2), "=&v"(a3), "=&v"(sc)
            : "v"(b_off), "v"(a_off), "v"(sc_off)
            : "memory");
        static_assert(kBlockPlaneBytes == 96, "A operand offsets of the asm block");
        uint32_t na[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) na[i] = kk::align_bytes(wv[i + 1], wv[i], 2);   // block 2g: bytes 2..17
        const int32x4 zero = {0, 0, 0, 0};
        int32x4 da = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b_operand(na[0], na[1]), zero, 0, 0, 0);
        int32x4 db = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, b_operand(wv[5], wv[6]), zero, 0, 0, 0);
        da = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b_operand(na[2], na[3]), da, 0, 0, 0);
        db = __builtin_amdgcn_mfma_i32_16x16x64_i8(a3, b_operand(wv[7], wv[8]), db, 0, 0, 0);
        epilogue(da, wv[0] & 0xffffu, static_cast<uint32_t>(sc.x), static_cast<uint32_t>(sc.y));
        epilogue(db, wv[4] >> 16, static_cast<uint32_t>(sc.z), static_cast<uint32_t>(sc.w));
    };

    int copy_slot = R - 1, comp_slot = 0;
    for (int st = 0; st < stages; ++st) {
        // refill: stage st + R - 1 into the slot stage st - 1 used (its reads are done)
        __builtin_amdgcn_s_waitcnt(0xc07f);                       // lgkmcnt(0)
        issue_copies(st + R - 1, copy_slot);
        copy_slot = copy_slot + 1 == R ? 0 : copy_slot + 1;
        // stage st has landed once at most R - 1 stages of copies are pending
        __builtin_amdgcn_s_waitcnt(0x0f70 | ((R - 1) * kCopies));   // vmcnt((R - 1) * 5) only
        const uint32_t slot = ring + static_cast<uint32_t>(comp_slot * kSlotBytes);
        comp_slot = comp_slot + 1 == R ? 0 : comp_slot + 1;
        const uint32_t info = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(desc_info), st));
        const int og = static_cast<int>((info >> 8) & 0xffu);
        if (info & 1u) {
            compute_octet(slot + b_off2, og);
            compute_octet(slot + b_off2 + kOctetBytes, og + 1);
        } else {
            compute_octet(slot + b_off1, og);
        }
        if (info & 2u) {                                          // the last stage of unit v
            // slot of unit v = (matrix * tw + tile) * 8 + chunk
            lds_store(lds_base + L.partial + 4u * ((info >> 16) * kWave + static_cast<uint32_t>(lane)),
                      __float_as_uint(acc));
            acc = 0.0f;
        }
    }
    lds_wait();
    __syncthreads();

    // 5. output rows: slot sums in a fixed order (chunk, then lane group)
    auto row_sum = [&](int mt, int row) {
        float v = 0.0f;
        for (int c = 0; c < kChunks; ++c) {
            const float *slot = partial + (mt * kChunks + c) * kWave + row;
            v += (slot[0] + slot[16]) + (slot[32] + slot[48]);
        }
        return v;
    };
    for (int j = threadIdx.x; j < tw * kTileRows; j += kThreads) {
        const int tl = j >> 4, row = j & 15;
        const int r = (t0 + tl) * kTileRows + row;
        if (r < n) y[r] = PAIR ? kk::swiglu_value(row_sum(tl, row), row_sum(tw + tl, row)) : row_sum(tl, row);
    }
}

struct PlanesPlan {
    int ring, groups, tiles_per_group, passes;
    size_t lds;
};

// Grid and ring depth: one workgroup per CU (more when a workgroup would
// hold more than 16 tiles), three ring slots per wave when the LDS allows.
PlanesPlan plan_planes(int k, int n, int cus, bool pair) {
    PlanesPlan p;
    const int tiles = (n + kTileRows - 1) / kTileRows;
    const int mats = pair ? 2 : 1;
    p.groups = std::max(1, std::min(tiles, std::max((tiles + kMaxTilesPerGroup - 1) / kMaxTilesPerGroup, cus)));
    p.tiles_per_group = (tiles + p.groups - 1) / p.groups;
    // stages per wave (mats * tiles_per_group units of at most ceil(octets / 16))
    // must fit one descriptor per lane
    const int stages_per_unit = (k / 256 + 2 * kChunks - 1) / (2 * kChunks);
    while (mats * p.tiles_per_group * stages_per_unit > kWave && p.groups < tiles) {
        p.groups = std::min(tiles, p.groups * 2);
        p.tiles_per_group = (tiles + p.groups - 1) / p.groups;
    }
    p.ring = 3;
    while (planes_layout(k, p.tiles_per_group, mats, p.ring).total > kLdsLimit) {
        if (p.ring > 2) {
            --p.ring;
        } else {
            p.groups = std::min(tiles, p.groups * 2);
            p.tiles_per_group = (tiles + p.groups - 1) / p.groups;
        }
    }
    p.lds = planes_layout(k, p.tiles_per_group, mats, p.ring).total;
    p.passes = (k / 8 + kThreads - 1) / kThreads;
    return p;
}

template <int R, int PASSES, bool PAIR>
hipError_t launch_planes_cfg(const uint8_t *w, const uint8_t *w2, const float *x, float *y, int k, int n,
                             const PlanesPlan &p, hipStream_t stream) {
    // dynamic LDS above 64 KiB is opted into once per device
    constexpr int kMaxDevices = 64;
    static bool configured[kMaxDevices] = {};
    int device = 0;
    hipError_t rc = hipGetDevice(&device);
    if (rc != hipSuccess) return rc;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    auto kernel = &q4_gemv_planes<R, PASSES, PAIR>;
    if (!configured[device]) {
        rc = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                 kLdsLimit);
        if (rc != hipSuccess) return rc;
        configured[device] = true;
    }
    const int tiles = (n + kTileRows - 1) / kTileRows;
    hipLaunchKernelGGL(kernel, dim3(p.groups), dim3(kThreads), p.lds, stream, w, w2, x, y, k, n, tiles,
                       p.tiles_per_group);
    return hipGetLastError();
}

template <bool PAIR>
hipError_t launch_planes(const uint8_t *w, const uint8_t *w2, const float *x, float *y, int k, int n, int cus,
                         hipStream_t stream) {
    const PlanesPlan p = plan_planes(k, n, cus, PAIR);
    if (p.lds > static_cast<size_t>(kLdsLimit)) return hipErrorInvalidValue;
#define KK_PLANES_CASE(RR, PP)                                                                       \
    if (p.ring == RR && p.passes == PP) return launch_planes_cfg<RR, PP, PAIR>(w, w2, x, y, k, n, p, stream);
    KK_PLANES_CASE(3, 1)
    KK_PLANES_CASE(3, 2)
    KK_PLANES_CASE(3, 3)
    KK_PLANES_CASE(3, 4)
    KK_PLANES_CASE(2, 1)
    KK_PLANES_CASE(2, 2)
    KK_PLANES_CASE(2, 3)
    KK_PLANES_CASE(2, 4)
#undef KK_PLANES_CASE
    return hipErrorInvalidValue;
}

} // namespace

extern "C" int kk_q4_gemv_planes_supported(const void *w, const float *x, int k, int n) {
    return w && x && n > 0 && k > 0 && k <= 16384 && (k % 256) == 0 && (reinterpret_cast<uintptr_t>(w) & 3) == 0 &&
           (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

extern "C" int kk_q4_gemv_planes(const void *w, const float *x, float *y, int k, int n, int cus, hipStream_t stream) {
    if (!y || !kk_q4_gemv_planes_supported(w, x, k, n) || cus <= 0) return hipErrorInvalidValue;
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    return launch_planes<false>(wb, wb, x, y, k, n, cus, stream);
}

extern "C" int kk_q4_gemv_planes_pair_swiglu(const void *w_gate, const void *w_up, const float *x, float *y, int k,
                                             int n, int cus, hipStream_t stream) {
    if (!y || !kk_q4_gemv_planes_supported(w_gate, x, k, n) || !kk_q4_gemv_planes_supported(w_up, x, k, n) ||
        cus <= 0)
        return hipErrorInvalidValue;
    return launch_planes<true>(static_cast<const uint8_t *>(w_gate), static_cast<const uint8_t *>(w_up), x, y, k,
                               n, cus, stream);
}
