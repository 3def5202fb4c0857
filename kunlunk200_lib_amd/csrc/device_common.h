// Device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace kk {

// Workgroup barrier for LDS data only: waits for this wave's LDS operations
// (lgkmcnt) but not for its global loads, which stay in flight across it.
// (__syncthreads also waits for every outstanding global load of the wave.)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}


constexpr int kWave = 64;

// IEEE binary16 bits -> binary32 (v_cvt_f32_f16): exact, subnormals included,
// as the reference decoder (reference kernels/kunlun-matvec.xpu:4-18).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    union { uint16_t u; _Float16 h; } v;
    v.u = static_cast<uint16_t>(bits);
    return static_cast<float>(v.h);
}

// Byte C of a 32-bit word as float, one v_cvt_f32_ubyte{C} instruction. The
// compiler does not select the byte forms by itself once the word was masked
// (it emits a bit-field extract first), so they are written out.
template <int C>
__device__ __forceinline__ float ubyte_to_float(uint32_t word) {
    float r;
    if constexpr (C == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(word));
    else if constexpr (C == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(word));
    else if constexpr (C == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(word));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(word));
    return r;
}

// Bytes [s, s+4) of the little-endian 64-bit value hi:lo (v_alignbyte_b32).
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbyte(hi, lo, s);
}

// DPP lane move within rows of 16 lanes (quad_perm / mirror controls).
template <int Ctrl>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xf, 0xf, false));
}

// Sum over the 64 lanes of a wave, returned uniformly (scalar) to every lane:
// four DPP steps reduce each row of 16 lanes, then the four row sums are read.
__device__ __forceinline__ float wave_sum_uniform(float v) {
    v += dpp_move<0xb1>(v);    // quad_perm [1,0,3,2]
    v += dpp_move<0x4e>(v);    // quad_perm [2,3,0,1]
    v += dpp_move<0x141>(v);   // row_half_mirror: quads 0<->1, 2<->3
    v += dpp_move<0x140>(v);   // row_mirror: halves of the row
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, kWave));
    return v;
}

// Round half away from zero by truncating v +/- 0.5f, clamp to [-limit, limit]:
// the host rule of the reference (reference src/k200.cpp:114,217,224).
// Written without contraction so it rounds exactly as the host does.
__device__ __forceinline__ int round_clamp(float value, int limit) {
#pragma clang fp contract(off)
    float shifted = value + (value >= 0.0f ? 0.5f : -0.5f);
    int q = static_cast<int>(shifted);
    q = q > limit ? limit : q;
    q = q < -limit ? -limit : q;
    return q;
}

// Eight Q4_0 values of nibble dword `qs` (its bytes j = 0..3 hold values j in
// the low nibble and 16 + j in the high nibble) as exact fp16 q - 8, in the
// order (0, 2, 1, 3, 16, 18, 17, 19): (0x6400 | q) is 1024 + q, minus 1032 in
// one packed add per pair; a high nibble left in place gives (0x6400 | 16 q) =
// 1024 + 16 q, times 1/16 minus 72 in one packed fma. One shift per dword; the
// bit inserts (v_bfi_b32) take their masks from VGPRs.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ uint32_t nibble_insert(uint32_t mask, uint32_t a) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(a), "v"(0x64006400u));   // (a & mask) | 0x6400 pair
    return r;
}
__device__ __forceinline__ half8 q4_dword_halves(uint32_t qs) {
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    const uint32_t s8 = qs >> 8;
    const half2v off = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    const half2v off16 = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    const half2v a = __builtin_bit_cast(half2v, nibble_insert(0x000f000fu, qs)) + off;
    const half2v b = __builtin_bit_cast(half2v, nibble_insert(0x000f000fu, s8)) + off;
    const half2v c = __builtin_elementwise_fma(__builtin_bit_cast(half2v, nibble_insert(0x00f000f0u, qs)), sixteenth, off16);
    const half2v d = __builtin_elementwise_fma(__builtin_bit_cast(half2v, nibble_insert(0x00f000f0u, s8)), sixteenth, off16);
    half8 out;
    out[0] = a[0]; out[1] = a[1]; out[2] = b[0]; out[3] = b[1];
    out[4] = c[0]; out[5] = c[1]; out[6] = d[0]; out[7] = d[1];
    return out;
}

// 16-byte load from an address that is only 4-byte aligned (global_load_dwordx4).
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ u32x4_a4 load_u32x4(const uint32_t *p) {
    return *reinterpret_cast<const u32x4_a4 *>(p);
}

// The same with the non-temporal hint, for weight bytes read once per call
// (streamed past the caches instead of displacing reused data such as X).
__device__ __forceinline__ u32x4_a4 load_u32x4_stream(const uint32_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4 *>(p));
}
__device__ __forceinline__ uint32_t load_u32_stream(const uint32_t *p) { return __builtin_nontemporal_load(p); }

// Eight activations as signed fixed point X_t = rint(v[t] * to_fixed) (round
// to nearest even via the 1.5 * 2^23 magic constant, one FMA), written as
// DIGITS balanced base-16 digits in [-8, 7]. With FRAC = 4 * DIGITS - 2,
// to_fixed = 2^(FRAC-e) and every |v[t]| < 2^e, |X_t| <= 2^FRAC, and
// Z = (X + 0x88..8) ^ 0x88..8 (DIGITS eights) holds the digits directly as
// 4-bit two's-complement nibbles; the nibbles above DIGITS are zero
// (as_uint(fma) - 0x4b400000 + 0x88..8 in one add). Digit dword l holds digit
// l of X_t in nibble t, so for signed nibbles w_t:
//   sum_t w_t X_t = sum_l 16^l sdot8(w, dig[l]).
template <int DIGITS = 6>
__device__ __forceinline__ void fixed_point_digits(const float (&v)[8], float to_fixed, uint32_t (&dig)[DIGITS]) {
    static_assert(DIGITS == 5 || DIGITS == 6, "5 or 6 digits (19- or 23-bit fixed point)");
    constexpr uint32_t kEights = DIGITS == 6 ? 0x888888u : 0x88888u;
    constexpr uint32_t kAdd = kEights - 0x4b400000u;   // mod 2^32
    uint32_t z[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) z[t] = (__float_as_uint(fmaf(v[t], to_fixed, 12582912.0f)) + kAdd) ^ kEights;
    // 8 x DIGITS nibble transpose. E[s] byte c = (z[2s].n(2c), z[2s+1].n(2c)),
    // O[s] byte c = (.. n(2c+1) ..); v_perm_b32(hi, lo, sel): selector byte
    // 0-3 picks a lo byte, 4-7 a hi byte, 0x0c gives 0.
    uint32_t ev[4], od[4];
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
        ev[s2] = (z[2 * s2] & 0x0f0f0f0fu) | ((z[2 * s2 + 1] << 4) & 0xf0f0f0f0u);
        od[s2] = ((z[2 * s2] >> 4) & 0x0f0f0f0fu) | (z[2 * s2 + 1] & 0xf0f0f0f0u);
    }
    const uint32_t e01 = __builtin_amdgcn_perm(ev[1], ev[0], 0x05010400u);   // E0.b0 E1.b0 E0.b1 E1.b1
    const uint32_t e23 = __builtin_amdgcn_perm(ev[3], ev[2], 0x05010400u);
    dig[0] = __builtin_amdgcn_perm(e23, e01, 0x05040100u);
    dig[2] = __builtin_amdgcn_perm(e23, e01, 0x07060302u);
    dig[4] = __builtin_amdgcn_perm(ev[1], ev[0], 0x0c0c0602u) | __builtin_amdgcn_perm(ev[3], ev[2], 0x06020c0cu);
    const uint32_t o01 = __builtin_amdgcn_perm(od[1], od[0], 0x05010400u);
    const uint32_t o23 = __builtin_amdgcn_perm(od[3], od[2], 0x05010400u);
    dig[1] = __builtin_amdgcn_perm(o23, o01, 0x05040100u);
    dig[3] = __builtin_amdgcn_perm(o23, o01, 0x07060302u);
    if constexpr (DIGITS == 6)
        dig[DIGITS - 1] = __builtin_amdgcn_perm(od[1], od[0], 0x0c0c0602u) | __builtin_amdgcn_perm(od[3], od[2], 0x06020c0cu);
}

// SiLU(g) * u in F32 with the reference's non-finite rules (reference
// kernels/kunlun-swiglu.xpu:27-39): finite inputs give (g / (1 + e^-g)) * u;
// otherwise NaN when g or u is NaN or g is -Inf, +-Inf with the product sign
// when exactly one side is infinite and the other side (SiLU(g) for a finite
// g) is non-zero, NaN for Inf * 0. SiLU(g) is computed once and the special
// cases are selected from integer tests, without branches.
__device__ __forceinline__ float swiglu_value(float g, float u) {
#pragma clang fp contract(off)
    const float act = g / (1.0f + expf(-g));
    const uint32_t gb = __float_as_uint(g), ub = __float_as_uint(u);
    const uint32_t ga = gb & 0x7fffffffu, ua = ub & 0x7fffffffu;
    const uint32_t signed_inf = ((gb ^ ub) & 0x80000000u) | 0x7f800000u;
    uint32_t bits = __float_as_uint(act * u);
    bits = ga == 0x7f800000u ? (ua == 0 ? 0x7fc00000u : signed_inf) : bits;            // g = +Inf (-Inf below)
    bits = ga < 0x7f800000u && ua == 0x7f800000u
               ? ((__float_as_uint(act) & 0x7fffffffu) == 0 ? 0x7fc00000u : signed_inf)   // finite g, u = +-Inf
               : bits;
    bits = ga > 0x7f800000u || ua > 0x7f800000u || gb == 0xff800000u ? 0x7fc00000u : bits;
    return __uint_as_float(bits);
}

} // namespace kk
