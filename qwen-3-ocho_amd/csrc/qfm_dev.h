// qfm_dev.h -- device helpers shared by the MoE kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qfm {

constexpr int WAVE = 64;

// ---- bf16 ----------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
// round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// ---- int8 x fp32 dot of one 16-byte chunk ---------------------------------
// w holds 16 signed int8 codes. Each code is widened exactly with a
// sign-extending bit-field extract and an int->float conversion.
__device__ __forceinline__ float i8x4_f(uint32_t d, int b) {
    return (float)__builtin_amdgcn_sbfe((int)d, b * 8, 8);
}
__device__ __forceinline__ float dot16_i8(const uint4 w, const float *x, float acc) {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc = fmaf(i8x4_f(d[q], b), x[q * 4 + b], acc);
    return acc;
}
// Offset-binary form for the gate/up GEMVs: u = q ^ 0x80 = q + 128 is an
// unsigned byte, converted by v_cvt_f32_ubyteN in one op; the caller seeds
// the accumulator with -128 * sum(x) over the same elements.
__device__ __forceinline__ float dot16_u8(const uint4 w, const float *x, float acc) {
    const uint32_t d[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u, w.w ^ 0x80808080u};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        acc = fmaf((float)(d[q] & 0xFFu), x[q * 4 + 0], acc);
        acc = fmaf((float)((d[q] >> 8) & 0xFFu), x[q * 4 + 1], acc);
        acc = fmaf((float)((d[q] >> 16) & 0xFFu), x[q * 4 + 2], acc);
        acc = fmaf((float)(d[q] >> 24), x[q * 4 + 3], acc);
    }
    return acc;
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt16(const void *p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- cross-lane reductions -------------------------------------------------
// Sum over aligned groups of G lanes (G a power of two <= 64); every lane of
// the group ends with the group total.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int m = G / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, WAVE);
    return v;
}

// ---- silu / sigmoid ----------------------------------------------------------
__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }
__device__ __forceinline__ float sigmoid(float g) { return 1.0f / (1.0f + __expf(-g)); }

// ---- NVFP4 number formats -----------------------------------------------------
// E2M1 code -> float: +-{0, .5, 1, 1.5, 2, 3, 4, 6}; built from the bit
// fields (exponent e = (n >> 1) & 3, mantissa m = n & 1, sign bit 3).
__device__ __forceinline__ float e2m1(uint32_t nib) {
    const uint32_t e = (nib >> 1) & 3u, m = nib & 1u;
    const uint32_t mag = e ? (((e + 126u) << 23) | (m << 22)) : (m ? 0x3F000000u : 0u);
    return __uint_as_float(mag | ((nib & 8u) << 28));
}
// E4M3 block scale -> float: e == 0 -> m * 2^-9; else (1 + m/8) * 2^(e-7);
// 0x7F -> +inf (the checkpoint never stores it).
__device__ __forceinline__ float e4m3(uint32_t b) {
    const uint32_t e = (b >> 3) & 15u, m = b & 7u;
    const float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0x1p-9f;
    return ((b & 0x7Fu) == 0x7Fu) ? __uint_as_float(0x7F800000u) : v;
}

// ---- Philox-4x32-10 (Salmon et al. 2011) ------------------------------------
struct u4 { uint32_t v[4]; };
__device__ __forceinline__ u4 philox(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                     uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; r++) {
        const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        if (r != 9) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    }
    u4 o; o.v[0] = c0; o.v[1] = c1; o.v[2] = c2; o.v[3] = c3;
    return o;
}

}  // namespace qfm
