// qfm_dev.h -- device helpers shared by the MoE kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qfm {

constexpr int WAVE = 64;

// Lanes per weight row for a row of cpr 16-byte chunks: the largest of
// 32/16/8/4 that divides it (every lane then owns cpr/lpr chunks).
constexpr int lpr_of(int cpr) { return cpr % 32 == 0 ? 32 : cpr % 16 == 0 ? 16 : cpr % 8 == 0 ? 8 : 4; }

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
// Codes are consumed in offset-binary form: u = q ^ 0x80 = q + 128 is an
// unsigned byte, widened exactly by v_cvt_f32_ubyteN (one op per code); the
// caller seeds the accumulator with -128 * sum(x) over the same elements.
// (A sign-extending extract followed by an int->float conversion is not
// used: hipcc 7.2 folds that pair into v_cvt_f32_u32_sdwa with a sext
// source, an unsigned conversion that turns negative codes into ~4e9.)
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

// ---- wave-wide reductions from the ROCm device library (ockl) -------------
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_max_u64(unsigned long long);
extern "C" __device__ __attribute__((const)) float __ockl_wfred_add_f32(float);

// Order-preserving 64-bit selection key of a logit: descending value, ties to
// the lower index. -0.0 is folded onto +0.0 (they compare equal as floats).
__device__ __forceinline__ unsigned long long topk_key(float v, int e) {
    const uint32_t b = __float_as_uint(v + 0.0f);
    const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}
__device__ __forceinline__ int topk_key_index(unsigned long long key) {
    return (int)(0xFFFFFFFFu - (uint32_t)key);
}
__device__ __forceinline__ float topk_key_value(unsigned long long key) {
    const uint32_t k = (uint32_t)(key >> 32);
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// ---- wave top-K --------------------------------------------------------------
// One wave selects the top-K (K <= 16) of E = 64*EPL logits lr[0..E) (EPL <= 16):
// descending value, ties to the lower index (64-bit keys, all distinct).
// Wave-uniform control flow; lds: kTopkLds u64 of wave-private LDS, 16-byte aligned.
//
// Method (latency-bound: one wave, so few dependent steps and independent
// accumulators). 31-bit keys k31 = (value prefix << IB) | (E - 1 - e), IB =
// index bits (9 for E = 512, 22-bit prefix of the sortable value bits), are distinct; T31 = the K-th largest of the 64 lane maxima of k31 (rank by
// broadcast compares, sign of the 31-bit difference), P = its value prefix.
// Every element of the true top-K has a prefix >= P (K distinct lane maxima
// have prefix >= P and the K-th largest element is >= the least of them), so
// C = {prefix >= P} contains the top-K; typically |C| ~ K. If |C| > 64 (ties
// in the prefix) the exact 64-bit form of the same bound is used instead:
// T = K-th largest 64-bit lane maximum, C = {key >= T}, |C| <= K*EPL. C is
// compacted to LDS with ballots and mbcnt and each candidate's exact rank
// within C is its rank among all E.
constexpr int kTopkLds = 16 + 256 + 64 + 64;   // results, candidates, junk slots, lane maxima
template <int EPL>
__device__ __forceinline__ int topk_candidates(const float *lr, int K, int lane, unsigned long long *lds,
                                               float (&v)[EPL]) {
    static_assert(EPL >= 1 && EPL <= 16, "E = 64 * EPL, EPL <= 16");
    constexpr int E = 64 * EPL;
    constexpr int IB = E <= 64 ? 6 : E <= 128 ? 7 : E <= 256 ? 8 : E <= 512 ? 9 : 10;   // index bits
    constexpr int PB = 31 - IB;                                                        // value-prefix bits
    unsigned long long key[EPL];
    uint32_t k31[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        v[i] = lr[i * 64 + lane];
        key[i] = topk_key(v[i], i * 64 + lane);
        k31[i] = ((uint32_t)(key[i] >> (64 - PB)) << IB) | (uint32_t)(E - 1 - (i * 64 + lane));
    }
    unsigned long long *cand = lds + 16, *lm = lds + 16 + 256 + 64;
    uint32_t *lm32 = reinterpret_cast<uint32_t *>(lm);
    uint32_t mx = k31[0];
#pragma unroll
    for (int i = 1; i < EPL; i++) mx = max(mx, k31[i]);
    lm32[lane] = mx;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    uint32_t r4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int h = 0; h < 2; h++) {
        uint4 p[8];
#pragma unroll
        for (int q = 0; q < 8; q++) p[q] = reinterpret_cast<const uint4 *>(lm32)[h * 8 + q];
#pragma unroll
        for (int q = 0; q < 8; q++) {      // keys < 2^31: the difference's sign bit is (other > mine)
            r4[0] += (mx - p[q].x) >> 31; r4[1] += (mx - p[q].y) >> 31;
            r4[2] += (mx - p[q].z) >> 31; r4[3] += (mx - p[q].w) >> 31;
        }
    }
    const uint32_t rank = r4[0] + r4[1] + r4[2] + r4[3];
    const uint32_t T31 = (uint32_t)__builtin_amdgcn_readlane((int)mx, __builtin_ctzll(__ballot(rank == (uint32_t)(K - 1))));
    const uint32_t P = T31 & ~((1u << IB) - 1u);
    unsigned long long b[EPL];
    int base[EPL], tot = 0;
#pragma unroll
    for (int i = 0; i < EPL; i++) b[i] = __ballot(k31[i] >= P);
#pragma unroll
    for (int i = 0; i < EPL; i++) { base[i] = tot; tot += __popcll(b[i]); }
    if (tot > 64) {
        // exact bound: 64-bit lane maxima (wave-uniform branch)
        unsigned long long m64 = key[0];
#pragma unroll
        for (int i = 1; i < EPL; i++) m64 = key[i] > m64 ? key[i] : m64;
        lm[lane] = m64;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        int ra[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 64; j += 8) {
            ulonglong2 p[4];
#pragma unroll
            for (int q = 0; q < 4; q++) p[q] = *reinterpret_cast<const ulonglong2 *>(lm + j + 2 * q);
#pragma unroll
            for (int q = 0; q < 4; q++) ra[q] += (p[q].x > m64 ? 1 : 0) + (p[q].y > m64 ? 1 : 0);
        }
        const int r64 = ra[0] + ra[1] + ra[2] + ra[3];
        const int tl = __builtin_ctzll(__ballot(r64 == K - 1));
        const uint32_t t_hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(m64 >> 32), tl);
        const uint32_t t_lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)m64, tl);
        const unsigned long long T = ((unsigned long long)t_hi << 32) | t_lo;
        tot = 0;
#pragma unroll
        for (int i = 0; i < EPL; i++) b[i] = __ballot(key[i] >= T);
#pragma unroll
        for (int i = 0; i < EPL; i++) { base[i] = tot; tot += __popcll(b[i]); }
    }
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const bool in = (b[i] >> lane) & 1ull;
        const int pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(b[i] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b[i], base[i]));
        cand[in ? pos : 256 + lane] = key[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    return tot;
}
// rank of candidate key c among the first n candidates (16 per pass, 4 accumulators)
__device__ __forceinline__ int topk_cand_rank(const unsigned long long *cand, int n, unsigned long long c) {
    int ra[4] = {0, 0, 0, 0};
    for (int i0 = 0; i0 < n; i0 += 16) {
        ulonglong2 p[8];
#pragma unroll
        for (int q = 0; q < 8; q++) p[q] = *reinterpret_cast<const ulonglong2 *>(cand + i0 + 2 * q);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            ra[q & 3] += (i0 + 2 * q < n && p[q].x > c) ? 1 : 0;
            ra[(q + 2) & 3] += (i0 + 2 * q + 1 < n && p[q].y > c) ? 1 : 0;
        }
    }
    return ra[0] + ra[1] + ra[2] + ra[3];
}
// Lane k < K receives the k-th expert id and its weight exp(l_k - l_max) /
// denom, denom = sum over the K selected (renorm) or over all E (plain softmax).
template <int EPL>
__device__ __forceinline__ void wave_topk(const float *lr, int K, int renorm, int lane,
                                          unsigned long long *lds, int &my_i, float &my_w) {
    float v[EPL];
    const int n = topk_candidates<EPL>(lr, K, lane, lds, v);
    const unsigned long long *cand = lds + 16;
    for (int j = lane; j < n; j += 64) {
        const unsigned long long cj = cand[j];
        const int r = topk_cand_rank(cand, n, cj);
        if (r < K) lds[r] = cj;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const unsigned long long mine = lane < K ? lds[lane] : 0ull;
    const unsigned long long first = lds[0];
    const float mxv = topk_key_value(first);
    const float ek = lane < K ? __expf(topk_key_value(mine) - mxv) : 0.0f;
    float denom;
    if (renorm) {
        denom = __ockl_wfred_add_f32(ek);
    } else {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; i++) t += __expf(v[i] - mxv);
        denom = __ockl_wfred_add_f32(t);
    }
    my_i = lane < K ? topk_key_index(mine) : -1;
    my_w = ek / denom;
}
// The expert id of rank `job` (< K) only (wave-uniform result): same candidate
// set and ranks as wave_topk, no permutation through LDS and no softmax.
template <int EPL>
__device__ __forceinline__ int wave_topk_one(const float *lr, int K, int job, int lane, unsigned long long *lds) {
    float v[EPL];
    const int n = topk_candidates<EPL>(lr, K, lane, lds, v);
    const unsigned long long *cand = lds + 16;
    int found = -1;
    for (int j = lane; j < n; j += 64) {
        const unsigned long long cj = cand[j];
        if (topk_cand_rank(cand, n, cj) == job) found = topk_key_index(cj);
    }
    return __builtin_amdgcn_readlane(found, __builtin_ctzll(__ballot(found >= 0)));
}

// x slice of one 32-lane group: lane l holds x[st*512 + 16l + i], i < 16.
template <int H>
__device__ __forceinline__ void load_x_slice_bf16(const uint16_t *x, int l, float (&xs)[H / 512][16]) {
#pragma unroll
    for (int st = 0; st < H / 512; st++) {
        const int k0 = st * 512 + l * 16;
        const uint4 a = *reinterpret_cast<const uint4 *>(x + k0);
        const uint4 b = *reinterpret_cast<const uint4 *>(x + k0 + 8);
        const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int q = 0; q < 8; q++) { xs[st][2 * q] = bf16_lo(d[q]); xs[st][2 * q + 1] = bf16_hi(d[q]); }
    }
}
template <int H>
__device__ __forceinline__ void load_x_slice_f32(const float *x, int l, float (&xs)[H / 512][16]) {
#pragma unroll
    for (int st = 0; st < H / 512; st++) {
        const int k0 = st * 512 + l * 16;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = *reinterpret_cast<const float4 *>(x + k0 + 4 * q);
            xs[st][4 * q] = f.x; xs[st][4 * q + 1] = f.y; xs[st][4 * q + 2] = f.z; xs[st][4 * q + 3] = f.w;
        }
    }
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

// NVFP4 chunk: 32 e2m1 values (adjacent pairs: byte i = value 2i low nibble,
// 2i+1 high nibble) with two e4m3 block scales (values 0..15 and 16..31).
// Codes are converted by the gfx950 v_cvt_scalef32_pk_f32_fp4 instruction
// with a unit scale (exact e2m1 values); each 16-value group is scaled once.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float f4_group16(uint32_t lo, uint32_t hi, const float *x) {
    float a = 0.0f;
    const uint32_t w[2] = {lo, hi};
#pragma unroll
    for (int d = 0; d < 2; d++) {
        f32x2_t v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 0);
        f32x2_t v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 1);
        f32x2_t v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 2);
        f32x2_t v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 3);
        a = fmaf(v0.x, x[d * 8 + 0], a); a = fmaf(v0.y, x[d * 8 + 1], a);
        a = fmaf(v1.x, x[d * 8 + 2], a); a = fmaf(v1.y, x[d * 8 + 3], a);
        a = fmaf(v2.x, x[d * 8 + 4], a); a = fmaf(v2.y, x[d * 8 + 5], a);
        a = fmaf(v3.x, x[d * 8 + 6], a); a = fmaf(v3.y, x[d * 8 + 7], a);
    }
    return a;
}
// ue4m3 block scale byte exactly as the reference decodes it
// (ocho/amd_server/qf_nvfp4_wave64.hip:68-73): e = b >> 3 (five bits: bytes
// >= 0x80 are large unsigned scales), m = b & 7; e == 0 -> m * 2^-9, else
// (1 + m/8) * 2^(e-7); 0x7F -> +inf. Not the OCP E4M3 hardware convert, which
// reads bit 7 as a sign and 0x7F as NaN.
__device__ __forceinline__ float e4m3_scale(uint32_t b) {
    b &= 0xFFu;
    const uint32_t e = b >> 3, m = b & 7u;
    const uint32_t bits = b == 0x7Fu ? 0x7F800000u : ((e + 120u) << 23) | (m << 20);
    return e ? __uint_as_float(bits) : (float)m * 0x1p-9f;
}
__device__ __forceinline__ float f4_chunk(uint4 w, uint32_t s2b, const float *x) {
    const float g0 = f4_group16(w.x, w.y, x);
    const float g1 = f4_group16(w.z, w.w, x + 16);
    return fmaf(e4m3_scale(s2b & 0xFFu), g0, e4m3_scale((s2b >> 8) & 0xFFu) * g1);
}

// NVFP4 chunk against bf16 activations: 32 e2m1 codes (w) with two e4m3 block
// scales (s2b) dotted with 32 bf16 values held as 16 packed pairs (xw[i] =
// x[2i] | x[2i+1] << 16, the memory order). gfx950 converts each code pair to
// a bf16 pair (v_cvt_scalef32_pk_bf16_fp4, unit scale: exact) and
// v_dot2_f32_bf16 multiplies a pair with fp32 accumulation (bf16 products
// are exact in fp32), so one conversion and one dot per two weights.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float f4_group16_bx(uint32_t lo, uint32_t hi, const uint32_t *xw) {
    float a = 0.0f;
    const uint32_t w[2] = {lo, hi};
#pragma unroll
    for (int d = 0; d < 2; d++) {
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 0),
                                            __builtin_bit_cast(bf16x2_t, xw[d * 4 + 0]), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 1),
                                            __builtin_bit_cast(bf16x2_t, xw[d * 4 + 1]), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 2),
                                            __builtin_bit_cast(bf16x2_t, xw[d * 4 + 2]), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 3),
                                            __builtin_bit_cast(bf16x2_t, xw[d * 4 + 3]), a, false);
    }
    return a;
}
__device__ __forceinline__ float f4_chunk_bx(uint4 w, uint32_t s2b, const uint32_t *xw) {
    const float g0 = f4_group16_bx(w.x, w.y, xw);
    const float g1 = f4_group16_bx(w.z, w.w, xw + 8);
    return fmaf(e4m3_scale(s2b & 0xFFu), g0, e4m3_scale((s2b >> 8) & 0xFFu) * g1);
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
