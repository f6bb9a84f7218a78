/*
 * qfm_oracle.c -- CPU restatement of the quantized MoE expert path.
 * TEST INFRASTRUCTURE ONLY (see qfm_oracle.h): the checker, never the product.
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).
 */
#include "qfm_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* Philox-4x32-10 (Salmon et al., SC'11), as frozen in the reference:
   stoch/include/philox.cuh:17-35 -- multipliers 0xD2511F53 / 0xCD9E8D57,
   Weyl bumps 0x9E3779B9 / 0xBB67AE85 after every round but the last. */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        const uint64_t p0 = (uint64_t)c0 * 0xD2511F53ull;
        const uint64_t p1 = (uint64_t)c2 * 0xCD9E8D57ull;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        const uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        if (r != 9) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* Word j of the stream (seed, layer, tensor): block j/4 of Philox with
   counter (lo32(j/4), hi32(j/4), tensor, layer) and key (seed, 0). */
uint32_t orc_word(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t j) {
    const uint64_t b = j >> 2;
    const uint32_t ctr[4] = {(uint32_t)b, (uint32_t)(b >> 32), tensor, layer};
    const uint32_t key[2] = {seed, 0u};
    uint32_t o[4];
    orc_philox4x32_10(ctr, key, o);
    return o[j & 3];
}

/* int8 code uniform over [-127, 127]: floor(w * 255 / 2^32) - 127 */
int8_t orc_gen_i8(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n) {
    const uint32_t w = orc_word(seed, layer, tensor, n);
    return (int8_t)((int)(((uint64_t)w * 255u) >> 32) - 127);
}

/* 24-bit uniform u = (w >> 8) * 2^-24, the reference's frozen extractor
   (stoch/include/philox.cuh:57-60). Row scale = (0.5 + u) * 0.02/127,
   evaluated as one fused multiply-add: fma(u, C, C/2). */
#define ORC_ROWSCALE_C  0x1.4a429ap-13f   /* float(0.02f / 127.0f) */
#define ORC_ROWSCALE_CH 0x1.4a429ap-14f   /* C / 2 (exact) */
float orc_gen_rowscale(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n) {
    const uint32_t w = orc_word(seed, layer, tensor, n);
    const float u = (float)(w >> 8) * 0x1p-24f;
    return fmaf(u, ORC_ROWSCALE_C, ORC_ROWSCALE_CH);
}

/* Gaussian by Irwin-Hall: sum of 12 24-bit uniforms (words 12n..12n+11,
   three whole Philox blocks), integer-exact, centred, one int->float rounding. */
float orc_gen_gauss(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n) {
    const uint64_t b0 = n * 3u;
    uint32_t s = 0;
    for (int i = 0; i < 3; i++) {
        const uint64_t b = b0 + (uint64_t)i;
        const uint32_t ctr[4] = {(uint32_t)b, (uint32_t)(b >> 32), tensor, layer};
        const uint32_t key[2] = {seed, 0u};
        uint32_t o[4];
        orc_philox4x32_10(ctr, key, o);
        s += (o[0] >> 8) + (o[1] >> 8) + (o[2] >> 8) + (o[3] >> 8);
    }
    const int32_t c = (int32_t)s - (int32_t)(6u << 24);
    return (float)c * 0x1p-24f;
}

/* packed e2m1 byte: two codes uniform over all 16 (low nibble = element 2i,
   high nibble = element 2i+1, the adjacent-pair order of
   qf_nvfp4_wave64.hip:75-101). */
uint8_t orc_gen_fp4byte(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n) {
    return (uint8_t)(orc_word(seed, layer, tensor, n) >> 24);
}

/* e4m3 block scale: nearest e4m3 of v = 0.25 + 1.75 u, v in [0.25, 2). */
uint8_t orc_gen_e4m3scale(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n) {
    const uint32_t w = orc_word(seed, layer, tensor, n);
    const float u = (float)(w >> 8) * 0x1p-24f;
    return orc_e4m3_encode(fmaf(1.75f, u, 0.25f));
}

void orc_fill_i8(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, int8_t *out) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)cnt; i++) out[i] = orc_gen_i8(seed, layer, tensor, n0 + (uint64_t)i);
}
void orc_fill_rowscale(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, float *out) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)cnt; i++) out[i] = orc_gen_rowscale(seed, layer, tensor, n0 + (uint64_t)i);
}
void orc_fill_gauss(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, float scale, float *out) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)cnt; i++) out[i] = orc_gen_gauss(seed, layer, tensor, n0 + (uint64_t)i) * scale;
}
void orc_fill_gauss_bf16(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, uint16_t *out) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)cnt; i++) out[i] = orc_bf16_rne(orc_gen_gauss(seed, layer, tensor, n0 + (uint64_t)i));
}
void orc_fill_fp4byte(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, uint8_t *out) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)cnt; i++) out[i] = orc_gen_fp4byte(seed, layer, tensor, n0 + (uint64_t)i);
}
void orc_fill_e4m3scale(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, uint8_t *out) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)cnt; i++) out[i] = orc_gen_e4m3scale(seed, layer, tensor, n0 + (uint64_t)i);
}

/* ------------------------------------------------------------------------ */
/* Number formats. E2M1: +-{0, .5, 1, 1.5, 2, 3, 4, 6}[n & 7], sign bit 3
   (qf_nvfp4_wave64.hip:62-67). UE4M3 as the reference decodes the scale
   byte (qf_nvfp4_wave64.hip:68-73): e = b >> 3 (the five high bits: codes
   >= 0x80 are larger unsigned scales, not negative ones), m = b & 7; e == 0
   -> m * 2^-9, else (1 + m/8) * 2^(e-7); 0x7F -> +inf. Written from the
   closed forms with ldexp. */
float orc_e2m1(uint32_t nib) {
    const uint32_t mag = nib & 7u, e = mag >> 1, m = mag & 1u;
    const float v = e ? ldexpf(1.0f + 0.5f * (float)m, (int)e - 1) : 0.5f * (float)m;
    return (nib & 8u) ? -v : v;
}
float orc_e4m3(uint32_t b) {
    const uint32_t e = (b & 0xFFu) >> 3, m = b & 7u;
    if (e == 0) return ldexpf((float)m, -9);
    if (e == 15 && m == 7) return INFINITY;
    return ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
}
uint8_t orc_e4m3_encode(float v) {
    uint32_t bits; memcpy(&bits, &v, 4);
    int e = (int)((bits >> 23) & 0xFF) - 127;
    uint32_t mant = bits & 0x7FFFFFu;
    uint32_t m3 = mant >> 20, rem = mant & 0xFFFFFu;
    if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) m3++;
    if (m3 == 8u) { m3 = 0; e++; }
    return (uint8_t)(((uint32_t)(e + 7) << 3) | m3);
}
uint16_t orc_bf16_rne(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);   /* quiet NaN */
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float orc_bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f; memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------------------ */
/* Router logits in the canonical fp32 order (the order the HIP router
   kernels execute): 64 lane partials, partial l = sequential fma over
   k = j*256 + 4l + c for j = 0..H/256-1, c = 0..3; then a butterfly
   p[l] = p[l] + p[l ^ m] for m = 1, 2, 4, 8, 16, 32. H % 256 == 0.
   Bias (prefill skew) is added last with one rounding. The reference's
   router is a plain fp32 dot (qf_router_wave64.hip:42-51); the order is
   fixed here so that GPU and CPU logits are bit-identical. */
static float canon_dot(const float *w, const float *xf, int H) {
    float p[64], q[64];
    for (int l = 0; l < 64; l++) {
        float a = 0.0f;
        for (int j = 0; j < H / 256; j++)
            for (int c = 0; c < 4; c++) {
                const int k = j * 256 + l * 4 + c;
                a = fmaf(w[k], xf[k], a);
            }
        p[l] = a;
    }
    for (int s = 1; s <= 32; s <<= 1) {
        for (int l = 0; l < 64; l++) q[l] = p[l] + p[l ^ s];
        memcpy(p, q, sizeof p);
    }
    return p[0];
}
void orc_router_logits(const float *W, const uint16_t *x, const float *bias,
                       int M, int E, int H, float *logits) {
    float *xf = (float *)malloc(sizeof(float) * (size_t)M * H);
    for (size_t i = 0; i < (size_t)M * H; i++) xf[i] = orc_bf16_to_f32(x[i]);
    #pragma omp parallel for schedule(static)
    for (int64_t me = 0; me < (int64_t)M * E; me++) {
        const int m = (int)(me / E), e = (int)(me % E);
        float v = canon_dot(W + (size_t)e * H, xf + (size_t)m * H, H);
        if (bias) v = v + bias[e];
        logits[(size_t)m * E + e] = v;
    }
    free(xf);
}

/* Top-K by descending logit, ties -> lower index (qf.cu:1230-1255 ranks
   logits; qf_router_wave64.hip:120-147 the same tie rule). Weights:
   p_e = exp(l_e - max) / sum_all (qf_router_wave64.hip:100-116), then
   renormalized over the selected K (qf_router_wave64.hip:149-154). */
void orc_topk(const float *logits, int M, int E, int K, int renorm,
              int *sel, double *w64, float *w32) {
    unsigned char *taken = (unsigned char *)malloc((size_t)E);
    for (int m = 0; m < M; m++) {
        const float *l = logits + (size_t)m * E;
        memset(taken, 0, (size_t)E);
        for (int k = 0; k < K; k++) {
            int bi = -1;
            for (int e = 0; e < E; e++) {
                if (taken[e]) continue;
                if (bi < 0 || l[e] > l[bi]) bi = e;   /* strict: the lower index wins a tie */
            }
            taken[bi] = 1;
            sel[(size_t)m * K + k] = bi;
        }
        const double mx = (double)l[sel[(size_t)m * K]];
        double denom = 0.0, wsum = 0.0;
        for (int e = 0; e < E; e++) denom += exp((double)l[e] - mx);
        double p[64];
        for (int k = 0; k < K; k++) {
            p[k] = exp((double)l[sel[(size_t)m * K + k]] - mx) / denom;
            wsum += p[k];
        }
        for (int k = 0; k < K; k++) {
            const double w = renorm ? p[k] / wsum : p[k];
            if (w64) w64[(size_t)m * K + k] = w;
            if (w32) w32[(size_t)m * K + k] = (float)w;
        }
    }
    free(taken);
}

/* ------------------------------------------------------------------------ */
/* INT8 expert, exact dequant-matmul in fp64 (reference structure qf8_moe_i8.hip:72-144 with exact activations):
   silu(g) = g / (1 + e^-g) as at qf8_moe_i8.hip:105. */
void orc_i8_expert(const double *x, const int8_t *Qg, const float *sg,
                   const int8_t *Qu, const float *su, const int8_t *Qd, const float *sd,
                   int H, int I, double *h, double *y) {
    for (int r = 0; r < I; r++) {
        double ag = 0.0, au = 0.0;
        const int8_t *wg = Qg + (size_t)r * H, *wu = Qu + (size_t)r * H;
        for (int k = 0; k < H; k++) { ag += (double)wg[k] * x[k]; au += (double)wu[k] * x[k]; }
        const double g = ag * (double)sg[r], u = au * (double)su[r];
        h[r] = g / (1.0 + exp(-g)) * u;
    }
    for (int c = 0; c < H; c++) {
        double a = 0.0;
        const int8_t *wd = Qd + (size_t)c * I;
        for (int r = 0; r < I; r++) a += (double)wd[r] * h[r];
        y[c] = a * (double)sd[c];
    }
}

/* NVFP4: w[r][k] = E2M1(nib(r,k)) * E4M3(S[r][k/16]) * s2, nib(r,k) = low
   nibble of byte k/2 for even k, high nibble for odd k (qf8_moe_i8.hip:170-174). */
void orc_nvfp4_dequant(const uint8_t *F, const uint8_t *S, float s2, int rows, int K, double *out) {
    for (int r = 0; r < rows; r++)
        for (int k = 0; k < K; k++) {
            const uint8_t b = F[(size_t)r * (K / 2) + k / 2];
            const uint32_t nib = (k & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 15u);
            out[(size_t)r * K + k] = (double)orc_e2m1(nib) * (double)orc_e4m3(S[(size_t)r * (K / 16) + k / 16]) * (double)s2;
        }
}
void orc_nvfp4_expert(const double *x, const uint8_t *Fg, const uint8_t *Sg, float s2g,
                      const uint8_t *Fu, const uint8_t *Su, float s2u,
                      const uint8_t *Fd, const uint8_t *Sd, float s2d,
                      int H, int I, double *h, double *y) {
    double *wg = (double *)malloc(sizeof(double) * (size_t)I * H);
    double *wu = (double *)malloc(sizeof(double) * (size_t)I * H);
    double *wd = (double *)malloc(sizeof(double) * (size_t)I * H);
    orc_nvfp4_dequant(Fg, Sg, s2g, I, H, wg);
    orc_nvfp4_dequant(Fu, Su, s2u, I, H, wu);
    orc_nvfp4_dequant(Fd, Sd, s2d, H, I, wd);
    for (int r = 0; r < I; r++) {
        double ag = 0.0, au = 0.0;
        for (int k = 0; k < H; k++) { ag += wg[(size_t)r * H + k] * x[k]; au += wu[(size_t)r * H + k] * x[k]; }
        h[r] = ag / (1.0 + exp(-ag)) * au;
    }
    for (int c = 0; c < H; c++) {
        double a = 0.0;
        for (int r = 0; r < I; r++) a += wd[(size_t)c * I + r] * h[r];
        y[c] = a;
    }
    free(wg); free(wu); free(wd);
}

/* X8: per 32-block s = absmax/127 (1 if absmax == 0), q = clamp(rint(v/s), +-127)
   (qf8_moe_i8.hip:58-70). */
void orc_x8_quant(const float *v, int n, int8_t *q, float *s) {
    for (int b = 0; b < n / 32; b++) {
        float mx = 0.0f;
        for (int i = 0; i < 32; i++) mx = fmaxf(mx, fabsf(v[b * 32 + i]));
        const float sc = mx > 0.0f ? mx * (1.0f / 127.0f) : 1.0f;
        for (int i = 0; i < 32; i++) {
            int qi = (int)rintf(v[b * 32 + i] / sc);
            qi = qi > 127 ? 127 : (qi < -127 ? -127 : qi);
            q[b * 32 + i] = (int8_t)qi;
        }
        s[b] = sc;
    }
}

/* NVFP4 -> INT8 arena conversion (qf8_moe_i8.hip:146-195): for each row,
   v_k = e2m1(nibble k) * ue4m3(scale byte k/16) * s2 in fp32, multiplied in
   that order; scale = absmax * (1/127) (1 when every v is zero); code =
   rint(v * (1/scale)) clamped to +-127. The scale decode is orc_e4m3 (the
   exponent read as byte >> 3, qf8_moe_i8.hip:154-159). */
void orc_nvfp4_to_i8(const uint8_t *W, const uint8_t *S, float s2, int rows, int K, int8_t *Wo, float *So) {
    float *v = (float *)malloc((size_t)K * sizeof(float));
    for (int r = 0; r < rows; r++) {
        float mx = 0.0f;
        for (int k = 0; k < K; k++) {
            const uint32_t byte = W[(size_t)r * (K / 2) + k / 2];
            const uint32_t nib = (k & 1) ? (byte >> 4) : (byte & 15u);
            const float a = orc_e2m1(nib) * orc_e4m3(S[(size_t)r * (K / 16) + k / 16]);
            v[k] = a * s2;
            mx = fmaxf(mx, fabsf(v[k]));
        }
        const float scale = mx > 0.0f ? mx * (1.0f / 127.0f) : 1.0f;
        const float inv = 1.0f / scale;
        for (int k = 0; k < K; k++) {
            int q = (int)rintf(v[k] * inv);
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            Wo[(size_t)r * K + k] = (int8_t)q;
        }
        So[r] = scale;
    }
    free(v);
}

/* Dense bf16 -> INT8 per-row (qf8_dense_i8.hip:41-60): scale = absmax / 127
   (IEEE division; 1 for an all-zero row), inv = 1 / scale, code =
   rint(w * inv) clamped to +-127. */
void orc_i8_quant_bf16(const uint16_t *W, int rows, int K, int8_t *Wo, float *So) {
    for (int r = 0; r < rows; r++) {
        float mx = 0.0f;
        for (int k = 0; k < K; k++) mx = fmaxf(mx, fabsf(orc_bf16_to_f32(W[(size_t)r * K + k])));
        const float scale = mx > 0.0f ? mx / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        for (int k = 0; k < K; k++) {
            int q = (int)rintf(orc_bf16_to_f32(W[(size_t)r * K + k]) * inv);
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            Wo[(size_t)r * K + k] = (int8_t)q;
        }
        So[r] = scale;
    }
}

/* FP8 lane-chunk format (qf8_moe_fp8.hip:19-37, :217-246).
   Decode: sign bit 7, exponent bits 6..3 (bias 7), mantissa bits 2..0;
   exponent 0 is m * 2^-9; no NaN or infinity (0x7F reads 480).
   Encode: |v| < 2^-9 (unbiased exponent < -9) -> signed zero; exponent >= 8
   -> 0x7E (448) with the sign; exponents -9..-7 -> subnormal code, mantissa
   truncated; otherwise 3-bit mantissa rounded to nearest even, a carry into
   exponent 8 saturating to 0x7E. */
float orc_f8_decode(uint8_t b) {
    const uint32_t x = b, sgn = (x & 0x80u) << 24, e = (x >> 3) & 0xFu, m = x & 7u;
    float v;
    if (e == 0) {
        v = (float)m * 0.001953125f;
        uint32_t u;
        memcpy(&u, &v, 4);
        u |= sgn;
        memcpy(&v, &u, 4);
        return v;
    }
    const uint32_t u = sgn | ((e + 120u) << 23) | (m << 20);
    memcpy(&v, &u, 4);
    return v;
}

uint8_t orc_f8_encode(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    const uint32_t sgn = (u >> 24) & 0x80u;
    int e = (int)((u >> 23) & 0xFFu) - 127;
    const uint32_t m = u & 0x7FFFFFu;
    if (e < -9) return (uint8_t)sgn;
    if (e >= 8) return (uint8_t)(sgn | 0x7Eu);
    if (e < -6) {
        const int sh = -6 - e;
        return (uint8_t)(sgn | (((m | 0x800000u) >> (sh + 20)) & 7u));
    }
    uint32_t mm = m >> 20;
    const uint32_t rem = m & 0xFFFFFu;
    if (rem > 0x80000u || (rem == 0x80000u && (mm & 1u))) {
        mm++;
        if (mm == 8u) {
            mm = 0;
            e++;
            if (e >= 8) return (uint8_t)(sgn | 0x7Eu);
        }
    }
    return (uint8_t)(sgn | (uint32_t)((e + 7) << 3) | (mm & 7u));
}

/* The packer's block-scale decode (qf8_moe_fp8.hip:231-234): e = b >> 3 (five
   bits), m = b & 7; e == 0 -> m * 2^-9, else (1 + m/8) * 2^(e-7). Unlike
   orc_e4m3 there is no infinity: 0x7F reads 480. */
static float orc_f8_block_scale(uint32_t b) {
    const uint32_t e = (b & 0xFFu) >> 3, m = b & 7u;
    return e ? ldexpf(1.0f + (float)m / 8.0f, (int)e - 7) : ldexpf((float)m, -9);
}

/* NVFP4 expert matrix rows x in -> lane-chunk E4M3: chunk l of row r holds
   values v = e2m1(nibble) * (block scale * s2) (orc_f8_block_scale), sc[r][l]
   = max|v| / 448 (1 for an all-zero chunk), code = orc_f8_encode(v / sc). */
void orc_fp8_pack_expert(const uint8_t *W, const uint8_t *S, float s2, int rows, int in, uint8_t *w8, float *sc) {
    const int ch = in / 64;
    float *v = (float *)malloc((size_t)ch * sizeof(float));
    for (int r = 0; r < rows; r++)
        for (int l = 0; l < 64; l++) {
            float mx = 0.0f;
            for (int c = 0; c < ch; c++) {
                const int k = l * ch + c;
                const uint32_t byte = W[(size_t)r * (in / 2) + k / 2];
                const uint32_t nib = (k & 1) ? (byte >> 4) : (byte & 15u);
                const float bs = orc_f8_block_scale(S[(size_t)r * (in / 16) + k / 16]);
                v[c] = orc_e2m1(nib) * (bs * s2);
                const float a = fabsf(v[c]);
                if (a > mx) mx = a;
            }
            const float scale = mx > 0.0f ? mx / 448.0f : 1.0f;
            sc[(size_t)r * 64 + l] = scale;
            for (int c = 0; c < ch; c++) w8[(size_t)r * in + (size_t)l * ch + c] = orc_f8_encode(v[c] / scale);
        }
    free(v);
}

/* INT8 x X8 GEMV (qf8_dense_i8.hip:78-103): y[r] = act(s[r] * sum_b xs[b] *
   (W[r] . xq)[32-block b]); each block dot is an exact integer, the sum over
   blocks is taken in fp64 here. act 0 none, 1 silu(v/4), 2 2*sigmoid(v/4). */
void orc_i8_gemv(const int8_t *W, const float *s, int rows, int K, const int8_t *xq, const float *xs, int act,
                 double *y) {
    for (int r = 0; r < rows; r++) {
        double acc = 0.0;
        for (int b = 0; b < K / 32; b++) {
            long d = 0;
            for (int k = b * 32; k < b * 32 + 32; k++) d += (long)W[(size_t)r * K + k] * (long)xq[k];
            acc += (double)d * (double)xs[b];
        }
        double v = acc * (double)s[r];
        if (act == 1) v = (v * 0.25) / (1.0 + exp(-v * 0.25));
        else if (act == 2) v = 2.0 / (1.0 + exp(-v * 0.25));
        y[r] = v;
    }
}

/* Zero-centered grouped RMS norm of the hyper-connection (qf8_dense_i8.hip:
   109-149), one stream of H values, fp64: normed = R * rstd * (1 + w),
   rstd = 1 / sqrt(mean(R^2) + 1e-6), w bf16. */
void orc_hc_norm(const float *R, const uint16_t *w, int H, double *normed) {
    double ss = 0.0;
    for (int i = 0; i < H; i++) ss += (double)R[i] * (double)R[i];
    const double rstd = 1.0 / sqrt(ss / H + 1e-6);
    for (int i = 0; i < H; i++) normed[i] = (double)R[i] * rstd * (1.0 + (double)orc_bf16_to_f32(w[i]));
}

/* Stream combine (qf8_dense_i8.hip:151-175), fp64: mixed[j] = 1/4 sum_c
   sigmoid(hcy[c*H + j]) * normed[c*H + j]. */
void orc_hc_combine(const float *hcy, const float *normed, int H, double *mixed) {
    for (int j = 0; j < H; j++) {
        double sum = 0.0;
        for (int c = 0; c < 4; c++) sum += (1.0 / (1.0 + exp(-(double)hcy[c * H + j]))) * (double)normed[c * H + j];
        mixed[j] = 0.25 * sum;
    }
}

/* Residual-stream inject (qf8_hc.hip:99-103): R[c*H + i] += inj[c] * y[i],
   one fused multiply-add (the compiled form of the reference expression). */
void orc_stream_inject(float *R, const float *y, const float *inj, int H) {
    for (int c = 0; c < 4; c++)
        for (int i = 0; i < H; i++) R[c * H + i] = fmaf(inj[c], y[i], R[c * H + i]);
}

/* The bf16 shared expert of the NVFP4 stage (qf8_layer.hip:23-54, weights
   Qf8ShexpW qf8_dense.h:275-277), fp64: eu = up . x, g1 = gate_inp . x,
   eg = silu(gate . x) * eu (k8_silu_mul, :8-12), ed = down . eg,
   y += sigmoid(g1) * ed (k8_shexp_add, :14-18), per row m < M. */
void orc_shexp_bf16(const uint16_t *gate, const uint16_t *up, const uint16_t *down, const uint16_t *gate_inp,
                    const float *x, int M, int H, int I, double *eg, double *eu, double *g1, double *ed, double *y) {
    for (int m = 0; m < M; m++) {
        const float *xm = x + (size_t)m * H;
        double gi = 0.0;
        for (int k = 0; k < H; k++) gi += (double)orc_bf16_to_f32(gate_inp[k]) * (double)xm[k];
        g1[m] = gi;
        for (int r = 0; r < I; r++) {
            double g = 0.0, u = 0.0;
            for (int k = 0; k < H; k++) {
                g += (double)orc_bf16_to_f32(gate[(size_t)r * H + k]) * (double)xm[k];
                u += (double)orc_bf16_to_f32(up[(size_t)r * H + k]) * (double)xm[k];
            }
            eu[(size_t)m * I + r] = u;
            eg[(size_t)m * I + r] = g / (1.0 + exp(-g)) * u;
        }
        const double sg = 1.0 / (1.0 + exp(-gi));
        for (int o = 0; o < H; o++) {
            double d = 0.0;
            for (int r = 0; r < I; r++) d += (double)orc_bf16_to_f32(down[(size_t)o * I + r]) * eg[(size_t)m * I + r];
            ed[(size_t)m * H + o] = d;
            y[(size_t)m * H + o] += sg * d;
        }
    }
}

/* Four-card combine: y[i] = ((y0[i] + y1[i]) + y2[i]) + y3[i], fp32, the
   left-to-right order of k_m8_reduce4 (qf_moe_m8_wave64.hip:216-221). */
void orc_m8_reduce4(float *y, const float *y0, const float *y1, const float *y2, const float *y3, long n) {
    for (long i = 0; i < n; i++) {
        float a = y0[i] + y1[i];
        a = a + y2[i];
        y[i] = a + y3[i];
    }
}

/* Routing inversion: experts ascending; within an expert, pairs in (token, k)
   order (qf8_moe_i8.hip:323-358; qf_moe_m8_wave64.hip:261-299). */
int orc_csr_build(const int *sel, const float *wt, int T, int K, int E,
                  int *exp_ids, int *exp_ptr, int *pair_tok, int *pair_k, float *pair_wt,
                  int *n_pairs) {
    int *cnt = (int *)calloc((size_t)E, sizeof(int));
    for (int p = 0; p < T * K; p++) {
        const int e = sel[p];
        if (e < 0 || e >= E) { free(cnt); return -1; }
        cnt[e]++;
    }
    int n = 0, off = 0;
    int *start = (int *)malloc(sizeof(int) * (size_t)E);
    for (int e = 0; e < E; e++) {
        start[e] = off;
        if (cnt[e]) { exp_ids[n] = e; exp_ptr[n] = off; n++; }
        off += cnt[e];
    }
    exp_ptr[n] = off;
    for (int t = 0; t < T; t++)
        for (int k = 0; k < K; k++) {
            const int e = sel[t * K + k], w = start[e]++;
            pair_tok[w] = t; pair_k[w] = k; pair_wt[w] = wt[t * K + k];
        }
    *n_pairs = off;
    free(cnt); free(start);
    return n;
}

/* ------------------------------------------------------------------------ */
static void gen_i8_expert(const orc_layer_cfg *c, int e, int8_t *qg, float *sg,
                          int8_t *qu, float *su, int8_t *qd, float *sd) {
    const uint64_t H = (uint64_t)c->H, I = (uint64_t)c->I;
    orc_fill_i8(c->seed, c->layer, ORC_T_QG, (uint64_t)e * I * H, I * H, qg);
    orc_fill_i8(c->seed, c->layer, ORC_T_QU, (uint64_t)e * I * H, I * H, qu);
    orc_fill_i8(c->seed, c->layer, ORC_T_QD, (uint64_t)e * H * I, H * I, qd);
    orc_fill_rowscale(c->seed, c->layer, ORC_T_SG, (uint64_t)e * I, I, sg);
    orc_fill_rowscale(c->seed, c->layer, ORC_T_SU, (uint64_t)e * I, I, su);
    orc_fill_rowscale(c->seed, c->layer, ORC_T_SD, (uint64_t)e * H, H, sd);
}

int orc_moe_layer(const orc_layer_cfg *c, int M, uint16_t *x_out, float *logits,
                  int *sel, double *w64, double *y64, uint16_t *ybf16) {
    const int H = c->H, I = c->I, E = c->E, K = c->K;
    if (H % 256 || I % 32 || K > 64 || K > E) return -1;
    uint16_t *x = x_out ? x_out : (uint16_t *)malloc(sizeof(uint16_t) * (size_t)M * H);
    orc_fill_gauss_bf16(c->seed, c->x_layer, ORC_T_X, (uint64_t)c->x_row0 * H, (uint64_t)M * H, x);
    float *W = (float *)malloc(sizeof(float) * (size_t)E * H);
    orc_fill_gauss(c->seed, c->layer, ORC_T_ROUTER, 0, (uint64_t)E * H, 0.02f, W);
    float *bias = NULL;
    if (c->use_bias) {
        bias = (float *)malloc(sizeof(float) * (size_t)E);
        orc_fill_gauss(c->seed, c->layer, ORC_T_BIAS, 0, (uint64_t)E, 1.5f, bias);
    }
    float *lg = logits ? logits : (float *)malloc(sizeof(float) * (size_t)M * E);
    orc_router_logits(W, x, bias, M, E, H, lg);
    orc_topk(lg, M, E, K, c->renorm, sel, w64, NULL);

    float *g = (float *)malloc(sizeof(float) * (size_t)H);
    orc_fill_gauss(c->seed, c->layer, ORC_T_SHGATE, 0, (uint64_t)H, 0.02f, g);
    int8_t *qg = (int8_t *)malloc((size_t)I * H), *qu = (int8_t *)malloc((size_t)I * H), *qd = (int8_t *)malloc((size_t)I * H);
    float *sg = (float *)malloc(4 * (size_t)I), *su = (float *)malloc(4 * (size_t)I), *sd = (float *)malloc(4 * (size_t)H);
    uint8_t *fg = NULL, *fu = NULL, *fd = NULL, *fsg = NULL, *fsu = NULL, *fsd = NULL;
    if (c->fmt == 1) {
        fg = (uint8_t *)malloc((size_t)I * H / 2); fu = (uint8_t *)malloc((size_t)I * H / 2); fd = (uint8_t *)malloc((size_t)I * H / 2);
        fsg = (uint8_t *)malloc((size_t)I * H / 16); fsu = (uint8_t *)malloc((size_t)I * H / 16); fsd = (uint8_t *)malloc((size_t)I * H / 16);
    }
    double *xd = (double *)malloc(sizeof(double) * (size_t)H), *h = (double *)malloc(sizeof(double) * (size_t)I);
    double *ye = (double *)malloc(sizeof(double) * (size_t)H);
    for (int m = 0; m < M; m++)
        for (int k = 0; k < H; k++) y64[(size_t)m * H + k] = 0.0;

    /* routed experts: visit each distinct expert once, in ascending order */
    unsigned char *used = (unsigned char *)calloc((size_t)E, 1);
    for (int p = 0; p < M * K; p++) used[sel[p]] = 1;
    for (int e = 0; e < E; e++) {
        if (!used[e]) continue;
        const uint64_t IH = (uint64_t)I * H;
        if (c->fmt == 0) {
            gen_i8_expert(c, e, qg, sg, qu, su, qd, sd);
        } else {
            orc_fill_fp4byte(c->seed, c->layer, ORC_T_FG, (uint64_t)e * IH / 2, IH / 2, fg);
            orc_fill_fp4byte(c->seed, c->layer, ORC_T_FU, (uint64_t)e * IH / 2, IH / 2, fu);
            orc_fill_fp4byte(c->seed, c->layer, ORC_T_FD, (uint64_t)e * IH / 2, IH / 2, fd);
            orc_fill_e4m3scale(c->seed, c->layer, ORC_T_FSG, (uint64_t)e * IH / 16, IH / 16, fsg);
            orc_fill_e4m3scale(c->seed, c->layer, ORC_T_FSU, (uint64_t)e * IH / 16, IH / 16, fsu);
            orc_fill_e4m3scale(c->seed, c->layer, ORC_T_FSD, (uint64_t)e * IH / 16, IH / 16, fsd);
        }
        /* a row selects an expert at most once: the rows of one expert are
           distinct, so the pairs of this expert run in parallel */
        #pragma omp parallel for schedule(dynamic)
        for (int mk = 0; mk < M * K; mk++) {
            if (sel[mk] != e) continue;
            const int m = mk / K;
            double *xl = (double *)malloc(sizeof(double) * (size_t)H);
            double *hl = (double *)malloc(sizeof(double) * (size_t)I);
            double *yl = (double *)malloc(sizeof(double) * (size_t)H);
            for (int i = 0; i < H; i++) xl[i] = (double)orc_bf16_to_f32(x[(size_t)m * H + i]);
            if (c->fmt == 0) orc_i8_expert(xl, qg, sg, qu, su, qd, sd, H, I, hl, yl);
            else orc_nvfp4_expert(xl, fg, fsg, 0.01f, fu, fsu, 0.01f, fd, fsd, 0.01f, H, I, hl, yl);
            const double w = w64[mk];
            for (int i = 0; i < H; i++) y64[(size_t)m * H + i] += w * yl[i];
            free(xl); free(hl); free(yl);
        }
    }
    /* shared expert (index E of the generator), always INT8 */
    gen_i8_expert(c, E, qg, sg, qu, su, qd, sd);
    #pragma omp parallel for schedule(dynamic)
    for (int m = 0; m < M; m++) {
        double *xl = (double *)malloc(sizeof(double) * (size_t)H);
        double *hl = (double *)malloc(sizeof(double) * (size_t)I);
        double *yl = (double *)malloc(sizeof(double) * (size_t)H);
        double gx = 0.0;
        for (int i = 0; i < H; i++) {
            xl[i] = (double)orc_bf16_to_f32(x[(size_t)m * H + i]);
            gx += (double)g[i] * xl[i];
        }
        orc_i8_expert(xl, qg, sg, qu, su, qd, sd, H, I, hl, yl);
        const double gam = c->gated ? 1.0 / (1.0 + exp(-gx)) : 1.0;
        for (int i = 0; i < H; i++) y64[(size_t)m * H + i] += gam * yl[i];
        free(xl); free(hl); free(yl);
    }
    if (ybf16)
        for (size_t i = 0; i < (size_t)M * H; i++) ybf16[i] = orc_bf16_rne((float)y64[i]);

    free(used); free(xd); free(h); free(ye); free(g);
    free(qg); free(qu); free(qd); free(sg); free(su); free(sd);
    free(fg); free(fu); free(fd); free(fsg); free(fsu); free(fsd);
    if (!logits) free(lg);
    free(bias); free(W);
    if (!x_out) free(x);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* CPU baseline: the same layer in fp32 accumulate over a resident host
   arena, parallel over output rows. Router in the canonical order. */
static float silu_f(float g) { return g / (1.0f + expf(-g)); }
void orc_cpu_moe_layer_fast(const orc_host_layer *L, int H, int I, int E, int K,
                            const uint16_t *x, int M, float *y, int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    float *lg = (float *)malloc(sizeof(float) * (size_t)M * E);
    float *xf = (float *)malloc(sizeof(float) * (size_t)M * H);
    for (size_t i = 0; i < (size_t)M * H; i++) xf[i] = orc_bf16_to_f32(x[i]);
    #pragma omp parallel for schedule(static)
    for (int me = 0; me < M * E; me++) {
        const int m = me / E, e = me % E;
        lg[me] = canon_dot(L->router + (size_t)e * H, xf + (size_t)m * H, H);
    }
    int *sel = (int *)malloc(sizeof(int) * (size_t)M * (K + 1));
    float *wt = (float *)malloc(sizeof(float) * (size_t)M * (K + 1));
    int *selk = (int *)malloc(sizeof(int) * (size_t)M * K);
    float *wk = (float *)malloc(sizeof(float) * (size_t)M * K);
    orc_topk(lg, M, E, K, 1, selk, NULL, wk);
    for (int m = 0; m < M; m++) {
        float gx = 0.0f;
        for (int i = 0; i < H; i++) gx += L->shgate[i] * xf[(size_t)m * H + i];
        for (int k = 0; k < K; k++) { sel[m * (K + 1) + k] = selk[m * K + k]; wt[m * (K + 1) + k] = wk[m * K + k]; }
        sel[m * (K + 1) + K] = E;
        wt[m * (K + 1) + K] = 1.0f / (1.0f + expf(-gx));
    }
    const int NE = K + 1;
    float *h = (float *)malloc(sizeof(float) * (size_t)M * NE * I);
    #pragma omp parallel for schedule(static)
    for (int idx = 0; idx < M * NE * I; idx++) {
        const int r = idx % I, mk = idx / I, m = mk / NE;
        const int e = sel[mk];
        const int8_t *wg = L->qg + ((size_t)e * I + r) * H, *wu = L->qu + ((size_t)e * I + r) * H;
        const float *xv = xf + (size_t)m * H;
        float ag = 0.0f, au = 0.0f;
        for (int k = 0; k < H; k++) { ag += (float)wg[k] * xv[k]; au += (float)wu[k] * xv[k]; }
        const float g = ag * L->sg[(size_t)e * I + r], u = au * L->su[(size_t)e * I + r];
        h[idx] = silu_f(g) * u;
    }
    #pragma omp parallel for schedule(static)
    for (int mc = 0; mc < M * H; mc++) {
        const int m = mc / H, c = mc % H;
        float tot = 0.0f;
        for (int k = 0; k < NE; k++) {
            const int e = sel[m * NE + k];
            const int8_t *wd = L->qd + ((size_t)e * H + c) * I;
            const float *hv = h + ((size_t)m * NE + k) * I;
            float a = 0.0f;
            for (int r = 0; r < I; r++) a += (float)wd[r] * hv[r];
            tot += wt[m * NE + k] * a * L->sd[(size_t)e * H + c];
        }
        y[mc] = tot;
    }
    free(h); free(sel); free(wt); free(selk); free(wk); free(lg); free(xf);
}
