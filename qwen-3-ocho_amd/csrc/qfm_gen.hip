// qfm_gen.hip -- on-device synthetic data generator.
//
// Every element is a pure function of (seed, layer, tensor, index): word j
// of a stream is word (j & 3) of Philox-4x32-10 with counter
// (lo32(j >> 2), hi32(j >> 2), tensor, layer) and key (seed, 0). Integer
// work is exact and the few float steps are single correctly rounded ops
// written as explicit fmaf / int->float conversions, so the host restatement
// regenerates the same bits. The 24-bit uniform u = (w >> 8) * 2^-24 is the
// reference's extractor (stoch/include/philox.cuh:57-60).
#include "qfm_dev.h"
#include "qfm_internal.h"

namespace qfm {

__device__ __forceinline__ u4 stream_block(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t b) {
    return philox((uint32_t)b, (uint32_t)(b >> 32), tensor, layer, seed, 0u);
}

__device__ __forceinline__ float gauss_at(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n) {
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const u4 o = stream_block(seed, layer, tensor, n * 3u + (uint64_t)i);
        s += (o.v[0] >> 8) + (o.v[1] >> 8) + (o.v[2] >> 8) + (o.v[3] >> 8);
    }
    const int32_t c = (int32_t)s - (int32_t)(6u << 24);
    return __int2float_rn(c) * 0x1p-24f;
}

__device__ __forceinline__ uint32_t e4m3_encode_pos(float v) {
    const uint32_t bits = __float_as_uint(v);
    int e = (int)((bits >> 23) & 0xFFu) - 127;
    const uint32_t mant = bits & 0x7FFFFFu;
    uint32_t m3 = mant >> 20;
    const uint32_t rem = mant & 0xFFFFFu;
    if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) m3++;
    if (m3 == 8u) { m3 = 0; e++; }
    return ((uint32_t)(e + 7) << 3) | m3;
}

constexpr float kRowScaleC = 0x1.4a429ap-13f;   // float(0.02f / 127.0f)
constexpr float kRowScaleCH = 0x1.4a429ap-14f;  // C / 2

__global__ void __launch_bounds__(256)
k_gen_words(void *out, int kind, uint64_t n0, uint64_t cnt, uint32_t seed, uint32_t layer, uint32_t tensor) {
    const uint64_t b_first = n0 >> 2, b_last = (n0 + cnt - 1) >> 2;
    const uint64_t nb = b_last - b_first + 1;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nb;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t b = b_first + i;
        const u4 o = stream_block(seed, layer, tensor, b);
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint64_t j = b * 4u + (uint64_t)w;
            if (j < n0 || j >= n0 + cnt) continue;
            const uint64_t d = j - n0;
            const uint32_t wd = o.v[w];
            switch (kind) {
            case QFM_GEN_I8:
                ((int8_t *)out)[d] = (int8_t)((int)(((uint64_t)wd * 255u) >> 32) - 127);
                break;
            case QFM_GEN_ROWSCALE: {
                const float u = __uint2float_rn(wd >> 8) * 0x1p-24f;
                ((float *)out)[d] = __fmaf_rn(u, kRowScaleC, kRowScaleCH);
                break;
            }
            case QFM_GEN_FP4BYTE:
                ((uint8_t *)out)[d] = (uint8_t)(wd >> 24);
                break;
            case QFM_GEN_E4M3SCALE: {
                const float u = __uint2float_rn(wd >> 8) * 0x1p-24f;
                ((uint8_t *)out)[d] = (uint8_t)e4m3_encode_pos(__fmaf_rn(1.75f, u, 0.25f));
                break;
            }
            default: break;
            }
        }
    }
}

__global__ void __launch_bounds__(256)
k_gen_gauss(void *out, int bf16, uint64_t n0, uint64_t cnt, uint32_t seed, uint32_t layer,
            uint32_t tensor, float scale) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cnt;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const float z = gauss_at(seed, layer, tensor, n0 + i);
        if (bf16) ((uint16_t *)out)[i] = f32_to_bf16(z);
        else ((float *)out)[i] = __fmul_rn(z, scale);
    }
}

__global__ void k_fill_f32(float *out, uint64_t cnt, float v) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < cnt;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = v;
}

static unsigned grid_for(uint64_t items) {
    const uint64_t g = (items + 255) / 256;
    return (unsigned)(g < 65536 ? (g ? g : 1) : 65536);
}

int launch_gen_fill(void *out, int kind, uint64_t n0, uint64_t cnt, uint32_t seed, uint32_t layer,
                    uint32_t tensor, float scale, hipStream_t s) {
    if (!out) { set_error(-1, "qfm_gen_fill: null output"); return -1; }
    if (cnt == 0) return 0;
    switch (kind) {
    case QFM_GEN_I8: case QFM_GEN_ROWSCALE: case QFM_GEN_FP4BYTE: case QFM_GEN_E4M3SCALE: {
        const uint64_t nb = ((n0 + cnt - 1) >> 2) - (n0 >> 2) + 1;
        hipLaunchKernelGGL(k_gen_words, dim3(grid_for(nb)), dim3(256), 0, s, out, kind, n0, cnt, seed, layer, tensor);
        break;
    }
    case QFM_GEN_GAUSS_F32: case QFM_GEN_GAUSS_BF16:
        hipLaunchKernelGGL(k_gen_gauss, dim3(grid_for(cnt)), dim3(256), 0, s, out,
                           kind == QFM_GEN_GAUSS_BF16 ? 1 : 0, n0, cnt, seed, layer, tensor, scale);
        break;
    default:
        set_error(-1, "qfm_gen_fill: unknown kind %d", kind);
        return -1;
    }
    return check_launch("qfm_gen_fill");
}

int launch_fill_f32(float *out, uint64_t cnt, float value, hipStream_t s) {
    if (!out) { set_error(-1, "qfm_fill_f32: null output"); return -1; }
    if (!cnt) return 0;
    hipLaunchKernelGGL(k_fill_f32, dim3(grid_for(cnt)), dim3(256), 0, s, out, cnt, value);
    return check_launch("qfm_fill_f32");
}

}  // namespace qfm
