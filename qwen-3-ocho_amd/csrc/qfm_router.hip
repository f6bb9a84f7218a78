// qfm_router.hip -- router GEMV and softmax/top-k selection.
//
// Reference behaviour: qf_rtr_gemv (ocho/amd_server/qf_router_wave64.hip:42-51),
// qf_rtr_topk10 (:69-155), Spark k_router_topk (ocho/engine_spark/cuda/qf.cu:1184-1271).
//
// Router logits are produced in one canonical fp32 order so that the host
// restatement reproduces them bit for bit: lane l of a wave owns elements
// k = j*256 + 4l + c (j = 0..H/256-1, c = 0..3) of the row and accumulates
// them with a sequential fmaf chain in (j, c) order; the 64 lane partials
// are then combined by an xor butterfly p[l] = p[l] + p[l ^ m], m = 32..1.
// Each lane's weights arrive as H/256 coalesced 16-byte loads (1 KiB per
// wave per load), so a router row is one wave and E rows are E waves.
//
// Top-k ranks the fp32 logits (monotone in the softmax probabilities, as the
// Spark router does, qf.cu:1230-1255), ties to the lower expert index; the
// selected weights are exp(l - max) renormalized over the K selected
// (norm_topk_prob, qf_router_wave64.hip:149-154) or divided by the full
// softmax denominator when renorm = 0.
#include "qfm_dev.h"
#include "qfm_internal.h"

namespace qfm {

template <int NJ>
__device__ __forceinline__ float canon_reduce_row(const float4 (&w)[NJ], const float (&x)[NJ][4]) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        a = __fmaf_rn(w[j].x, x[j][0], a);
        a = __fmaf_rn(w[j].y, x[j][1], a);
        a = __fmaf_rn(w[j].z, x[j][2], a);
        a = __fmaf_rn(w[j].w, x[j][3], a);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) a = __fadd_rn(a, __shfl_xor(a, m, WAVE));
    return a;
}

// W fp32 [E][H]; x bf16 [M][H]; logits [M][ld]. Row E (when g != nullptr)
// is the shared-expert gate vector g [H], written to column E without bias.
template <int NJ>
__global__ void __launch_bounds__(256)
k_router_f32w(const float *__restrict__ W, const float *__restrict__ bias, const float *__restrict__ g,
              const uint16_t *__restrict__ x, int M, int E, float *__restrict__ logits, int ld) {
    constexpr int H = NJ * 256;
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
    const bool is_g = (g != nullptr) && e == E;
    if (e > E || (e == E && !is_g)) return;
    const float *wr = is_g ? g : W + (size_t)e * H;
    float4 w[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) w[j] = *reinterpret_cast<const float4 *>(wr + j * 256 + lane * 4);
    const float b = (!is_g && bias) ? bias[e] : 0.0f;
    const int m0 = blockIdx.y * 8, m1 = min(M, m0 + 8);
    for (int m = m0; m < m1; m++) {
        float xv[NJ][4];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint2 p = *reinterpret_cast<const uint2 *>(x + (size_t)m * H + j * 256 + lane * 4);
            xv[j][0] = bf16_lo(p.x); xv[j][1] = bf16_hi(p.x);
            xv[j][2] = bf16_lo(p.y); xv[j][3] = bf16_hi(p.y);
        }
        float a = canon_reduce_row<NJ>(w, xv);
        if (bias && !is_g) a = __fadd_rn(a, b);
        if (lane == 0) logits[(size_t)m * ld + e] = a;
    }
}

// Reference form: W bf16 [E][H], x fp32 [H] (qf_rtr_gemv signature).
template <int NJ>
__global__ void __launch_bounds__(256)
k_router_bf16w(const uint16_t *__restrict__ W, const float *__restrict__ x, int E, float *__restrict__ logits) {
    constexpr int H = NJ * 256;
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (e >= E) return;
    float4 w[NJ];
    float xv[NJ][4];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint2 p = *reinterpret_cast<const uint2 *>(W + (size_t)e * H + j * 256 + lane * 4);
        w[j] = make_float4(bf16_lo(p.x), bf16_hi(p.x), bf16_lo(p.y), bf16_hi(p.y));
        const float4 xx = *reinterpret_cast<const float4 *>(x + j * 256 + lane * 4);
        xv[j][0] = xx.x; xv[j][1] = xx.y; xv[j][2] = xx.z; xv[j][3] = xx.w;
    }
    const float a = canon_reduce_row<NJ>(w, xv);
    if (lane == 0) logits[e] = a;
}

// One wave per row: EPL = E/64 logits per lane (lane l holds e = i*64 + l).
template <int EPL>
__global__ void __launch_bounds__(256)
k_topk(const float *__restrict__ logits, int ld, int M, int K, int renorm,
       int *__restrict__ sel, float *__restrict__ wts) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    const float *lr = logits + (size_t)m * ld;
    float v[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) v[i] = lr[i * 64 + lane];
    uint32_t taken = 0;
    float my_v = 0.0f, mx = 0.0f;
    int my_i = 0;
    for (int k = 0; k < K; k++) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int e = i * 64 + lane;
            if (!((taken >> i) & 1u) && (v[i] > bv || (v[i] == bv && e < bi))) { bv = v[i]; bi = e; }
        }
#pragma unroll
        for (int msk = 32; msk >= 1; msk >>= 1) {
            const float ov = __shfl_xor(bv, msk, WAVE);
            const int oi = __shfl_xor(bi, msk, WAVE);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (k == 0) mx = bv;
        if (lane == k) { my_v = bv; my_i = bi; }
    }
    const float ek = lane < K ? __expf(my_v - mx) : 0.0f;
    float denom;
    if (renorm) {
        denom = group_sum<64>(ek);
    } else {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; i++) s += __expf(v[i] - mx);
        denom = group_sum<64>(s);
    }
    if (lane < K) {
        sel[(size_t)m * K + lane] = my_i;
        wts[(size_t)m * K + lane] = ek / denom;
    }
}

int launch_router_f32w(const float *W, const float *bias, const float *g, const uint16_t *x, int M,
                       float *logits, int ld, hipStream_t s) {
    const int E = g_cfg.E, rows = E + (g ? 1 : 0);
    const dim3 grid((rows + 3) / 4, (M + 7) / 8), block(256);
    switch (g_cfg.H) {
    case 2048: hipLaunchKernelGGL(k_router_f32w<8>, grid, block, 0, s, W, bias, g, x, M, E, logits, ld); break;
    case 2560: hipLaunchKernelGGL(k_router_f32w<10>, grid, block, 0, s, W, bias, g, x, M, E, logits, ld); break;
    default: set_error(-2, "router: unsupported hidden %d", g_cfg.H); return -2;
    }
    return check_launch("router_f32w");
}

int launch_router_bf16w(const uint16_t *W, const float *x, float *logits, hipStream_t s) {
    const int E = g_cfg.E;
    const dim3 grid((E + 3) / 4), block(256);
    switch (g_cfg.H) {
    case 2048: hipLaunchKernelGGL(k_router_bf16w<8>, grid, block, 0, s, W, x, E, logits); break;
    case 2560: hipLaunchKernelGGL(k_router_bf16w<10>, grid, block, 0, s, W, x, E, logits); break;
    default: set_error(-2, "router: unsupported hidden %d", g_cfg.H); return -2;
    }
    return check_launch("router_bf16w");
}

int launch_topk(const float *logits, int ld, int M, int *sel, float *wts, hipStream_t s) {
    const int E = g_cfg.E, K = g_cfg.K;
    const dim3 grid((M + 3) / 4), block(256);
    switch (E / 64) {
    case 1: hipLaunchKernelGGL(k_topk<1>, grid, block, 0, s, logits, ld, M, K, g_cfg.renorm, sel, wts); break;
    case 2: hipLaunchKernelGGL(k_topk<2>, grid, block, 0, s, logits, ld, M, K, g_cfg.renorm, sel, wts); break;
    case 4: hipLaunchKernelGGL(k_topk<4>, grid, block, 0, s, logits, ld, M, K, g_cfg.renorm, sel, wts); break;
    case 8: hipLaunchKernelGGL(k_topk<8>, grid, block, 0, s, logits, ld, M, K, g_cfg.renorm, sel, wts); break;
    case 16: hipLaunchKernelGGL(k_topk<16>, grid, block, 0, s, logits, ld, M, K, g_cfg.renorm, sel, wts); break;
    default: set_error(-2, "topk: unsupported expert count %d", E); return -2;
    }
    return check_launch("topk");
}

}  // namespace qfm
