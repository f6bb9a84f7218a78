// qfm_router.hip -- router GEMV and softmax/top-k selection.
//
// Reference behaviour: qf_rtr_gemv (ocho/amd_server/qf_router_wave64.hip:42-51),
// qf_rtr_topk10 (:69-155), Spark k_router_topk (ocho/engine_spark/cuda/qf.cu:1184-1271).
//
// Router logits are produced in one canonical fp32 order so that the host
// restatement reproduces them bit for bit: lane l of a wave owns elements
// k = j*256 + 4l + c (j = 0..H/256-1, c = 0..3) of the row and accumulates
// them with a sequential fmaf chain in (j, c) order; the 64 lane partials
// are then combined by an xor butterfly p[l] = p[l] + p[l ^ m], m = 1..32
// (canon_butterfly: DPP for the first four steps).
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
    return canon_butterfly(a);
}

// One wave per block. Blocks [0, E): router rows of W fp32 [E][H]; block E
// (when g != nullptr): the shared-expert gate vector g [H], written to
// column E without bias; the remaining I/2 blocks (when sh.qg != nullptr):
// two shared-expert gate/up rows each, one per half-wave, giving
// hsh[m][r] = silu(sg_r <Qg_r, x_m>) * (su_r <Qu_r, x_m>). x is bf16 [M][H],
// logits [M][ld]. Every output depends on x only, so one launch covers all.
// MR rows of x are processed together: their fma chains are independent and
// their canonical reductions share cross-lane steps (canon_reduce_rows; each
// row keeps the canonical order). With
// MR > 1 the shared-expert rows are also split over x rows: block (pair, mg)
// computes rows [2 mg, 2 mg + 2) of x for its row pair, MG = ceil(M / 2) blocks
// per pair, laid out so that one pair's blocks share an XCD (and its L2).
// With x16 != nullptr one more block (the first) writes x row 0 as scaled
// fp16 with its (sum, 2^-k) for the M = 1 gate/up kernel.
//
// With TAIL (the M <= 8 forward; tail.lw != nullptr) the launch also selects: each
// router row's logits go out a second time as 64-bit words (fp32 bits | tag <<
// 32, stored at agent scope), tag = next_tag(ctl[m]) for row m; the grid's last
// blocks are then (INT8) x as scaled fp16 chunks (chunk16_to_f16, the fork
// rows' dot16_i8h input) and one selector wave per row, which reads its row's
// words until every tag is that tag (bounded: a timeout is counted in
// ctl[kTailRows] and the words are used as found), ranks them from registers
// (wave_topk_regs: the same selection as wave_topk), writes sel/wts and then
// ctl[m] = the tag. Every router wave has read ctl before it writes a word, so
// no wave of this launch reads the updated ctl[m]; the next call tags with
// the tag after it, so words left by this call are never taken for the next
// call's. A selector waits only on router waves dispatched before it, which
// never wait, so the waits end.
template <int NJ, int I, int MR, bool TAIL>
__global__ void __launch_bounds__(64)
k_router_shared(const float *__restrict__ W, const float *__restrict__ bias, const float *__restrict__ g,
                ShPtrs sh, const uint16_t *__restrict__ x, int M, int E, float *__restrict__ logits, int ld,
                float *__restrict__ hsh, int ldh, uint4 *__restrict__ x16, float2 *__restrict__ x16i,
                RouteTail tail, int tail0) {
    constexpr int H = NJ * 256;
    const int lane = threadIdx.x;
    args_now(W, bias, g, sh.qg, sh.qu, sh.sg, sh.su, x, M, E, logits, ld, hsh, ldh, x16, x16i);
    if (x16 && blockIdx.x == 0) {                   // the first block: x row 0 as scaled fp16
        wave_row_to_f16<H>(x, x16, x16i, lane);
        return;
    }
    const int b = (int)blockIdx.x - (x16 ? 1 : 0);
    const int ng = g ? 1 : 0;
    if (TAIL && b >= tail0) {                       // the selection tail (block-uniform)
        const int nxb = tail.xh ? (M * (H / 16) + 63) / 64 : 0;
        if (b < tail0 + nxb) {                      // x as scaled fp16 chunks
            const int ch = (b - tail0) * 64 + lane;
            if (ch < M * (H / 16)) {
                const uint4 a = reinterpret_cast<const uint4 *>(x)[2 * ch], c = reinterpret_cast<const uint4 *>(x)[2 * ch + 1];
                const uint32_t d[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
                float v[16];
#pragma unroll
                for (int i = 0; i < 8; i++) { v[2 * i] = bf16_lo(d[i]); v[2 * i + 1] = bf16_hi(d[i]); }
                uint4 ha, hb;
                tail.xci[ch] = chunk16_to_f16(v, ha, hb);
                tail.xh[2 * ch] = ha;
                tail.xh[2 * ch + 1] = hb;
            }
            return;
        }
        const int m = b - tail0 - nxb;              // selector of row m
        constexpr int EPL = 8;                      // E == 512 (checked by the host)
        __shared__ __align__(16) unsigned long long s_tk[kTopkLds];
        const uint32_t tg = next_tag(tail.ctl[m]);
        const unsigned long long *row = tail.lw + (size_t)m * E;
        float v[EPL];
        uint32_t pend = 0u;
        {
            unsigned long long w[EPL];
#pragma unroll
            for (int i = 0; i < EPL; i++) w[i] = ld_agent_u64(row + i * 64 + lane);
#pragma unroll
            for (int i = 0; i < EPL; i++) {
                v[i] = __uint_as_float((uint32_t)w[i]);
                if ((uint32_t)(w[i] >> 32) != tg) pend |= 1u << i;
            }
        }
        for (int it = 0; __builtin_amdgcn_ballot_w64(pend != 0u) != 0; it++) {
            if (it == kTailSpinMax) {               // bounded: count it, rank what is there
                if (lane == 0) __hip_atomic_fetch_add(tail.ctl + kTailRows, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            unsigned long long w[EPL];
#pragma unroll
            for (int i = 0; i < EPL; i++) w[i] = ld_agent_u64(row + i * 64 + lane);
#pragma unroll
            for (int i = 0; i < EPL; i++)
                if ((pend & (1u << i)) && (uint32_t)(w[i] >> 32) == tg) {
                    v[i] = __uint_as_float((uint32_t)w[i]);
                    pend &= ~(1u << i);
                }
        }
        int my_i;
        float my_w;
        wave_topk_regs<EPL>(v, tail.K, tail.renorm, lane, s_tk, my_i, my_w);
        if (lane < tail.K) {
            tail.sel[m * tail.K + lane] = my_i;
            tail.wts[m * tail.K + lane] = my_w;
        }
        if (lane == 0) tail.ctl[m] = tg;
        return;
    }
    if (b < E + ng) {
        const bool is_g = b == E;
        const float *wr = is_g ? g : W + (size_t)b * H;
        float4 w[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) w[j] = *reinterpret_cast<const float4 *>(wr + j * 256 + lane * 4);
        const float bb = (!is_g && bias) ? bias[b] : 0.0f;
        for (int m0 = 0; m0 < M; m0 += MR) {
            // the tag of the row this lane ends with (lane r < MR: row m0 + r),
            // requested with the pass's x rows
            const uint32_t tgl = (TAIL && lane < MR && m0 + lane < M) ? next_tag(tail.ctl[m0 + lane]) : 0u;
            uint2 xp[MR][NJ];
#pragma unroll
            for (int r = 0; r < MR; r++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    xp[r][j] = m0 + r < M ? *reinterpret_cast<const uint2 *>(x + (size_t)(m0 + r) * H + j * 256 + lane * 4)
                                          : make_uint2(0u, 0u);
            float a[MR];
#pragma unroll
            for (int r = 0; r < MR; r++) {
                a[r] = 0.0f;
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    a[r] = __fmaf_rn(w[j].x, bf16_lo(xp[r][j].x), a[r]);
                    a[r] = __fmaf_rn(w[j].y, bf16_hi(xp[r][j].x), a[r]);
                    a[r] = __fmaf_rn(w[j].z, bf16_lo(xp[r][j].y), a[r]);
                    a[r] = __fmaf_rn(w[j].w, bf16_hi(xp[r][j].y), a[r]);
                }
            }
            if constexpr (MR == 1) {
                float v = canon_butterfly(a[0]);
                if (bias && !is_g) v = __fadd_rn(v, bb);
                if (lane == 0 && m0 < M) {
                    logits[(size_t)m0 * ld + b] = v;
                    if (TAIL && !is_g) st_agent_u64(tail.lw + (size_t)m0 * E + b, __float_as_uint(v) | ((unsigned long long)tgl << 32));
                }
            } else {
                // lane r < MR ends with row m0 + r (the same addition tree per row)
                float v = canon_reduce_rows<MR>(a, lane);
                if (bias && !is_g) v = __fadd_rn(v, bb);
                if (lane < MR && m0 + lane < M) {
                    logits[(size_t)(m0 + lane) * ld + b] = v;
                    if (TAIL && !is_g)
                        st_agent_u64(tail.lw + (size_t)(m0 + lane) * E + b, __float_as_uint(v) | ((unsigned long long)tgl << 32));
                }
            }
        }
        return;
    }
    // shared-expert gate/up rows
    constexpr int NST = H / 512;
    const int l = lane & 31;
    const int sb = b - E - ng;
    int pair = sb, mlo = 0, mhi = M;
    if (MR > 1) {
        const int MG = (M + 1) / 2, t = sb >> 3, mg = t % MG;
        pair = (t / MG) * 8 + (sb & 7);
        mlo = mg * 2;
        mhi = min(M, mlo + 2);
    }
    const int r = pair * 2 + (lane >> 5);
    uint4 wg[NST], wu[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        wg[st] = ld_nt16(sh.qg + (size_t)r * H + st * 512 + l * 16);
        wu[st] = ld_nt16(sh.qu + (size_t)r * H + st * 512 + l * 16);
    }
    const float sg = sh.sg[r], su = sh.su[r];
    constexpr int SR = MR > 1 ? 2 : 1;          // x rows per pass of the shared rows
    for (int m0 = mlo; m0 < mhi; m0 += SR) {
        float ag[SR], au[SR];
#pragma unroll
        for (int q = 0; q < SR; q++) {
            ag[q] = 0.0f; au[q] = 0.0f;
            if (m0 + q < mhi) {
                float xs[NST][16];
                load_x_slice_bf16<H>(x + (size_t)(m0 + q) * H, l, xs);
                float xsum = 0.0f;
#pragma unroll
                for (int st = 0; st < NST; st++)
#pragma unroll
                    for (int i = 0; i < 16; i++) xsum += xs[st][i];
                ag[q] = -128.0f * xsum; au[q] = ag[q];
#pragma unroll
                for (int st = 0; st < NST; st++) {
                    ag[q] = dot16_u8(wg[st], xs[st], ag[q]);
                    au[q] = dot16_u8(wu[st], xs[st], au[q]);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < SR; q++) { ag[q] = group_sum<32>(ag[q]); au[q] = group_sum<32>(au[q]); }
#pragma unroll
        for (int q = 0; q < SR; q++)
            if (l == 0 && m0 + q < mhi) hsh[(size_t)(m0 + q) * ldh + r] = silu(ag[q] * sg) * (au[q] * su);
    }
}

// Reference form: W bf16 [E][H], x fp32 [H] (qf_rtr_gemv signature).
template <int NJ>
__global__ void __launch_bounds__(64)
k_router_bf16w(const uint16_t *__restrict__ W, const float *__restrict__ x, int E, float *__restrict__ logits) {
    constexpr int H = NJ * 256;
    const int lane = threadIdx.x;
    const int e = blockIdx.x;
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

// One wave per row; see wave_topk.
template <int EPL>
__global__ void __launch_bounds__(256)
k_topk(const float *__restrict__ logits, int ld, int M, int K, int renorm,
       int *__restrict__ sel, float *__restrict__ wts) {
    __shared__ __align__(16) unsigned long long s_tk[4][kTopkLds];
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    int my_i;
    float my_w;
    wave_topk<EPL>(logits + (size_t)m * ld, K, renorm, lane, s_tk[threadIdx.x >> 6], my_i, my_w);
    if (lane < K) {
        sel[(size_t)m * K + lane] = my_i;
        wts[(size_t)m * K + lane] = my_w;
    }
}

int launch_router_shared(const float *W, const float *bias, const float *g, const ShPtrs *sh,
                         const uint16_t *x, int M, float *logits, int ld, float *hsh, int ldh, hipStream_t s,
                         void *x16, const RouteTail *tail) {
    const int E = g_cfg.E, I = g_cfg.I;
    if (sh && !hsh) { set_error(-1, "router: shared rows need an output"); return -1; }
    if (x16 && M != 1) { set_error(-1, "router: the fp16 x row is for M = 1"); return -1; }
    if (tail && (x16 || E != 512 || M > kTailRows || !tail->lw || !tail->ctl || !tail->sel || !tail->wts ||
                 tail->K < 1 || tail->K > 16 || (!tail->xh) != (!tail->xci))) {
        set_error(-1, "router: bad selection tail"); return -1;
    }
    ShPtrs sp{};
    if (sh) sp = *sh;
    uint4 *xh = static_cast<uint4 *>(x16);
    float2 *xi = xh ? reinterpret_cast<float2 *>(xh + g_cfg.H / 8) : nullptr;
    int nblk = E + (g ? 1 : 0) + (sh ? (I / 2) * (M == 1 ? 1 : (M + 1) / 2) : 0) + (xh ? 1 : 0);
    RouteTail tl{};
    const int tail0 = nblk - (xh ? 1 : 0);           // first tail block (counted without the fp16-row block)
    if (tail) {
        tl = *tail;
        nblk += (tl.xh ? (M * (g_cfg.H / 16) + 63) / 64 : 0) + M;
    }
#define QFM_ROUTER(NJ, II, MR)                                                                                 \
    if (tail)                                                                                                  \
        hipLaunchKernelGGL((k_router_shared<NJ, II, MR, true>), dim3(nblk), dim3(64), 0, s, W, bias, g, sp, x, M, E, \
                           logits, ld, hsh, ldh, xh, xi, tl, tail0);                                          \
    else                                                                                                       \
        hipLaunchKernelGGL((k_router_shared<NJ, II, MR, false>), dim3(nblk), dim3(64), 0, s, W, bias, g, sp, x, M, E, \
                           logits, ld, hsh, ldh, xh, xi, tl, tail0)
    if (shape_2048()) {
        if (M == 1) { QFM_ROUTER(8, 512, 1); }
        else if (M <= 4) { QFM_ROUTER(8, 512, 4); }
        else { QFM_ROUTER(8, 512, 8); }
    } else if (shape_shard() && M == 1 && !sh && !tail) {
        hipLaunchKernelGGL((k_router_shared<8, 64, 1, false>), dim3(nblk), dim3(64), 0, s, W, bias, g, sp, x, M, E,
                           logits, ld, hsh, ldh, xh, xi, tl, tail0);
    } else if (shape_2560()) {
        if (M == 1) { QFM_ROUTER(10, 640, 1); }
        else { QFM_ROUTER(10, 640, 4); }
    } else {
        set_error(-2, "router: unsupported shape"); return -2;
    }
#undef QFM_ROUTER
    return check_launch("router_shared");
}

int launch_router_bf16w(const uint16_t *W, const float *x, float *logits, hipStream_t s) {
    const int E = g_cfg.E;
    const dim3 grid(E), block(64);
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
