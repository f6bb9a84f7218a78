// qfm_i8_m1.hip -- INT8 routed + shared experts for one row (M = 1 decode).
//
// Reference behaviour: k_i8_gateup_all / k_i8_downacc_all
// (ocho/amd_server/qf8_moe_i8.hip:72-144) and the int8 shared expert
// qf8_i8_shexp_m1 (ocho/amd_server/qf8_dense_i8.hip:346-358). The fused
// forward keeps the activations exact (bf16 x, fp16-chunked hidden) instead of
// the reference's X8 int8 re-quantization; the reference-named gate/up entry
// takes X8 rows as the reference does (qf8_moe_i8.hip:416-421).
//
// gate/up: grid (I/8, K), 256 threads; one 32-lane half-wave per weight
// row. Lane l owns bytes [st*512 + 16l, +16) of the H-byte row for
// st = 0..H/512-1, so a half-wave reads 512 contiguous bytes per step and
// all H/256 weight loads of a row pair (gate + up) are in flight before the
// first multiply. The activation slice a lane needs is the same for every
// row, so it is held in registers (no LDS). In the fused forward x arrives as
// fp16 scaled per row (written by the router launch) and each code is widened
// to fp16 (dot16_i8h: 1024 + (q ^ 0x80), one v_perm per two codes), the
// 1152 * sum(x16) offset removed from the row total; with fp32 or bf16 x, or
// X8 rows (int8 codes with one fp32 scale per 32 values, the reference-named
// entry's input, dequantized in registers), each code is used in offset-binary
// form q + 128 (one v_cvt_f32_ubyte per code) and the accumulator starts at
// -128 * sum(x_slice).
// When the launch carries the
// router logits, every wave runs the top-K selection itself (the 2 KiB row of
// logits is L2-resident), which removes a dependent launch from the decode
// chain; block (0, 0) publishes sel/wts for the down kernel. With a shared
// expert the last grid row computes its gate/up rows (job K, hidden row K):
// those blocks need no selection, so their weight stream runs while the
// routed blocks are still selecting.
//
// down: one LPR-lane group per output row (LPR = 32 for I = 512, 8 for
// I = 640). The hidden vectors are loaded first, then every weight load of
// the row is issued (the 16-byte chunks of all K + 1 expert rows), and while
// those are in flight the hidden vectors are staged in LDS as fp16 chunks
// scaled by powers of two (chunk16_to_f16; the codes are widened to fp16,
// dot16_i8h). Each lane accumulates sum_j w_j * sd_j[c] * <Wd_j slice, h_j slice> across all
// jobs and the group reduces once, so every output row has one writer and a
// fixed summation order (deterministic; y is seeded, not accumulated).
#include "qfm_dev.h"
#include "qfm_internal.h"

namespace qfm {

// (H = 2048: three waves per SIMD, so the 11 x 64 blocks of a decode step are all resident at once)
template <int H, int I, int EPL, bool X16>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(H == 2048 ? 3 : 1)))
k_i8_gateup_m1(const int8_t *__restrict__ Qg, const int8_t *__restrict__ Qu,
               const float *__restrict__ Sg, const float *__restrict__ Su,
               const uint16_t *__restrict__ xb, const float *__restrict__ xf,
               const float *__restrict__ logits, int *__restrict__ sel, float *__restrict__ wts,
               int K, int renorm, float *__restrict__ hidden, ShPtrs sh,
               const uint4 *__restrict__ x16, const float2 *__restrict__ x16i,
               const int8_t *__restrict__ x8q, const float *__restrict__ x8s) {
    constexpr int NST = H / 512;
    __shared__ __align__(16) unsigned long long s_tk[4][kTopkLds];
    const int job = blockIdx.y;
    const bool shared_job = sh.qg != nullptr && job == (int)gridDim.y - 1;
    const int l = threadIdx.x & 31;
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    float xs[X16 ? 1 : NST][16];
    if constexpr (!X16) {
        if (x8q) {
            // X8 rows: values [512 st + 16 l, +16) are codes of one 32-value block
#pragma unroll
            for (int st = 0; st < NST; st++) {
                const int k0 = st * 512 + l * 16;
                const uint4 q = *reinterpret_cast<const uint4 *>(x8q + k0);
                const float sc = x8s[k0 >> 5];
                // offset-binary widening (u - 128, exact), not a sign-extend + convert pair
                const uint32_t d[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
#pragma unroll
                for (int i = 0; i < 16; i++) xs[st][i] = ((float)((d[i >> 2] >> (8 * (i & 3))) & 0xFFu) - 128.0f) * sc;
            }
        } else if (xb) {
            load_x_slice_bf16<H>(xb, l, xs);
        } else {
            load_x_slice_f32<H>(xf, l, xs);
        }
    }
    int e = 0;
    if (shared_job) {
        Qg = sh.qg; Qu = sh.qu; Sg = sh.sg; Su = sh.su;     // expert 0 of a one-expert arena
    } else if (logits) {
        // every wave selects its block's expert itself (no barrier): the rank-`job`
        // id only; wave 0 of block (0, 0) also writes the routing (ids + weights)
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        if (blockIdx.x == 0 && job == 0 && wave == 0) {
            int my_i;
            float my_w;
            wave_topk<EPL>(logits, K, renorm, lane, s_tk[0], my_i, my_w);
            if (lane < K) {
                sel[lane] = my_i;
                wts[lane] = my_w;
            }
            e = __builtin_amdgcn_readfirstlane(my_i);
        } else {
            e = wave_topk_one<EPL>(logits, K, job, lane, s_tk[wave]);
        }
    } else {
        e = sel[job];
    }
    uint4 xh[X16 ? NST : 1][2];
    float2 xinf = make_float2(0.0f, 1.0f);
    if constexpr (X16) {
        // the x slice as fp16 (scaled per row), loaded after the selection (fewer
        // registers live through it) and before the weights (waiting for it never
        // waits for them): values [512 st + 16 l, +16) are words 64 st + 2 l, +1
#pragma unroll
        for (int st = 0; st < NST; st++) {
            xh[st][0] = x16[st * 64 + 2 * l];
            xh[st][1] = x16[st * 64 + 2 * l + 1];
        }
        xinf = *x16i;
    }
    const int8_t *qg = Qg + (size_t)e * ((size_t)I * H) + (size_t)row * H + l * 16;
    const int8_t *qu = Qu + (size_t)e * ((size_t)I * H) + (size_t)row * H + l * 16;
    uint4 wg[NST], wu[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        wg[st] = ld_nt16(qg + st * 512);
        wu[st] = ld_nt16(qu + st * 512);
    }
    const float sg = Sg[(size_t)e * I + row], su = Su[(size_t)e * I + row];
    float ag, au;
    if constexpr (X16) {
        // fp16-widened codes (dot16_i8h); the 1152 * sum(x16) offset is removed
        // once from the row total
        ag = 0.0f; au = 0.0f;
#pragma unroll
        for (int st = 0; st < NST; st++) {
            ag = dot16_i8h(wg[st], xh[st][0], xh[st][1], ag);
            au = dot16_i8h(wu[st], xh[st][0], xh[st][1], au);
        }
        ag = group_sum<32>(ag);
        au = group_sum<32>(au);
        ag = (ag - kI8hOffset * xinf.x) * xinf.y;
        au = (au - kI8hOffset * xinf.x) * xinf.y;
    } else {
        float xsum = 0.0f;
#pragma unroll
        for (int st = 0; st < NST; st++)
#pragma unroll
            for (int i = 0; i < 16; i++) xsum += xs[st][i];
        ag = -128.0f * xsum; au = ag;
#pragma unroll
        for (int st = 0; st < NST; st++) {
            ag = dot16_u8(wg[st], xs[st], ag);
            au = dot16_u8(wu[st], xs[st], au);
        }
        ag = group_sum<32>(ag);
        au = group_sum<32>(au);
    }
    if (l == 0) hidden[(size_t)job * I + row] = silu(ag * sg) * (au * su);
}

constexpr int kMaxJobs = 17;   // top_k <= 16 plus the shared expert

// NJ jobs (routed experts, then the shared one when HAS_SH) are a template
// parameter so that every register array is indexed at compile time: no
// branches around loads and no scratch, which keeps all loads of a batch in
// flight together (memory-counter waits retire in issue order).
template <int H, int I, int LPR, int NJ, bool HAS_SH, int CH>
__global__ void __launch_bounds__(256)
k_i8_down_m1(const int8_t *__restrict__ Qd, const float *__restrict__ Sd,
             const float *__restrict__ hidden, const float *__restrict__ wts,
             const int *__restrict__ sel, ShPtrs sh,
             const float *__restrict__ gdot, float *__restrict__ y32, uint16_t *__restrict__ ybf) {
    constexpr int NST = I / (16 * LPR);
    constexpr int RPB = 256 / LPR;
    constexpr int NEXP = HAS_SH ? NJ - 1 : NJ;
    constexpr int NCH = NJ * I / 16;                  // 16-value hidden chunks
    constexpr int CPT = (NCH + 255) / 256;            // chunks per thread
    __shared__ uint4 s_h16[NCH * 2];                  // the hidden rows as scaled fp16 (chunk16_to_f16)
    __shared__ float2 s_hci[NCH];
    const int l = threadIdx.x % LPR;
    const int c = blockIdx.x * RPB + threadIdx.x / LPR;
    // batch 1: routing, router weights, shared gate, this thread's hidden chunks (to registers)
    float hv[CPT][16];
#pragma unroll
    for (int q = 0; q < CPT; q++) {
        const int ch = min((int)threadIdx.x + q * 256, NCH - 1);   // shared hidden follows the routed ones
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float4 f = reinterpret_cast<const float4 *>(hidden)[ch * 4 + v];
            hv[q][4 * v] = f.x; hv[q][4 * v + 1] = f.y; hv[q][4 * v + 2] = f.z; hv[q][4 * v + 3] = f.w;
        }
    }
    int ex[NEXP > 0 ? NEXP : 1];
    float wt[NEXP > 0 ? NEXP : 1];
#pragma unroll
    for (int j = 0; j < NEXP; j++) { ex[j] = sel[j]; wt[j] = wts[j]; }
    float sh_sd = 0.0f, gd = 0.0f;
    if constexpr (HAS_SH) {
        sh_sd = sh.sd[c];
        if (gdot) gd = gdot[0];
    }
    // batch 2: weight chunks and row scales
    float wsc[NJ];
#pragma unroll
    for (int j = 0; j < NEXP; j++) wsc[j] = wt[j] * Sd[(size_t)ex[j] * H + c];
    uint4 w[CH][NST];
#pragma unroll
    for (int u = 0; u < CH && u < NJ; u++) {
        const int8_t *p = (u < NEXP ? Qd + (size_t)ex[u] * ((size_t)H * I) : sh.qd) + (size_t)c * I;
#pragma unroll
        for (int st = 0; st < NST; st++) w[u][st] = ld_nt16(p + (st * LPR + l) * 16);
    }
#pragma unroll
    for (int q = 0; q < CPT; q++) {
        const int ch = (int)threadIdx.x + q * 256;
        if (ch < NCH) {
            uint4 ha, hb;
            s_hci[ch] = chunk16_to_f16(hv[q], ha, hb);
            s_h16[2 * ch] = ha;
            s_h16[2 * ch + 1] = hb;
        }
    }
    __syncthreads();
    if constexpr (HAS_SH) wsc[NJ - 1] = (gdot ? sigmoid(gd) : 1.0f) * sh_sd;
    float acc = 0.0f;
#pragma unroll
    for (int j0 = 0; j0 < NJ; j0 += CH) {
        if (j0 > 0) {
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int j = j0 + u;
                if (j < NJ) {
                    const int8_t *p = (j < NEXP ? Qd + (size_t)ex[j < NEXP ? j : 0] * ((size_t)H * I) : sh.qd) + (size_t)c * I;
#pragma unroll
                    for (int st = 0; st < NST; st++) w[u][st] = ld_nt16(p + (st * LPR + l) * 16);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const int j = j0 + u;
            if (j < NJ) {
                float d = 0.0f;
#pragma unroll
                for (int st = 0; st < NST; st++) {
                    const int ch = j * (I / 16) + st * LPR + l;
                    const float2 ci = s_hci[ch];
                    d = fmaf(dot16_i8h(w[u][st], s_h16[2 * ch], s_h16[2 * ch + 1], ci.x), ci.y, d);
                }
                acc = fmaf(wsc[j], d, acc);
            }
        }
    }
    acc = group_sum<LPR>(acc);
    if (l == 0) {
        if (y32) y32[c] = acc;
        if (ybf) ybf[c] = f32_to_bf16(acc);
    }
}

template <int H, int I, int LPR, int NJ, bool HAS_SH, int CH>
static void down_launch(const Qf4ExpCache *c, const float *hidden, const float *wts, const int *sel, ShPtrs sp,
                        const float *gdot, float *y32, uint16_t *ybf, hipStream_t s) {
    hipLaunchKernelGGL((k_i8_down_m1<H, I, LPR, NJ, HAS_SH, CH>), dim3(H / (256 / LPR)), dim3(256), 0, s,
                       c->i8_down, c->i8s_down, hidden, wts, sel, sp, gdot, y32, ybf);
}

template <int H, int I, int LPR, int CH, int NJ>
static bool down_dispatch_nj(int nj, bool has_sh, const Qf4ExpCache *c, const float *hidden, const float *wts,
                             const int *sel, ShPtrs sp, const float *gdot, float *y32,
                             uint16_t *ybf, hipStream_t s) {
    if constexpr (NJ > kMaxJobs) {
        return false;
    } else {
        if (nj == NJ) {
            if (has_sh) down_launch<H, I, LPR, NJ, true, (CH < NJ ? CH : NJ)>(c, hidden, wts, sel, sp, gdot, y32, ybf, s);
            else down_launch<H, I, LPR, NJ, false, (CH < NJ ? CH : NJ)>(c, hidden, wts, sel, sp, gdot, y32, ybf, s);
            return true;
        }
        return down_dispatch_nj<H, I, LPR, CH, NJ + 1>(nj, has_sh, c, hidden, wts, sel, sp, gdot, y32, ybf, s);
    }
}

int launch_i8_gateup_m1(const Qf4ExpCache *c, const uint16_t *xb, const float *xf, const float *logits, int *sel,
                        float *wts, int nexp, float *hidden, hipStream_t s, const ShPtrs *sh, const void *x16,
                        const int8_t *x8q, const float *x8s) {
    if (!c || !c->i8_gate || !c->i8_up || !c->i8s_gate || !c->i8s_up) {
        set_error(-1, "i8_gateup_m1: arena has no INT8 gate/up"); return -1;
    }
    if (c->slots < g_cfg.E) {   // expert ids address slots directly
        set_error(-1, "i8_gateup_m1: the INT8 arena holds %d slots, not all %d experts", c->slots, g_cfg.E); return -1;
    }
    if (nexp < 1 || nexp > 16 || (!xb && !xf && !x16 && !(x8q && x8s)) || !hidden || !sel || (logits && !wts)) {
        set_error(-1, "i8_gateup_m1: bad arguments"); return -1;
    }
    if (logits && (nexp != g_cfg.K || g_cfg.E != 512)) {
        set_error(-2, "i8_gateup_m1: in-kernel selection needs nexp == top_k and 512 experts"); return -2;
    }
    const dim3 block(256);
    const int K = g_cfg.K, rn = g_cfg.renorm;
    ShPtrs sp{};
    if (sh) sp = *sh;
    const unsigned jobs = (unsigned)nexp + (sh ? 1u : 0u);   // shared expert: last grid row, hidden row nexp
    const uint4 *xh = static_cast<const uint4 *>(x16);
    const float2 *xi = xh ? reinterpret_cast<const float2 *>(xh + g_cfg.H / 8) : nullptr;
#define QFM_GU_M1(HH, II, X16)                                                                                  \
    hipLaunchKernelGGL((k_i8_gateup_m1<HH, II, 8, X16>), dim3(II / 8, jobs), block, 0, s, c->i8_gate, c->i8_up, \
                       c->i8s_gate, c->i8s_up, xb, xf, logits, sel, wts, K, rn, hidden, sp, xh, xi, x8q, x8s)
    if (shape_2048()) {
        if (xh) QFM_GU_M1(2048, 512, true); else QFM_GU_M1(2048, 512, false);
    } else if (shape_2560()) {
        if (xh) QFM_GU_M1(2560, 640, true); else QFM_GU_M1(2560, 640, false);
    } else if (shape_shard()) {
        if (xh) QFM_GU_M1(2048, 64, true); else QFM_GU_M1(2048, 64, false);
    } else {
        set_error(-2, "i8_gateup_m1: unsupported shape"); return -2;
    }
#undef QFM_GU_M1
    return check_launch("i8_gateup_m1");
}

int launch_i8_down_m1(const Qf4ExpCache *c, const float *hidden, const float *wts, const int *sel, int nexp,
                      const ShPtrs *sh, const float *gdot, float *y32, uint16_t *ybf, hipStream_t s) {
    if (!c || !c->i8_down || !c->i8s_down) { set_error(-1, "i8_down_m1: arena has no INT8 down"); return -1; }
    if (c->slots < g_cfg.E) {   // expert ids address slots directly
        set_error(-1, "i8_down_m1: the INT8 arena holds %d slots, not all %d experts", c->slots, g_cfg.E); return -1;
    }
    if (nexp < 0 || nexp > 16 || (!y32 && !ybf) || !hidden || (nexp && (!sel || !wts))) {
        set_error(-1, "i8_down_m1: bad arguments"); return -1;
    }
    ShPtrs sp{};
    if (sh) sp = *sh;
    const int nj = nexp + (sh ? 1 : 0);
    if (nj == 0) { set_error(-1, "i8_down_m1: nothing to do"); return -1; }
    bool ok;
    if (shape_2048()) {
        ok = down_dispatch_nj<2048, 512, 32, kMaxJobs, 1>(nj, sh != nullptr, c, hidden, wts, sel, sp, gdot, y32, ybf, s);
    } else if (shape_2560()) {
        ok = down_dispatch_nj<2560, 640, 8, 3, 1>(nj, sh != nullptr, c, hidden, wts, sel, sp, gdot, y32, ybf, s);
    } else if (shape_shard()) {   // 64-byte down rows: 4 lanes each
        ok = down_dispatch_nj<2048, 64, 4, kMaxJobs, 1>(nj, sh != nullptr, c, hidden, wts, sel, sp, gdot, y32, ybf, s);
    } else {
        set_error(-2, "i8_down_m1: unsupported shape"); return -2;
    }
    if (!ok) { set_error(-2, "i8_down_m1: unsupported job count %d", nj); return -2; }
    return check_launch("i8_down_m1");
}

}  // namespace qfm
