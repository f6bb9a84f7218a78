// qfm_i8_m1.hip -- INT8 routed + shared experts for one row (M = 1 decode).
//
// Reference behaviour: k_i8_gateup_all / k_i8_downacc_all
// (ocho/amd_server/qf8_moe_i8.hip:72-144) and the int8 shared expert
// qf8_i8_shexp_m1 (ocho/amd_server/qf8_dense_i8.hip:346-358), with the
// activations kept exact (bf16/fp32) instead of the reference's X8 int8
// re-quantization.
//
// gate/up: grid (I/8, jobs), 256 threads; one 32-lane half-wave per weight
// row. Lane l owns bytes [st*512 + 16l, +16) of the H-byte row for
// st = 0..H/512-1, so a half-wave reads 512 contiguous bytes per step and
// all H/256 weight loads of a row pair (gate + up) are in flight before the
// first multiply. The activation slice a lane needs is the same for every
// row, so it is held in registers as fp32 (no LDS). Each code q is used in
// offset-binary form q + 128 (one v_cvt_f32_ubyte per code) and the
// accumulator starts at -128 * sum(x_slice).
//
// down: one LPR-lane group per output row (LPR = 32 for I = 512, 8 for
// I = 640); the jobs' hidden vectors are staged once per block in LDS. Each
// lane accumulates sum_j w_j * sd_j[c] * <Wd_j slice, h_j slice> across all
// jobs and the group reduces once, so every output row has one writer and
// a fixed summation order (deterministic; y is seeded, not accumulated).
#include "qfm_dev.h"
#include "qfm_internal.h"

namespace qfm {

struct JobPtrs {
    const int8_t *qg, *qu, *qd;
    const float *sg, *su, *sd;
};

template <int H>
__device__ __forceinline__ void load_x_slice(const uint16_t *xb, const float *xf, int l, float (&xs)[H / 512][16]) {
#pragma unroll
    for (int st = 0; st < H / 512; st++) {
        const int k0 = st * 512 + l * 16;
        if (xb) {
            const uint4 a = *reinterpret_cast<const uint4 *>(xb + k0);
            const uint4 b = *reinterpret_cast<const uint4 *>(xb + k0 + 8);
            const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int q = 0; q < 8; q++) { xs[st][2 * q] = bf16_lo(d[q]); xs[st][2 * q + 1] = bf16_hi(d[q]); }
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 f = *reinterpret_cast<const float4 *>(xf + k0 + 4 * q);
                xs[st][4 * q] = f.x; xs[st][4 * q + 1] = f.y; xs[st][4 * q + 2] = f.z; xs[st][4 * q + 3] = f.w;
            }
        }
    }
}

template <int H, int I>
__global__ void __launch_bounds__(256)
k_i8_gateup_m1(const int8_t *__restrict__ Qg, const int8_t *__restrict__ Qu,
               const float *__restrict__ Sg, const float *__restrict__ Su,
               const uint16_t *__restrict__ xb, const float *__restrict__ xf,
               const int *__restrict__ sel, int nexp, JobPtrs sh, float *__restrict__ hidden) {
    constexpr int NST = H / 512;
    const int job = blockIdx.y;
    const int l = threadIdx.x & 31;
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int8_t *qg, *qu;
    const float *sg, *su;
    if (job < nexp) {
        const size_t e = (size_t)sel[job];
        qg = Qg + e * ((size_t)I * H); qu = Qu + e * ((size_t)I * H);
        sg = Sg + e * I; su = Su + e * I;
    } else {
        qg = sh.qg; qu = sh.qu; sg = sh.sg; su = sh.su;
    }
    uint4 wg[NST], wu[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        wg[st] = ld_nt16(qg + (size_t)row * H + st * 512 + l * 16);
        wu[st] = ld_nt16(qu + (size_t)row * H + st * 512 + l * 16);
    }
    float xs[NST][16];
    load_x_slice<H>(xb, xf, l, xs);
    float xsum = 0.0f;
#pragma unroll
    for (int st = 0; st < NST; st++)
#pragma unroll
        for (int i = 0; i < 16; i++) xsum += xs[st][i];
    float ag = -128.0f * xsum, au = ag;
#pragma unroll
    for (int st = 0; st < NST; st++) {
        ag = dot16_u8(wg[st], xs[st], ag);
        au = dot16_u8(wu[st], xs[st], au);
    }
    ag = group_sum<32>(ag);
    au = group_sum<32>(au);
    if (l == 0) {
        const float gv = ag * sg[row], uv = au * su[row];
        hidden[(size_t)job * I + row] = silu(gv) * uv;
    }
}

constexpr int kMaxJobs = 17;   // top_k <= 16 plus the shared expert

template <int H, int I, int LPR>
__global__ void __launch_bounds__(256)
k_i8_down_m1(const int8_t *__restrict__ Qd, const float *__restrict__ Sd,
             const float *__restrict__ hidden, const float *__restrict__ wts,
             const int *__restrict__ sel, int nexp, JobPtrs sh, const float *__restrict__ gdot,
             float *__restrict__ y32, uint16_t *__restrict__ ybf) {
    constexpr int NST = I / (16 * LPR);
    constexpr int RPB = 256 / LPR;
    __shared__ __align__(16) float sh_h[kMaxJobs * I];
    __shared__ const int8_t *sh_q[kMaxJobs];
    __shared__ const float *sh_s[kMaxJobs];
    __shared__ float sh_w[kMaxJobs];
    const int njobs = nexp + (sh.qd ? 1 : 0);
    for (int i = threadIdx.x; i < njobs * I / 4; i += 256)
        reinterpret_cast<float4 *>(sh_h)[i] = reinterpret_cast<const float4 *>(hidden)[i];
    if (threadIdx.x < njobs) {
        const int j = threadIdx.x;
        if (j < nexp) {
            const size_t e = (size_t)sel[j];
            sh_q[j] = Qd + e * ((size_t)H * I);
            sh_s[j] = Sd + e * H;
            sh_w[j] = wts[j];
        } else {
            sh_q[j] = sh.qd;
            sh_s[j] = sh.sd;
            sh_w[j] = gdot ? sigmoid(gdot[0]) : 1.0f;
        }
    }
    __syncthreads();
    const int l = threadIdx.x % LPR;
    const int c = blockIdx.x * RPB + threadIdx.x / LPR;
    float acc = 0.0f;
    int j = 0;
    for (; j + 4 <= njobs; j += 4) {
        uint4 w[4][NST];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int st = 0; st < NST; st++)
                w[u][st] = ld_nt16(sh_q[j + u] + (size_t)c * I + (st * LPR + l) * 16);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            float d = 0.0f;
#pragma unroll
            for (int st = 0; st < NST; st++)
                d = dot16_i8(w[u][st], sh_h + (j + u) * I + (st * LPR + l) * 16, d);
            acc = fmaf(sh_w[j + u] * sh_s[j + u][c], d, acc);
        }
    }
    for (; j < njobs; j++) {
        uint4 w[NST];
#pragma unroll
        for (int st = 0; st < NST; st++) w[st] = ld_nt16(sh_q[j] + (size_t)c * I + (st * LPR + l) * 16);
        float d = 0.0f;
#pragma unroll
        for (int st = 0; st < NST; st++) d = dot16_i8(w[st], sh_h + j * I + (st * LPR + l) * 16, d);
        acc = fmaf(sh_w[j] * sh_s[j][c], d, acc);
    }
    acc = group_sum<LPR>(acc);
    if (l == 0) {
        if (y32) y32[c] = acc;
        if (ybf) ybf[c] = f32_to_bf16(acc);
    }
}

int launch_i8_gateup_m1(const Qf4ExpCache *c, const uint16_t *xb, const float *xf, const int *sel,
                        int nexp, const I8Shared *sh, float *hidden, hipStream_t s) {
    if (!c || !c->i8_gate || !c->i8_up || !c->i8s_gate || !c->i8s_up) {
        set_error(-1, "i8_gateup_m1: arena has no INT8 gate/up"); return -1;
    }
    if (nexp < 0 || nexp > 16 || (!xb && !xf) || !hidden || (nexp && !sel)) {
        set_error(-1, "i8_gateup_m1: bad arguments"); return -1;
    }
    JobPtrs jp{};
    if (sh) { jp.qg = sh->qg; jp.qu = sh->qu; jp.sg = sh->sg; jp.su = sh->su; }
    const int jobs = nexp + (sh ? 1 : 0);
    if (!jobs) return 0;
    const dim3 block(256);
    if (shape_2048()) {
        hipLaunchKernelGGL((k_i8_gateup_m1<2048, 512>), dim3(512 / 8, jobs), block, 0, s, c->i8_gate, c->i8_up,
                           c->i8s_gate, c->i8s_up, xb, xf, sel, nexp, jp, hidden);
    } else if (shape_2560()) {
        hipLaunchKernelGGL((k_i8_gateup_m1<2560, 640>), dim3(640 / 8, jobs), block, 0, s, c->i8_gate, c->i8_up,
                           c->i8s_gate, c->i8s_up, xb, xf, sel, nexp, jp, hidden);
    } else {
        set_error(-2, "i8_gateup_m1: unsupported shape"); return -2;
    }
    return check_launch("i8_gateup_m1");
}

int launch_i8_down_m1(const Qf4ExpCache *c, const float *hidden, const float *wts, const int *sel, int nexp,
                      const I8Shared *sh, const float *gdot, float *y32, uint16_t *ybf, hipStream_t s) {
    if (!c || !c->i8_down || !c->i8s_down) { set_error(-1, "i8_down_m1: arena has no INT8 down"); return -1; }
    if (nexp < 0 || nexp > 16 || !hidden || (!y32 && !ybf) || (nexp && (!sel || !wts))) {
        set_error(-1, "i8_down_m1: bad arguments"); return -1;
    }
    JobPtrs jp{};
    if (sh) { jp.qd = sh->qd; jp.sd = sh->sd; }
    const dim3 block(256);
    if (shape_2048()) {
        hipLaunchKernelGGL((k_i8_down_m1<2048, 512, 32>), dim3(2048 / 8), block, 0, s, c->i8_down, c->i8s_down,
                           hidden, wts, sel, nexp, jp, gdot, y32, ybf);
    } else if (shape_2560()) {
        hipLaunchKernelGGL((k_i8_down_m1<2560, 640, 8>), dim3(2560 / 32), block, 0, s, c->i8_down, c->i8s_down,
                           hidden, wts, sel, nexp, jp, gdot, y32, ybf);
    } else {
        set_error(-2, "i8_down_m1: unsupported shape"); return -2;
    }
    return check_launch("i8_down_m1");
}

}  // namespace qfm
