// qfm_shexp.hip -- the bf16 shared expert of the NVFP4 stage (qf8_shexp /
// qf8_shexp_M).
//
// Reference behaviour: ocho/amd_server/qf8_layer.hip:23-54 with the weights of
// Qf8ShexpW (qf8_dense.h:275-286), all bf16:
//   eu[m] = up . x[m],  g1[m] = gate_inp . x[m],  eg[m] = silu(gate . x[m]) * eu[m]
//   ed[m] = down . eg[m],  y[m] += sigmoid(g1[m]) * ed[m]
// with x fp32 [M][H] (the mixer output), gate/up bf16 [I][H], gate_inp bf16
// [H], down bf16 [H][I]; M <= 8 rows (the reference's QF8_M_MAX,
// qf8_gemv_m.hip:10-12). Its call sites: qf_hip4_stage.hip:1631-1635 (rows)
// and :2105-2107 (one row).
//
// The reference makes it four launches for one row (fused gate/up/gate_inp
// GEMV, silu-mul, down GEMV, gated add) and 2 + 2M for M rows; here it is two,
// each with the M rows as a template parameter (all of a thread's activation
// loads issued together, one reduction for every row):
//   k_shexp_gu   block b: intermediate rows R b + i, i < R (row I is
//                gate_inp, gate only). Thread t owns the 8-value chunks
//                c = t + 256 q of the H dimension for all R rows and both
//                matrices (each x element read once per block for 2R weight
//                rows); per-wave reduce-scatter of the R x 2 x M
//                partial sums, then the four waves' sums added in LDS in wave
//                order.
//   k_shexp_down block b, wave w: output rows o = D (W b + w) + j, j < D;
//                lane l owns the chunks c = l + 64 q of the I dimension of all
//                D rows; reduce-scatter of the D x M sums; the gated add into
//                y fused.
// Sums accumulate in fp32 over chunk order, then across lanes.
#include "qfm_dev.h"
#include "qfm_internal.h"
#include "../../include/qf_dense.h"

namespace qfm {

constexpr int kShexpMaxRows = 8;
static_assert(sizeof(Qf8ShexpW) == 32, "Qf8ShexpW layout (qf8_dense.h:275-277)");

// dot of one 8-value bf16 chunk with 8 fp32 activations
__device__ __forceinline__ float dot8_bf16(const uint4 w, const float4 a, const float4 b, float acc) {
    acc = fmaf(bf16_lo(w.x), a.x, acc); acc = fmaf(bf16_hi(w.x), a.y, acc);
    acc = fmaf(bf16_lo(w.y), a.z, acc); acc = fmaf(bf16_hi(w.y), a.w, acc);
    acc = fmaf(bf16_lo(w.z), b.x, acc); acc = fmaf(bf16_hi(w.z), b.y, acc);
    acc = fmaf(bf16_lo(w.w), b.z, acc); acc = fmaf(bf16_hi(w.w), b.w, acc);
    return acc;
}

constexpr int pow2_ceil(int v) { return v <= 1 ? 1 : v <= 2 ? 2 : v <= 4 ? 4 : 8; }

// Reduce-scatter of N = 2^k <= 32 per-lane values over the 64 lanes of a wave:
// lane l returns the wave total of value l & (N - 1).
template <int N>
__device__ __forceinline__ float wave_scatter_sum(const float (&v)[N], int lane) {
    static_assert(N >= 1 && N <= 32 && (N & (N - 1)) == 0, "2^k <= 32 values");
    if constexpr (N == 1) return group_sum<64>(v[0]);
    else return canon_scatter_level<N, 1>(v, lane);
}

// Rows per k_shexp_gu block and per k_shexp_down wave, and waves per down
// block, as measured best over 48 graph-replayed weight sets (H 2048, I 512):
// gate/up 1 row per block (1, 2, 4, 8 measured: more rows per block saves L2
// reads of x but leaves fewer blocks to stream the weights; M = 1 5.4-5.6 us
// per layer against 6.0-7.7 us with 2-8 rows), down 1 row per wave up to
// M = 2 and 2 rows above (M = 8: 7.7 us against 8.0 with 1 row and 8.2-8.8
// with 4-8), 4 waves per down block.
constexpr int gu_rows(int) { return 1; }
constexpr int dn_rows(int M) { return M <= 2 ? 1 : 2; }
constexpr int kDnWaves = 4;

template <int H, int I, int M>
__global__ void __launch_bounds__(256)
k_shexp_gu(const uint16_t *__restrict__ Wg, const uint16_t *__restrict__ Wu, const uint16_t *__restrict__ Wgi,
           const float *__restrict__ x, float *__restrict__ eg, float *__restrict__ eu, float *__restrict__ g1) {
    constexpr int NCH = H / 8, CPT = (NCH + 255) / 256, MP = pow2_ceil(M), kGuRows = gu_rows(M);
    constexpr int NV = kGuRows * 2 * MP;                     // value (i, mat, m) at (2 i + mat) MP + m
    static_assert(NV <= 32, "partial sums per lane");
    __shared__ float s_red[4][NV];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int r0 = (int)blockIdx.x * kGuRows;
    uint4 wg[kGuRows][CPT], wu[kGuRows][CPT];
#pragma unroll
    for (int i = 0; i < kGuRows; i++) {
        const int r = r0 + i;
        const uint16_t *gp = r < I ? Wg + (size_t)r * H : Wgi;   // row I: gate_inp
#pragma unroll
        for (int q = 0; q < CPT; q++) {
            const int c = t + 256 * q;
            const bool in = c < NCH;
            wg[i][q] = (in && r <= I) ? ld_nt16(gp + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
            wu[i][q] = (in && r < I) ? ld_nt16(Wu + (size_t)r * H + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    float4 xa[M][CPT], xb[M][CPT];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int q = 0; q < CPT; q++) {
            const int c = t + 256 * q;
            const float4 *xp = reinterpret_cast<const float4 *>(x + (size_t)m * H) + 2 * c;
            xa[m][q] = c < NCH ? xp[0] : make_float4(0.f, 0.f, 0.f, 0.f);
            xb[m][q] = c < NCH ? xp[1] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    float v[NV];
#pragma unroll
    for (int i = 0; i < kGuRows; i++)
#pragma unroll
        for (int m = 0; m < MP; m++) {
            float ag = 0.0f, au = 0.0f;
            if (m < M) {
#pragma unroll
                for (int q = 0; q < CPT; q++) {
                    ag = dot8_bf16(wg[i][q], xa[m < M ? m : 0][q], xb[m < M ? m : 0][q], ag);
                    au = dot8_bf16(wu[i][q], xa[m < M ? m : 0][q], xb[m < M ? m : 0][q], au);
                }
            }
            v[(2 * i) * MP + m] = ag;
            v[(2 * i + 1) * MP + m] = au;
        }
    const float sw = wave_scatter_sum<NV>(v, lane);
    if (lane < NV) s_red[wave][lane] = sw;
    __syncthreads();
    if (t < kGuRows * MP) {
        const int i = t / MP, m = t % MP, r = r0 + i;
        if (m < M && r <= I) {
            const float g = ((s_red[0][2 * i * MP + m] + s_red[1][2 * i * MP + m]) + s_red[2][2 * i * MP + m]) +
                            s_red[3][2 * i * MP + m];
            if (r == I) {
                g1[m] = g;
            } else {
                const int ku = (2 * i + 1) * MP + m;
                const float u = ((s_red[0][ku] + s_red[1][ku]) + s_red[2][ku]) + s_red[3][ku];
                eu[(size_t)m * I + r] = u;
                eg[(size_t)m * I + r] = silu(g) * u;
            }
        }
    }
}

template <int H, int I, int M>
__global__ void __launch_bounds__(64 * kDnWaves)
k_shexp_down(const uint16_t *__restrict__ Wd, const float *__restrict__ eg, const float *__restrict__ g1,
             float *__restrict__ ed, float *__restrict__ y, int ys) {
    constexpr int NCH = I / 8, CPL = (NCH + 63) / 64, MP = pow2_ceil(M), kDnRows = dn_rows(M);
    constexpr int NV = kDnRows * MP;                         // value (j, m) at j MP + m
    static_assert(NV <= 32, "partial sums per lane");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int o0 = ((int)blockIdx.x * kDnWaves + wave) * kDnRows;
    uint4 wd[kDnRows][CPL];
#pragma unroll
    for (int j = 0; j < kDnRows; j++)
#pragma unroll
        for (int q = 0; q < CPL; q++) {
            const int c = lane + 64 * q;
            wd[j][q] = (c < NCH && o0 + j < H) ? ld_nt16(Wd + (size_t)(o0 + j) * I + 8 * c)
                                               : make_uint4(0u, 0u, 0u, 0u);
        }
    float4 ea[M][CPL], eb[M][CPL];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int q = 0; q < CPL; q++) {
            const int c = lane + 64 * q;
            const float4 *ep = reinterpret_cast<const float4 *>(eg + (size_t)m * I) + 2 * c;
            ea[m][q] = c < NCH ? ep[0] : make_float4(0.f, 0.f, 0.f, 0.f);
            eb[m][q] = c < NCH ? ep[1] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    float v[NV];
#pragma unroll
    for (int j = 0; j < kDnRows; j++)
#pragma unroll
        for (int m = 0; m < MP; m++) {
            float a = 0.0f;
            if (m < M) {
#pragma unroll
                for (int q = 0; q < CPL; q++) a = dot8_bf16(wd[j][q], ea[m < M ? m : 0][q], eb[m < M ? m : 0][q], a);
            }
            v[j * MP + m] = a;
        }
    const float a = wave_scatter_sum<NV>(v, lane);
    const int j = (lane & (NV - 1)) / MP, m = lane & (MP - 1), o = o0 + j;
    if (lane < NV && m < M && o < H) {
        ed[(size_t)m * H + o] = a;
        float *yo = y + (size_t)m * ys + o;
        *yo = fmaf(sigmoid(g1[m]), a, *yo);
    }
}

static int shexp_launch(const Qf8ShexpW *w, const float *x, int M, float *eg, float *eu, float *g1, float *ed,
                        float *y, int ys, hipStream_t s, const char *who) {
    if (!w || !w->gate || !w->up || !w->down || !w->gate_inp || !x || !eg || !eu || !g1 || !ed || !y) {
        set_error(-1, "%s: null pointer", who); return -1;
    }
    if (M < 1 || M > kShexpMaxRows || ys < g_cfg.H) {
        set_error(-1, "%s: M = %d (1..%d rows) or y stride %d below H = %d", who, M, kShexpMaxRows, ys, g_cfg.H);
        return -1;
    }
    const dim3 bgu(256), bd(64 * kDnWaves);
#define QFM_SHEXP_M(HH, II, MM)                                                                                    \
    case MM:                                                                                                       \
        hipLaunchKernelGGL((k_shexp_gu<HH, II, MM>), dim3((II + gu_rows(MM)) / gu_rows(MM)), bgu, 0, s, w->gate,   \
                           w->up, w->gate_inp, x, eg, eu, g1);                                                     \
        hipLaunchKernelGGL((k_shexp_down<HH, II, MM>), dim3((HH + dn_rows(MM) * kDnWaves - 1) /                    \
                           (dn_rows(MM) * kDnWaves)), bd, 0, s, w->down, eg, g1, ed, y, ys);                       \
        break;
#define QFM_SHEXP(HH, II)                                                                                          \
    switch (M) {                                                                                                   \
        QFM_SHEXP_M(HH, II, 1) QFM_SHEXP_M(HH, II, 2) QFM_SHEXP_M(HH, II, 3) QFM_SHEXP_M(HH, II, 4)                \
        QFM_SHEXP_M(HH, II, 5) QFM_SHEXP_M(HH, II, 6) QFM_SHEXP_M(HH, II, 7) QFM_SHEXP_M(HH, II, 8)                \
        default: break;                                                                                            \
    }
    if (shape_2048()) { QFM_SHEXP(2048, 512) }
    else if (shape_2560()) { QFM_SHEXP(2560, 640) }
    else { set_error(-2, "%s: unsupported shape", who); return -2; }
#undef QFM_SHEXP
#undef QFM_SHEXP_M
    return check_launch(who);
}

}  // namespace qfm

using namespace qfm;

extern "C" {

int qf8_shexp_ex(const Qf8ShexpW *w, const float *mixed, float *eg, float *eu, float *g1, float *ed, float *y2560,
                 hipStream_t s) {
    return shexp_launch(w, mixed, 1, eg, eu, g1, ed, y2560, g_cfg.H, s, "qf8_shexp");
}
void qf8_shexp(const Qf8ShexpW *w, const float *mixed, float *eg, float *eu, float *g1, float *ed, float *y2560,
               hipStream_t s) {
    (void)qf8_shexp_ex(w, mixed, eg, eu, g1, ed, y2560, s);
}
int qf8_shexp_M_ex(const Qf8ShexpW *w, const float *mixed, int M, float *eg, float *eu, float *g1, float *ed,
                   float *y2560, int eg_stride, int y_stride, hipStream_t s) {
    (void)eg_stride;   // eg / eu rows are I apart, as in the reference (qf8_layer.hip:39)
    return shexp_launch(w, mixed, M, eg, eu, g1, ed, y2560, y_stride, s, "qf8_shexp_M");
}
void qf8_shexp_M(const Qf8ShexpW *w, const float *mixed, int M, float *eg, float *eu, float *g1, float *ed,
                 float *y2560, int eg_stride, int y_stride, hipStream_t s) {
    (void)qf8_shexp_M_ex(w, mixed, M, eg, eu, g1, ed, y2560, eg_stride, y_stride, s);
}

}  // extern "C"
