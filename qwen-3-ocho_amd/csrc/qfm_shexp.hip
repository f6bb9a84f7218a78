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
// GEMV, silu-mul, down GEMV, gated add) and 2 + 2M for M rows; here it is two:
//   k_shexp_gu   one wave per intermediate row, the gate and up rows of r
//                read once and dotted against every x row; one more wave for
//                gate_inp; silu(g) * u formed in registers.
//   k_shexp_down one wave per output row o of down, dotted against every
//                eg row, the gated add into y fused.
// Each lane owns the 8-value chunks c = lane + 64 j of a row (16-byte bf16
// loads, all issued before the first multiply), accumulates in fp32 in chunk
// order and the wave sums once (group_sum<64>). x and eg are read as fp32 from
// global memory (L2-resident: at most 8 rows).
#include "qfm_dev.h"
#include "qfm_internal.h"
#include "../../include/qf_dense.h"

namespace qfm {

constexpr int kShexpMaxRows = 8;
static_assert(sizeof(Qf8ShexpW) == 32, "Qf8ShexpW layout (qf8_dense.h:275-277)");

// dot of one 8-value bf16 chunk with 8 fp32 activations
__device__ __forceinline__ float dot8_bf16(const uint4 w, const float *__restrict__ x, float acc) {
    const float4 a = *reinterpret_cast<const float4 *>(x), b = *reinterpret_cast<const float4 *>(x + 4);
    acc = fmaf(bf16_lo(w.x), a.x, acc); acc = fmaf(bf16_hi(w.x), a.y, acc);
    acc = fmaf(bf16_lo(w.y), a.z, acc); acc = fmaf(bf16_hi(w.y), a.w, acc);
    acc = fmaf(bf16_lo(w.z), b.x, acc); acc = fmaf(bf16_hi(w.z), b.y, acc);
    acc = fmaf(bf16_lo(w.w), b.z, acc); acc = fmaf(bf16_hi(w.w), b.w, acc);
    return acc;
}

// NCH = 8-value chunks per row of length K (K / 8); chunk c = lane + 64 j, j < NJ
template <int K>
struct RowChunks {
    static constexpr int NCH = K / 8;
    static constexpr int NJ = (NCH + 63) / 64;
};

// blocks of 4 waves; wave w of block b handles intermediate row r = 4 b + w
// (r < I: gate and up rows r) or the gate_inp row (r == I)
template <int H, int I>
__global__ void __launch_bounds__(256)
k_shexp_gu(const uint16_t *__restrict__ Wg, const uint16_t *__restrict__ Wu, const uint16_t *__restrict__ Wgi,
           const float *__restrict__ x, int M, float *__restrict__ eg, float *__restrict__ eu,
           float *__restrict__ g1) {
    using RC = RowChunks<H>;
    const int lane = threadIdx.x & 63;
    const int r = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r > I) return;
    const bool gi = r == I;
    const uint4 *pg = reinterpret_cast<const uint4 *>((gi ? Wgi : Wg + (size_t)r * H));
    const uint4 *pu = reinterpret_cast<const uint4 *>(Wu + (size_t)(gi ? 0 : r) * H);
    uint4 wg[RC::NJ], wu[RC::NJ];
#pragma unroll
    for (int j = 0; j < RC::NJ; j++) {
        const int c = lane + 64 * j;
        const bool in = c < RC::NCH;
        wg[j] = in ? ld_nt16(pg + c) : make_uint4(0u, 0u, 0u, 0u);
        wu[j] = (in && !gi) ? ld_nt16(pu + c) : make_uint4(0u, 0u, 0u, 0u);
    }
    for (int m = 0; m < M; m++) {
        const float *xm = x + (size_t)m * H;
        float ag = 0.0f, au = 0.0f;
#pragma unroll
        for (int j = 0; j < RC::NJ; j++) {
            const int c = lane + 64 * j;
            if (c < RC::NCH) {
                ag = dot8_bf16(wg[j], xm + 8 * c, ag);
                if (!gi) au = dot8_bf16(wu[j], xm + 8 * c, au);
            }
        }
        ag = group_sum<64>(ag);
        au = group_sum<64>(au);
        if (lane == 0) {
            if (gi) {
                g1[m] = ag;
            } else {
                eu[(size_t)m * I + r] = au;
                eg[(size_t)m * I + r] = silu(ag) * au;
            }
        }
    }
}

// wave w of block b: output row o = 4 b + w of down; y[m * ys + o] += sigmoid(g1[m]) * ed[m][o]
template <int H, int I>
__global__ void __launch_bounds__(256)
k_shexp_down(const uint16_t *__restrict__ Wd, const float *__restrict__ eg, const float *__restrict__ g1, int M,
             float *__restrict__ ed, float *__restrict__ y, int ys) {
    using RC = RowChunks<I>;
    const int lane = threadIdx.x & 63;
    const int o = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= H) return;
    const uint4 *pd = reinterpret_cast<const uint4 *>(Wd + (size_t)o * I);
    uint4 wd[RC::NJ];
#pragma unroll
    for (int j = 0; j < RC::NJ; j++) {
        const int c = lane + 64 * j;
        wd[j] = c < RC::NCH ? ld_nt16(pd + c) : make_uint4(0u, 0u, 0u, 0u);
    }
    for (int m = 0; m < M; m++) {
        const float *em = eg + (size_t)m * I;
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < RC::NJ; j++) {
            const int c = lane + 64 * j;
            if (c < RC::NCH) a = dot8_bf16(wd[j], em + 8 * c, a);
        }
        a = group_sum<64>(a);
        if (lane == 0) {
            ed[(size_t)m * H + o] = a;
            float *yo = y + (size_t)m * ys + o;
            *yo = fmaf(sigmoid(g1[m]), a, *yo);
        }
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
    const int H = g_cfg.H, I = g_cfg.I;
    const dim3 b(256), ggu((unsigned)((I + 1 + 3) / 4)), gd((unsigned)((H + 3) / 4));
#define QFM_SHEXP(HH, II)                                                                                          \
    do {                                                                                                           \
        hipLaunchKernelGGL((k_shexp_gu<HH, II>), ggu, b, 0, s, w->gate, w->up, w->gate_inp, x, M, eg, eu, g1);     \
        hipLaunchKernelGGL((k_shexp_down<HH, II>), gd, b, 0, s, w->down, eg, g1, M, ed, y, ys);                    \
    } while (0)
    if (shape_2048()) QFM_SHEXP(2048, 512);
    else if (shape_2560()) QFM_SHEXP(2560, 640);
    else { set_error(-2, "%s: unsupported shape", who); return -2; }
#undef QFM_SHEXP
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
