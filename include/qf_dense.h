/*
 * qf_dense.h -- the dense INT8 projections either side of the MoE: the
 * INT8 x X8 GEMV (router and shared-expert in-projections, hyper-connection
 * projections), the FFN-side hyper-connection pre-mixer that emits the MoE
 * input, and the residual-stream inject after the MoE.
 *
 * Shapes: the residual holds HCC = 4 streams of H values (R [4][H]); the
 * hyper-connection low rank is HCL = 320. X8 rows: int8 codes with one fp32
 * scale per 32 values (value = code * scale; qf8_i8_x8's rule).
 */
#ifndef QF_DENSE_H
#define QF_DENSE_H
#include "qf_moe.h"

#ifdef __cplusplus
extern "C" {
#endif
#pragma GCC visibility push(default)

#define QF8_HCC 4     /* residual streams */
#define QF8_HCL 320   /* hyper-connection low rank */

/* Up to 4 INT8 matrices sharing one X8 activation row (ocho/amd_server/
 * qf8_dense_i8.h:31-33): y[i][r] = act_i(s_i[r] * sum_b xs[b] * (W_i[r] .
 * xq)[block b]) with the block dots exact in int32. act: 0 none, 1
 * silu(v/4) = (v/4) / (1 + exp(-v/4)), 2 2*sigmoid(v/4). Every matrix has the
 * same K, one of 320, 512, 640, 2048, 2560, 6144, 8192, 10240. */
typedef struct { const Qf8I8Mat *m[4]; float *y[4]; int act[4]; int n; } Qf8I8Multi;
/* Replaces qf8_i8_gemv_multi (qf8_dense_i8.h:33, qf8_dense_i8.hip:328-345). */
void qf8_i8_gemv_multi(const Qf8I8Multi *mm, const int8_t *xq, const float *xs, hipStream_t s);
/* T X8 rows: xq [T][K], xs [T][K/32]; y[i] [T][rows_i]. 0 or -1. Replaces
 * qf8_i8_gemv_rows (qf8_dense_i8.h:35, qf8_dense_i8.hip:252-263). */
int  qf8_i8_gemv_rows(const Qf8I8Multi *mm, const int8_t *xq, const float *xs, int T, hipStream_t s);

/* FFN-side hyper-connection pre-mixer, one row (qf8_dense_i8.h:47-58,
 * qf8_dense_i8.hip:109-175, :360-375):
 *   (optional) R[c] += inj_prev[c] * y_prev          (previous mixer's inject, fused)
 *   normed[c] = R[c] * rstd_c * (1 + wn[c])           rstd_c = 1/sqrt(mean(R[c]^2) + 1e-6), wn bf16 [4H]
 *   n8q/n8s = X8(normed)                              [4H] / [4H/32]
 *   hc_d = silu(down . normed / 4) [320];  inj = 2 sigmoid(inject . normed / 4) [4] (inject may be NULL)
 *   d8q/d8s = X8(hc_d);  hcy = up . hc_d [4H]
 *   mixed[j] = 1/4 sum_c sigmoid(hcy[c][j]) * normed[c][j] [H];  xq_out/xs_out = X8(mixed)
 * down [320][4H], inject [4][4H], up [4H][320] INT8 matrices. Replaces qf8_i8_hc_m1.
 * One row (T = 1) runs as one launch whose up blocks take hc_d and normed from
 * the down blocks through a hand-off area that the library keeps in device
 * memory, one per GPU: one-row calls (here, qf8_i8_hc_rows and qfm_hc_premix
 * at T = 1) that overlap in time on one GPU must be serialized by the caller. */
void qf8_i8_hc_m1(float *normed, float *hc_d, float *mixed, float *inj, float *R, const uint16_t *wn,
                  const Qf8I8Mat *down, const Qf8I8Mat *inject, const Qf8I8Mat *up, int8_t *n8q, float *n8s,
                  int8_t *d8q, float *d8s, float *hcy, const float *y_prev, const float *inj_prev, int8_t *xq_out,
                  float *xs_out, hipStream_t s);
/* The same over T rows (every buffer gains a leading [T]). 0 or -1. Replaces
 * qf8_i8_hc_rows (qf8_dense_i8.h:36-39, qf8_dense_i8.hip:265-281). */
int  qf8_i8_hc_rows(float *normed, float *hc_d, float *mixed, float *inj, float *R, const uint16_t *wn,
                    const Qf8I8Mat *down, const Qf8I8Mat *inject, const Qf8I8Mat *up, int8_t *n8q, float *n8s,
                    int8_t *d8q, float *d8s, float *hcy, const float *y_prev, const float *inj_prev, int8_t *xq_out,
                    float *xs_out, int T, hipStream_t s);
/* qf8_i8_hc_m1 (T = 1) / qf8_i8_hc_rows that also writes x_bf16 [T][H] =
 * bf16(mixed) (round to nearest even): the input row of qfm_moe_forward /
 * qfm_moe_forward_f32, so the fused MoE path follows the mixer with no
 * conversion launch (the reference's experts read X8(mixed) instead,
 * qf_hip4_stage.hip:1508-1515). Every other output as in qf8_i8_hc_m1. No
 * counterpart in the reference. 0 or -1 / -2 / -3. */
int  qfm_hc_premix(float *normed, float *hc_d, float *mixed, float *inj, float *R, const uint16_t *wn,
                   const Qf8I8Mat *down, const Qf8I8Mat *inject, const Qf8I8Mat *up, int8_t *n8q, float *n8s,
                   int8_t *d8q, float *d8s, float *hcy, const float *y_prev, const float *inj_prev, int8_t *xq_out,
                   float *xs_out, uint16_t *x_bf16, int T, hipStream_t s);
/* The count of hand-off words whose bounded wait ran out in one-row pre-mixer
 * calls on the current GPU since the library was loaded (0 unless a launch
 * could not run its blocks together). Synchronous copy. No counterpart in the
 * reference. 0, or -1 / -3 / -5. */
int  qfm_hc_wait_timeouts(uint32_t *count);
/* R[c][i] = fma(inj[c], y[i], R[c][i]) for the 4 streams: the MoE output
 * written back into the residual. Replaces qf8_stream_inject (qf8_dense.h:158,
 * qf8_hc.hip:99-103, :148-150). */
void qf8_stream_inject(float *R, const float *y, const float *inj, hipStream_t s);

/* bf16 shared expert of the NVFP4 stage (ocho/amd_server/qf8_dense.h:275-286):
 * gate, up [I][H], gate_inp [H], down [H][I], all bf16. */
typedef struct { const uint16_t *gate, *up, *down, *gate_inp; } Qf8ShexpW;
/* One row: y2560[H] += sigmoid(g1) * ed, with x = mixed fp32 [H] and, written
 * as in the reference, eu [I] = up . x, g1 [1] = gate_inp . x,
 * eg [I] = silu(gate . x) * eu, ed [H] = down . eg (fp32 accumulate).
 * Replaces qf8_shexp (qf8_dense.h:280-282, qf8_layer.hip:42-54). */
void qf8_shexp(const Qf8ShexpW *w, const float *mixed, float *eg, float *eu, float *g1, float *ed,
               float *y2560, hipStream_t s);
/* 1 <= M <= 8 rows (the reference's QF8_M_MAX): mixed [M][H], eg / eu [M][I],
 * g1 [M], ed [M][H], y2560 row m at m * y_stride (>= H); eg_stride is accepted
 * and not used (eg rows are I apart, as in the reference). Each weight byte is
 * read once for all rows. Replaces qf8_shexp_M (qf8_dense.h:284-286,
 * qf8_layer.hip:23-40). */
void qf8_shexp_M(const Qf8ShexpW *w, const float *mixed, int M, float *eg, float *eu, float *g1, float *ed,
                 float *y2560, int eg_stride, int y_stride, hipStream_t s);

/* Validated twins: 0, or -1 / -2 on a rejected argument (nothing launched),
 * -3 on a launch error. */
int  qf8_i8_gemv_multi_ex(const Qf8I8Multi *mm, const int8_t *xq, const float *xs, hipStream_t s);
int  qf8_i8_hc_m1_ex(float *normed, float *hc_d, float *mixed, float *inj, float *R, const uint16_t *wn,
                     const Qf8I8Mat *down, const Qf8I8Mat *inject, const Qf8I8Mat *up, int8_t *n8q, float *n8s,
                     int8_t *d8q, float *d8s, float *hcy, const float *y_prev, const float *inj_prev, int8_t *xq_out,
                     float *xs_out, hipStream_t s);
int  qf8_stream_inject_ex(float *R, const float *y, const float *inj, hipStream_t s);
int  qf8_shexp_ex(const Qf8ShexpW *w, const float *mixed, float *eg, float *eu, float *g1, float *ed,
                  float *y2560, hipStream_t s);
int  qf8_shexp_M_ex(const Qf8ShexpW *w, const float *mixed, int M, float *eg, float *eu, float *g1, float *ed,
                    float *y2560, int eg_stride, int y_stride, hipStream_t s);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
