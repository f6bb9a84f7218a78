/*
 * qf_fp8.h -- the FP8 lane-chunk expert arena and its MoE kernels.
 *
 * Format (ocho/amd_server/qf8_moe_fp8.h:8-23): every weight row of `in`
 * values is cut into 64 contiguous chunks of in/64 values; chunk l is stored
 * as E4M3 codes of value / sc[row][l], with one fp32 scale per (row, chunk).
 *   weights [slot][rows][in] bytes, scales [slot][rows][64] fp32;
 *   gate/up: rows = I, in = H; down: rows = H, in = I.
 * Every code byte decodes as the reference's integer decode does
 * (qf8_moe_fp8.hip:19-26): sign, 4-bit exponent (bias 7, subnormal step
 * 2^-9), 3-bit mantissa and no NaN, so 0x7F / 0xFF read +-480. (The packer,
 * qf8_fp8_pack_expert in qf_store.h, saturates at 0x7E and never emits them;
 * an arena filled another way may hold them.)
 *
 * Execution: a descriptor per distinct selected expert (ascending expert id,
 * its rows in token order, at most 16), then a fused gate/up and a fused
 * down + routed-weight accumulate over (descriptor, output-row tile) items.
 * The item count is read on the device (ctl[0]); each kernel is a fixed grid
 * that walks the items with a grid stride, so no cursor is shared between
 * workgroups. The arena must be fully resident: slot = slot_base + expert.
 */
#ifndef QF_FP8_H
#define QF_FP8_H
#include "qf_moe.h"

#ifdef __cplusplus
extern "C" {
#endif
#pragma GCC visibility push(default)

#define QF8_FP8_MAXROW 16   /* rows a descriptor carries */
#define QF8_FP8_CTL    4    /* ints of the control block */

/* Device expert descriptor (qf8_moe_fp8.h:37-44): byte-compatible. */
typedef struct {
    int   slot;
    int   nrow;
    int   row[QF8_FP8_MAXROW];
    float wt[QF8_FP8_MAXROW];
} Qf8MoeDesc;

/* sel/wt [M][K] -> descriptors (ascending expert id; rows t in order with the
 * first k where sel[t][k] == e; at most 16 rows, later rows dropped as in the
 * reference), ctl[0] = count, ctl[1] = ctl[2] = 0. desc holds min(M*K,
 * n_experts) entries. Replaces qf8_fp8_build_desc (qf8_moe_fp8.h:60-63). */
void qf8_fp8_build_desc(const int *sel_dev, const float *wt_dev, int M, int K, int slot_base, Qf8MoeDesc *desc,
                        int *ctl, hipStream_t s);
/* hidden[d][t][I] = silu(g) * u for every descriptor d and row t < nrow, with
 * g = sum over chunks l of sc_g[l] * (codes_l . x_l) (fp32), same for u.
 * x fp32 [M][H]. Replaces qf8_fp8_gateup (qf8_moe_fp8.h:64-67). */
void qf8_fp8_gateup(const uint8_t *Wg, const float *Sg, const uint8_t *Wu, const float *Su, const float *x,
                    float *hidden, const Qf8MoeDesc *desc, int *ctl, hipStream_t s);
/* y[row_t][o] += wt_t * down_o(hidden[d][t]) with atomics; y [M][H] fp32
 * pre-zeroed by the caller. Replaces qf8_fp8_downacc (qf8_moe_fp8.h:68-72). */
void qf8_fp8_downacc(const uint8_t *Wd, const float *Sd, const float *hidden, float *y, const Qf8MoeDesc *desc,
                     int *ctl, hipStream_t s);

/* Validated twins: 0, or -1 / -2 on a rejected argument (nothing launched),
 * -3 on a launch error. */
int qf8_fp8_build_desc_ex(const int *sel_dev, const float *wt_dev, int M, int K, int slot_base, Qf8MoeDesc *desc,
                          int *ctl, hipStream_t s);
int qf8_fp8_gateup_ex(const uint8_t *Wg, const float *Sg, const uint8_t *Wu, const float *Su, const float *x,
                      float *hidden, const Qf8MoeDesc *desc, int *ctl, hipStream_t s);
int qf8_fp8_downacc_ex(const uint8_t *Wd, const float *Sd, const float *hidden, float *y, const Qf8MoeDesc *desc,
                       int *ctl, hipStream_t s);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
