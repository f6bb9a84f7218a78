/*
 * qf_moe.h -- C ABI of the MI355X (gfx950) quantized MoE expert path.
 *
 * Drop-in for the MoE operator layer of the qwen-3-ocho engine: the router
 * GEMV + softmax/top-k, the per-row expert gather (routing inversion), the
 * INT8 and NVFP4 expert gate/up/down GEMVs/GEMMs and the gated shared expert.
 * Reference-named entry points keep the reference's names, argument order and
 * meaning; each cites the declaration it replaces (paths relative to the
 * reference checkout). Entry points prefixed qfm_ are this library's own: the
 * runtime shape configuration, the fused per-layer forward, the synthetic
 * arena generator and the harness utilities (device memory, streams, events)
 * used by tests and benchmarks that do not link a HIP runtime themselves.
 *
 * Conventions (as in the reference):
 *   - all launchers are asynchronous and stream-ordered; none synchronizes
 *     the host and none allocates device memory;
 *   - reference-named launchers return void; errors are latched and read with
 *     qfm_last_error() / qfm_status() (the reference surfaces launch errors
 *     through hipGetLastError at the caller);
 *   - qfm_ entry points return 0 on success and a negative code on a rejected
 *     argument (nothing is launched then);
 *   - every buffer is caller-owned device memory unless stated otherwise.
 */
#ifndef QF_MOE_H
#define QF_MOE_H
#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif
#pragma GCC visibility push(default)

/* ------------------------------------------------------------------------ */
/* Shape configuration. Replaces the reference's compile-time dimensions
 * QF5_NEMBD / QF5_NFF / QF5_NEXP / QF5_NEXPUSED (ocho/amd_server/
 * qf_nvfp4_wave64.h:54-57) and QF5_K (qf8_moe_i8.hip:5-7). Supported:
 * (hidden, inter) = (2048, 512) [benchmark shape] and (2560, 640) [reference
 * checkpoint]; n_experts == 512 (the reference's QF5_NEXP, which every path
 * here is built for; other counts are rejected); 1 <= top_k <= 16. */
typedef struct {
    int hidden;        /* H */
    int inter;         /* I: expert intermediate size */
    int n_experts;     /* E: routed experts */
    int top_k;         /* K: experts per row */
    int renorm;        /* 1: renormalize the K selected weights (norm_topk_prob,
                          qf_router_wave64.hip:149-154); 0: plain softmax probs */
    int shared_gated;  /* 1: y += sigmoid(<g,x>) * shared(x) (qf8_dense_i8.hip:177-181) */
} qfm_config;
int         qfm_init(const qfm_config *cfg);
int         qfm_get_config(qfm_config *cfg);
const char *qfm_last_error(void);   /* "" when no error is latched; reading clears it */
int         qfm_status(void);       /* 0, or the latched error code; also polls hipGetLastError */
const char *qfm_version(void);
/* Memory preflight, the reference's budget guard (qf_hip4_stage.hip:792-813):
 * every entry that allocates arena-sized memory (qfm_arena_init,
 * qfm_synth_layer_create, qfm_expcache_init / qf4_expcache_init,
 * qfm_layer_load) prices all of its device bytes first and refuses, with -4
 * and nothing allocated, a plan larger than the device's free memory or one
 * that would take the device's memory in use above the budget. budget 0: no
 * limit beyond the device. Default: QFM_HBM_BUDGET_MIB from the environment
 * (MiB), else 0. Process-wide, not thread-safe. */
int         qfm_set_hbm_budget(size_t bytes);
size_t      qfm_get_hbm_budget(void);
/* sizeof of the ABI structs (0 Qf4ExpCache, 1 qfm_layer, 2 qfm_synth_layer,
   3 Qf8I8Mat, 4 Qf5M8Route, 5 qfm_config, 6 qfm_ws_view, 7 QfEntry, 8 QfStore,
   9 Qf4ExpXfer, 10 QfRouteMailbox) for FFI layout checks. */
size_t      qfm_sizeof(int which);

/* ------------------------------------------------------------------------ */
/* Expert arena: byte-compatible with the reference's Qf4ExpCache
 * (ocho/amd_server/qf_nvfp4_wave64.h:133-173) so an engine built against it
 * passes the same struct. Fields this library reads:
 *   INT8  : i8_gate/i8_up [slots][I][H], i8_down [slots][H][I] int8,
 *           i8s_gate/i8s_up [slots][I], i8s_down [slots][H] fp32 row scales
 *           (qf8_moe_i8.h:10-17);
 *   NVFP4 : w_gate/w_up [slots][I][H/2], w_down [slots][H][I/2] packed e2m1
 *           (byte i = element 2i low nibble | element 2i+1 high nibble),
 *           s_gate/s_up [slots][I][H/16], s_down [slots][H][I/16] e4m3 block
 *           scales, s2g_dev/s2u_dev/s2d_dev [E] fp32 per-expert global scales;
 *   slots == n_experts with slot == expert (fully resident arena). */
typedef struct QfRouteMailbox QfRouteMailbox;   /* opaque here; pointer only */
typedef struct {
    int       layer;
    int       slots;
    uint8_t  *w_gate, *w_up, *w_down;
    uint8_t  *w8_gate, *w8_up, *w8_down;
    float    *sc_gate, *sc_up, *sc_down;
    int8_t   *i8_gate, *i8_up, *i8_down;
    float    *i8s_gate, *i8s_up, *i8s_down;
    int       nv_ring;
    uint8_t  *s_gate, *s_up, *s_down;
    int      *slot_for_expert;
    int      *expert_in_slot;
    uint64_t *age;
    uint64_t  clock;
    float    *s2g, *s2u, *s2d;
    int       fully_resident;
    int      *slot_for_expert_dev;
    int      *expert_in_slot_dev;
    uint64_t *age_dev;
    uint64_t *clock_dev;
    float    *s2g_dev, *s2u_dev, *s2d_dev;
    int      *route_slot_dev;
    QfRouteMailbox *mb_host;
    QfRouteMailbox *mb_dev;
    uint32_t  expected_seq;
} Qf4ExpCache;

/* INT8 dense matrix: [rows][K] int8 + fp32 per-row scale
 * (ocho/amd_server/qf8_dense_i8.h:19). */
typedef struct { int8_t *w; float *s; int rows, K; } Qf8I8Mat;

/* Per-batch routing view of the M=8 kernels (ocho/amd_server/qf_moe_m8_wave64.h:33-45). */
typedef struct {
    int  n_exp;
    int  n_pairs;
    int  M;
    int  n_exp_max;
    const int   *n_exp_dev;
    const int   *exp_slot;
    const int   *exp_ptr;
    const int   *pair_tok;
    const float *pair_wt;
} Qf5M8Route;

/* ------------------------------------------------------------------------ */
/* Router. */
/* logits[E] = Router_bf16[E][H] . x_f32[H], fp32 accumulate.
 * Replaces qf_rtr_gemv / qf_rtr_gemv_launch (ocho/amd_server/qf_router_wave64.h:48, :81-84). */
void qf_rtr_gemv_launch(const uint16_t *router, const float *x, float *logits, hipStream_t s);
/* Softmax over all E logits + top-K (ties to the lower expert index) + renorm.
 * Replaces qf_rtr_topk10 / qf_rtr_topk10_launch (qf_router_wave64.h:53, :91-94)
 * and the rows form qf_rtr_topk10_rows_launch (:96-98). K = qfm_config.top_k. */
void qf_rtr_topk10_launch(const float *logits, int *sel_ids, float *wts, hipStream_t s);
void qf_rtr_topk10_rows_launch(const float *logits, int *sel_ids, float *wts, int T, hipStream_t s);
/* Benchmark router form (fp32 weights): logits[m][e] = W_f32[e] . x_bf16[m] (+ bias[e]) in the
 * library's canonical fp32 order (bit-reproducible on the host), M rows. */
int qfm_router_logits(const float *W, const float *bias, const uint16_t *x, int M,
                      float *logits, hipStream_t s);
int qfm_topk(const float *logits, int M, int *sel, float *wts, hipStream_t s);

/* ------------------------------------------------------------------------ */
/* INT8 routed experts, one row (M=1). */
/* hidden[k][I] = silu(sg * Wg.x) * (su * Wu.x) for the nexp experts sel_ids[0..nexp).
 * The activations are X8 rows, as in the reference (qf8_moe_i8.hip:416-421):
 * x8q int8 [H] codes with x8s fp32 [H/32] block scales (value = code * scale,
 * dequantized in registers). quant_x != 0: x (fp32 [H]) is quantized into
 * x8q/x8s first (qf8_i8_x8's rule); quant_x == 0: x8q/x8s already hold the
 * caller's X8 row and x is not read (may be NULL).
 * Replaces qf8_i8_gateup_m1 (ocho/amd_server/qf8_moe_i8.h:41-42). */
void qf8_i8_gateup_m1(const Qf4ExpCache *c, const float *x, int8_t *x8q, float *x8s,
                      float *hidden, const int *sel_ids, int nexp, int quant_x, hipStream_t s);
/* y[H] = sum_k wts[k] * sd * Wd.hidden[k] in fixed k order; y is SEEDED
 * (overwritten, one writer per row). h8q/h8s are accepted and not written:
 * the hidden vectors stay fp32 (staged as fp16 chunks with a power-of-two
 * scale per 16 values) instead of the reference's X8 re-quantization.
 * Replaces qf8_i8_down_m1 (qf8_moe_i8.h:45-46). */
void qf8_i8_down_m1(const Qf4ExpCache *c, const float *hidden, int8_t *h8q, float *h8s,
                    const float *wts, const int *sel_ids, float *y, int nexp, hipStream_t s);

/* X8 activation quantizer: per 32-value block s = absmax/127 (1 for an
 * all-zero block), q = rint(v/s) clamped to +-127; n a multiple of 32.
 * Replaces qf8_i8_x8 (ocho/amd_server/qf8_dense_i8.h:30); same rule as
 * k_i8_x8quant (qf8_moe_i8.hip:58-70). */
void qf8_i8_x8(const float *x, int8_t *q, float *sc, int n, hipStream_t s);

/* ------------------------------------------------------------------------ */
/* INT8 chunk (CSR) tier: T token rows with their own routing. */
/* Routing inversion of sel/wt [T][K]: exp_slot[n] ascending expert ids,
 * exp_ptr[n+1], pair_tok/pair_wt [T*K] in (expert, token) order,
 * counts = {n_exp, n_pairs}. Any T; deterministic.
 * Replaces qf8_i8_csr_build (ocho/amd_server/qf8_moe_i8.h:53-54). */
void qf8_i8_csr_build(const int *sel, const float *wt, int T, int *exp_slot, int *exp_ptr,
                      int *pair_tok, float *pair_wt, int *counts, hipStream_t s);
/* Every distinct expert's rows read once and dotted with its tokens' X8 rows
 * xq/xs [T][H]; hidden [pairs][I] fp32; owned partials part [T*K][H]
 * (the k of a pair is the position of exp_slot in the token's sel row); y
 * [T][H] fp32 OVERWRITTEN with the sum of the K partials in k order.
 * h8q/h8s and n_pairs_max are accepted and unused (hidden stays fp32).
 * Replaces qf8_i8_experts_chunk (qf8_moe_i8.h:55-59). */
void qf8_i8_experts_chunk(const Qf4ExpCache *c, const int8_t *xq, const float *xs,
                          float *hidden, int8_t *h8q, float *h8s,
                          const int *exp_slot, const int *exp_ptr, const int *pair_tok,
                          const float *pair_wt, const int *n_exp_dev, int n_exp_max,
                          int n_pairs_max, const int *sel, float *part, int T, float *y, hipStream_t s);

/* INT8 arena from the NVFP4 slots: value = e2m1 * ue4m3 * s2 (s2 per slot),
 * row scale = absmax/127, code = rint(value/scale) clamped to +-127. c->i8_*
 * must be allocated. Returns 0, or -1 on a missing buffer / launch error.
 * Replaces qf8_i8_build and qf8_i8_build_slot (qf8_moe_i8.h:34-37; the slot
 * form uses the s2 of `expert`). */
int qf8_i8_build(Qf4ExpCache *c, hipStream_t s);
int qf8_i8_build_slot(Qf4ExpCache *c, int src_slot, int dst_slot, int expert, hipStream_t s);

/* ------------------------------------------------------------------------ */
/* NVFP4 routed experts, one row (M=1). Weights by slot_ids[k] (slot < 0:
 * hidden row zero, no contribution), s2 tables by expert sel_ids[k]; x fp32
 * [H]; hidden [nexp][I]; y [H] SEEDED (one writer per row, fixed k order).
 * Replace qf5_nvfp4_moe_all, qf5_nvfp4_gateup_all_launch and
 * qf5_nvfp4_downacc_all_launch (ocho/amd_server/qf_nvfp4_wave64.h:218-237). */
void qf5_nvfp4_moe_all(const uint8_t *Wg, const uint8_t *Sg,
                       const uint8_t *Wu, const uint8_t *Su,
                       const uint8_t *Wd, const uint8_t *Sd,
                       const float *x, float *hidden, float *y,
                       const float *s2g_dev, const float *s2u_dev,
                       const float *s2d_dev, const float *wts,
                       const int *sel_ids, const int *slot_ids,
                       int nexp, hipStream_t stream);
void qf5_nvfp4_gateup_all_launch(const uint8_t *Wg, const uint8_t *Sg,
                                 const uint8_t *Wu, const uint8_t *Su,
                                 const float *x, float *hidden,
                                 const float *s2g_dev, const float *s2u_dev,
                                 const int *sel_ids, const int *slot_ids,
                                 int nexp, hipStream_t stream);
void qf5_nvfp4_downacc_all_launch(const uint8_t *Wd, const uint8_t *Sd,
                                  const float *hidden, const float *wts, float *y,
                                  const float *s2d_dev, const int *sel_ids,
                                  const int *slot_ids, int nexp, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* NVFP4 M=8 tier (ocho/amd_server/qf_moe_m8_wave64.h:51-70). x fp32 [M][H];
 * hidden [pairs][I]; s2*_res indexed by the resident slot; y_partial
 * [M][H] PRE-ZEROED by the caller, pairs accumulate with atomics. */
void qf5_m8_gateup(const uint8_t *Wg, const uint8_t *Sg,
                   const uint8_t *Wu, const uint8_t *Su,
                   const float *s2g_res, const float *s2u_res,
                   const float *x, float *hidden,
                   const Qf5M8Route *rt, hipStream_t stream);
void qf5_m8_downacc(const uint8_t *Wd, const uint8_t *Sd, const float *s2d_res,
                    const float *hidden, float *y_partial,
                    const Qf5M8Route *rt, hipStream_t stream);
/* Device routing inversion over the experts [card*epc, card*epc + epc):
 * exp_slot = il*epc + (e - card*epc), ascending; counts = {n_exp, n_pairs}.
 * M*K <= 1024. */
void qf5_m8_build_csr(const int *sel_dev, const float *wt_dev, int M, int K,
                      int card, int epc, int il, int *exp_slot, int *exp_ptr,
                      int *pair_tok, float *pair_wt, int *counts, hipStream_t s);
/* Four-card combine of fp32 partials already in this device's memory:
 * y_out[i] = ((y0[i] + y1[i]) + y2[i]) + y3[i], i < n (n = M*H). y_out may be
 * one of the inputs. Replaces qf5_m8_reduce4
 * (ocho/amd_server/qf_moe_m8_wave64.h:72-75; kernel k_m8_reduce4,
 * qf_moe_m8_wave64.hip:216-221). */
void qf5_m8_reduce4(float *y_out, const float *y0, const float *y1,
                    const float *y2, const float *y3, int n, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* INT8 shared expert on X8 rows: eg = silu(gate.x) * up.x, eu = up.x,
 * g1 = gate_inp.x (row 0), ed = down.eg, y2560 += sigmoid(g1) * ed.
 * e8q/e8s are accepted and unused (eg stays fp32).
 * Replace qf8_i8_shexp_m1 (ocho/amd_server/qf8_dense_i8.h:88-91) and the rows
 * form qf8_i8_shexp_rows (:41-43; returns 0 or a negative code). */
void qf8_i8_shexp_m1(const Qf8I8Mat *gate, const Qf8I8Mat *up, const Qf8I8Mat *gate_inp,
                     const Qf8I8Mat *down, const int8_t *xq, const float *xs,
                     float *eg, float *eu, float *g1, float *ed, int8_t *e8q, float *e8s,
                     float *y2560, hipStream_t s);
int qf8_i8_shexp_rows(const Qf8I8Mat *gate, const Qf8I8Mat *up, const Qf8I8Mat *gate_inp,
                      const Qf8I8Mat *down, const int8_t *xq, const float *xs, float *eg,
                      float *eu, float *g1, float *ed, int8_t *e8q, float *e8s, float *y2560,
                      int T, hipStream_t s);

/* ------------------------------------------------------------------------ */
/* Validated twins of the reference's void launchers (the error convention of
 * ocho/amd_server/qf8_moe_i8.h:34-37 extended to every launcher): the same
 * arguments and work, returning 0, -1 (a rejected argument: nothing was
 * launched), -2 (unsupported shape configuration) or -3 (launch failure). The
 * void forms call these and leave the code in the error latch. */
int qf_rtr_gemv_launch_ex(const uint16_t *router, const float *x, float *logits, hipStream_t s);
int qf_rtr_topk10_launch_ex(const float *logits, int *sel_ids, float *wts, hipStream_t s);
int qf_rtr_topk10_rows_launch_ex(const float *logits, int *sel_ids, float *wts, int T, hipStream_t s);
int qf8_i8_gateup_m1_ex(const Qf4ExpCache *c, const float *x, int8_t *x8q, float *x8s,
                        float *hidden, const int *sel_ids, int nexp, int quant_x, hipStream_t s);
int qf8_i8_down_m1_ex(const Qf4ExpCache *c, const float *hidden, int8_t *h8q, float *h8s,
                      const float *wts, const int *sel_ids, float *y, int nexp, hipStream_t s);
int qf8_i8_x8_ex(const float *x, int8_t *q, float *sc, int n, hipStream_t s);
int qf8_i8_csr_build_ex(const int *sel, const float *wt, int T, int *exp_slot, int *exp_ptr,
                        int *pair_tok, float *pair_wt, int *counts, hipStream_t s);
int qf8_i8_experts_chunk_ex(const Qf4ExpCache *c, const int8_t *xq, const float *xs,
                            float *hidden, int8_t *h8q, float *h8s,
                            const int *exp_slot, const int *exp_ptr, const int *pair_tok,
                            const float *pair_wt, const int *n_exp_dev, int n_exp_max,
                            int n_pairs_max, const int *sel, float *part, int T, float *y, hipStream_t s);
int qf5_nvfp4_moe_all_ex(const uint8_t *Wg, const uint8_t *Sg, const uint8_t *Wu, const uint8_t *Su,
                         const uint8_t *Wd, const uint8_t *Sd, const float *x, float *hidden, float *y,
                         const float *s2g_dev, const float *s2u_dev, const float *s2d_dev, const float *wts,
                         const int *sel_ids, const int *slot_ids, int nexp, hipStream_t stream);
int qf5_nvfp4_gateup_all_launch_ex(const uint8_t *Wg, const uint8_t *Sg, const uint8_t *Wu, const uint8_t *Su,
                                   const float *x, float *hidden, const float *s2g_dev, const float *s2u_dev,
                                   const int *sel_ids, const int *slot_ids, int nexp, hipStream_t stream);
int qf5_nvfp4_downacc_all_launch_ex(const uint8_t *Wd, const uint8_t *Sd, const float *hidden, const float *wts,
                                    float *y, const float *s2d_dev, const int *sel_ids, const int *slot_ids,
                                    int nexp, hipStream_t stream);
int qf5_m8_gateup_ex(const uint8_t *Wg, const uint8_t *Sg, const uint8_t *Wu, const uint8_t *Su,
                     const float *s2g_res, const float *s2u_res, const float *x, float *hidden,
                     const Qf5M8Route *rt, hipStream_t stream);
int qf5_m8_downacc_ex(const uint8_t *Wd, const uint8_t *Sd, const float *s2d_res, const float *hidden,
                      float *y_partial, const Qf5M8Route *rt, hipStream_t stream);
int qf5_m8_build_csr_ex(const int *sel_dev, const float *wt_dev, int M, int K, int card, int epc, int il,
                        int *exp_slot, int *exp_ptr, int *pair_tok, float *pair_wt, int *counts, hipStream_t s);
int qf5_m8_reduce4_ex(float *y_out, const float *y0, const float *y1, const float *y2, const float *y3,
                      int n, hipStream_t stream);
int qf8_i8_shexp_m1_ex(const Qf8I8Mat *gate, const Qf8I8Mat *up, const Qf8I8Mat *gate_inp,
                       const Qf8I8Mat *down, const int8_t *xq, const float *xs, float *eg, float *eu,
                       float *g1, float *ed, int8_t *e8q, float *e8s, float *y2560, hipStream_t s);

/* ------------------------------------------------------------------------ */
/* Fused MoE layer (this library's entry point for the whole path). */
enum { QFM_FMT_INT8 = 0, QFM_FMT_NVFP4 = 1 };
typedef struct {
    const Qf4ExpCache *arena;     /* routed experts, slot == expert */
    int                fmt;       /* QFM_FMT_INT8 or QFM_FMT_NVFP4 */
    const float       *router;    /* [E][H] fp32 */
    const float       *router_bias; /* [E] fp32 or NULL */
    Qf8I8Mat           sh_gate, sh_up, sh_down;  /* shared expert (INT8); sh_gate.w == NULL: none */
    const float       *sh_gate_inp;              /* [H] fp32 sigmoid-gate vector */
} qfm_layer;

/* Workspace for M rows (device memory, caller-owned, >= 256-byte aligned).
 * Zero it once after allocating it, ordered before the first call (on that
 * call's stream, or finished; qfm_dev_malloc returns zeroed memory):
 * its first bytes hold per-row sequence tags that the M <= 8 forward keeps
 * across calls (the same offsets for every M, so one workspace of the largest
 * size serves calls of any M); calls that share a workspace must not overlap. */
size_t qfm_workspace_bytes(int M);
/* For M > 8 (prefill) logits is [M][E] of the MFMA router GEMM (the exact
 * canonical logits are computed only for the selection candidates), hidden is
 * NULL and counters points at {tokens whose candidate set overflowed and had
 * every logit recomputed, gate/up work items, down work items} (int, device
 * memory; NULL for M <= 8). */
typedef struct {
    float *logits;   /* [M][E+1]: router logits; column E = <sh_gate_inp, x> */
    int   *sel;      /* [M][K] */
    float *wts;      /* [M][K] */
    float *hidden;   /* routed / shared intermediate activations */
    int   *counters; /* prefill: {n_fallback, n_items_gateup, n_items_down}; else NULL */
} qfm_ws_view;
int qfm_workspace_view(void *ws, int M, qfm_ws_view *v);

/* y[M][H] (bf16) = MoE(x[M][H] bf16). Stream-ordered, allocates nothing. */
int qfm_moe_forward(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y,
                    void *ws, size_t ws_bytes, hipStream_t s);

/* qfm_moe_forward with the engine's y contract: y[M][H] fp32, seeded (the
 * routed experts plus the gated shared expert, as qf8_i8_down_m1 seeds y2560
 * and qf8_i8_shexp_m1 adds to it, qf_hip4_stage.hip:1563-1571, :1626-1640),
 * ready for qf8_stream_inject. Same kernels and routing as qfm_moe_forward;
 * only the final store differs (fp32 instead of bf16). No counterpart in the
 * reference (its whole layer is a sequence of the launchers above). */
int qfm_moe_forward_f32(const qfm_layer *L, const uint16_t *x, int M, float *y,
                        void *ws, size_t ws_bytes, hipStream_t s);

/* qfm_moe_forward for callers that cannot allocate or pass a workspace (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. The workspace is a 3 MiB
 * device array inside the library (one per GPU, held until the process ends),
 * which serves 1 <= M <= 8 rows at either supported shape; larger M is
 * rejected with -1 and a message (prefill needs qfm_moe_forward and a caller
 * workspace). Allocates nothing, same kernels and results as qfm_moe_forward.
 * The array's address is resolved by qfm_init for the device current then, or
 * by the first call on another device: make that first call outside a stream
 * capture. Calls that overlap on one GPU (two streams or host threads) share
 * the array and race: serialize them. */
int qfm_moe_forward_noalloc(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y, hipStream_t s);

/* Profiling form of the M=1 forward: launches only the sections in mask
 * (bit 0 router + shared gate/up, bit 1 top-K + routed gate/up, bit 2 down +
 * combine), reading the workspace the earlier sections left behind. */
int qfm_moe_forward_sections(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y,
                             void *ws, size_t ws_bytes, int mask, hipStream_t s);

/* nl layers back to back on one stream: layer l reads x + l*x_stride and
 * writes y + l*y_stride (elements); layer l+1 starts after layer l ends. */
int qfm_moe_forward_layers(const qfm_layer *layers, int nl, const uint16_t *x, long x_stride, int M,
                           uint16_t *y, long y_stride, void *ws, size_t ws_bytes, hipStream_t s);

/* Section profiler: while enabled, every M=1 qfm_moe_forward records
 * hipEvents between its launches (also inside a stream capture, where they
 * become event-record nodes that fire on every replay). read() waits for the
 * last mark and returns the summed milliseconds of section 0 (router + shared
 * gate/up), 1 (routed gate/up with the top-K selection) and 2 (down +
 * combine) over the recorded forwards, and their number; enable() (on or
 * off) clears the marks. */
int qfm_profile_enable(int on);
int qfm_profile_read(double *ms, int n_sections, int *calls);

/* HIP graph capture of whatever is enqueued on a stream between begin and
 * end (used to replay a whole decode step without host launch cost). */
int   qfm_graph_capture_begin(void *stream);
void *qfm_graph_capture_end(void *stream);   /* returns an executable graph or NULL */
int   qfm_graph_launch(void *graph_exec, void *stream);
int   qfm_graph_destroy(void *graph_exec);

/* ------------------------------------------------------------------------ */
/* Synthetic data generator (Philox-4x32-10, counter = (lo32(j/4), hi32(j/4),
 * tensor, layer), key = (seed, 0)); writes cnt elements n0..n0+cnt-1. */
enum {
    QFM_GEN_I8 = 0,          /* int8 uniform over [-127, 127]                  */
    QFM_GEN_ROWSCALE = 1,    /* fp32 (0.5 + u) * 0.02/127                       */
    QFM_GEN_GAUSS_F32 = 2,   /* fp32 Irwin-Hall(12) * scale                      */
    QFM_GEN_GAUSS_BF16 = 3,  /* bf16 Irwin-Hall(12)                              */
    QFM_GEN_FP4BYTE = 4,     /* packed byte of two uniform e2m1 codes           */
    QFM_GEN_E4M3SCALE = 5    /* e4m3 nearest to 0.25 + 1.75 u                    */
};
int qfm_gen_fill(void *out, int kind, uint64_t n0, uint64_t cnt, uint32_t seed,
                 uint32_t layer, uint32_t tensor, float scale, hipStream_t s);
int qfm_fill_f32(float *out, uint64_t cnt, float value, hipStream_t s);

/* Resident arenas (slot == expert for all n_experts slots; the reference's
 * full-residency layout, ocho/amd_server/qf_expert_slots.cpp:332-365).
 * qfm_arena_init allocates the INT8 (i8_*) or NVFP4 (w_*, s_*, s2*_dev)
 * blobs; qfm_arena_generate fills whatever is allocated from the generator. */
int  qfm_arena_init(Qf4ExpCache *c, int fmt, int layer);
/* Device bytes qfm_arena_init allocates for fmt at the current shape (0 for an unknown fmt). */
size_t qfm_arena_bytes(int fmt);
int  qfm_arena_generate(Qf4ExpCache *c, uint32_t seed, uint32_t layer, hipStream_t s);
void qfm_arena_free(Qf4ExpCache *c);
/* A complete synthetic layer: arena + fp32 router (+ optional skew bias) +
 * INT8 shared expert + sigmoid-gate vector, all generated on device.
 * layer.arena points at the arena member: do not move the struct. */
typedef struct {
    qfm_layer   layer;
    Qf4ExpCache arena;
} qfm_synth_layer;
int  qfm_synth_layer_create(qfm_synth_layer *out, int fmt, uint32_t seed, uint32_t layer, int with_bias, hipStream_t s);
void qfm_synth_layer_destroy(qfm_synth_layer *l);
/* x[M][H] bf16 = generator rows row0..row0+M-1 of input stream x_layer. */
int  qfm_gen_input_rows(uint16_t *x, int M, uint32_t seed, uint32_t x_layer, int row0, hipStream_t s);

/* ------------------------------------------------------------------------ */
/* Harness utilities (thin wrappers over the HIP runtime). */
void  *qfm_dev_malloc(size_t bytes);   /* zeroed (the fill has finished at return) */
int    qfm_dev_free(void *p);
int    qfm_memcpy_h2d(void *dst, const void *src, size_t bytes);
int    qfm_memcpy_d2h(void *dst, const void *src, size_t bytes);
int    qfm_memcpy_d2d(void *dst, const void *src, size_t bytes);   /* device copy (runtime blit kernel) */
int    qfm_memset(void *dst, int value, size_t bytes);
void  *qfm_stream_create(void);
int    qfm_stream_destroy(void *s);
int    qfm_stream_sync(void *s);
int    qfm_device_sync(void);
void  *qfm_event_create(void);
int    qfm_event_destroy(void *e);
int    qfm_event_record(void *e, void *s);
float  qfm_event_elapsed_ms(void *e0, void *e1);
int    qfm_device_info(char *name, int name_len, int *n_cu, size_t *mem_bytes, int *arch_major, int *arch_minor);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
