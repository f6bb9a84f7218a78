// qfm_internal.h -- host-side internals shared by the translation units.
#pragma once
#include "../../include/qf_moe.h"
#include <hip/hip_runtime.h>

namespace qfm {

// Active shape configuration (set by qfm_init; defaults to H=2048, I=512, E=512, K=10).
struct Cfg {
    int H = 2048, I = 512, E = 512, K = 10, renorm = 1, gated = 1;
};
extern Cfg g_cfg;

// Error latch: the first error since the last read is kept.
void set_error(int code, const char *fmt, ...);
int  check_launch(const char *what);   // polls hipGetLastError after a launch

// Memory preflight (the reference's budget guard, qf_hip4_stage.hip:792-813):
// 0 when `bytes` more device memory fit both the device's free memory and the
// budget (qfm_set_hbm_budget / QFM_HBM_BUDGET_MIB) on the memory already in
// use; otherwise -4 latched with `who` and the figures. Allocates nothing.
int preflight_device_bytes(size_t bytes, const char *who);

// shape dispatch helpers
inline bool shape_2048() { return g_cfg.H == 2048 && g_cfg.I == 512; }
inline bool shape_2560() { return g_cfg.H == 2560 && g_cfg.I == 640; }
// one GPU's share of the 8-way split of every expert's intermediate dimension
// (2048, 512 / 8): only the M = 1 INT8 forward, the router and top-K run at it
inline bool shape_shard() { return g_cfg.H == 2048 && g_cfg.I == 64; }

// ---- launchers (defined in the .hip files) ----------------------------------
// generator
int launch_gen_fill(void *out, int kind, uint64_t n0, uint64_t cnt, uint32_t seed,
                    uint32_t layer, uint32_t tensor, float scale, hipStream_t s);
int launch_fill_f32(float *out, uint64_t cnt, float value, hipStream_t s);

// Shared-expert (or any single INT8 expert) pointers, passed by value to kernels.
struct ShPtrs { const int8_t *qg, *qu, *qd; const float *sg, *su, *sd; };

// router: W_f32 [E][H] (+ row g [H] written at column E when g != nullptr)
// and, when sh != nullptr, the shared-expert hidden hsh[m * ld_hsh + r], in one launch.
// With x16 != nullptr (M = 1) the launch also writes x as scaled fp16 (H / 8
// 16-byte words) followed by a float2 (sum of the scaled values, 2^-k).
// With tail != nullptr (1 <= M <= kTailRows, E = 512, no x16) the launch also
// ranks every row (k_router_shared's selection tail): sel/wts [M][K], and for
// INT8 fork rows x as scaled fp16 chunks (xh [M][H] fp16, xci [M][H/16]).
// lw: [M][E] 64-bit words; ctl: kTailRows + 1 words (per-row tags, then the
// count of bounded waits that ran out).
constexpr int kTailRows = 8;
constexpr int kTailSpinMax = 1 << 16;
// The tag after c: c + 1, skipping 0 (zeroed words never carry a live tag).
__host__ __device__ constexpr uint32_t next_tag(uint32_t c) { return c + 1u ? c + 1u : 1u; }
struct RouteTail {
    unsigned long long *lw;
    uint32_t *ctl;
    int *sel;
    float *wts;
    uint4 *xh;
    float2 *xci;
    int K, renorm;
};
int launch_router_shared(const float *W, const float *bias, const float *g, const ShPtrs *sh,
                         const uint16_t *x, int M, float *logits, int ld_logits, float *hsh, int ld_hsh,
                         hipStream_t s, void *x16 = nullptr, const RouteTail *tail = nullptr);
int launch_router_bf16w(const uint16_t *W, const float *x, float *logits, hipStream_t s);
int launch_topk(const float *logits, int ld_logits, int M, int *sel, float *wts, hipStream_t s);

// INT8 M=1 routed gate/up: hidden[k][I] for the nexp experts sel[0..nexp).
// With logits != nullptr the selection is made inside the kernel (every block
// runs the top-K of its row of logits) and block 0 writes sel/wts; otherwise
// sel is an input. x is bf16 (xb) or fp32 (xf). With sh != nullptr the shared
// expert's hidden vector is computed too, into hidden row nexp.
// With x16 != nullptr (launch_router_shared's fp16 row) x is read from there
// and the codes are widened to fp16 (dot16_i8h); xb/xf are then unused.
// With x8q/x8s != nullptr (X8 rows: int8 codes, one fp32 scale per 32 values)
// x is read from there, dequantized in registers (value = code * scale).
int launch_i8_gateup_m1(const Qf4ExpCache *c, const uint16_t *xb, const float *xf, const float *logits,
                        int *sel, float *wts, int nexp, float *hidden, hipStream_t s, const ShPtrs *sh = nullptr,
                        const void *x16 = nullptr, const int8_t *x8q = nullptr, const float *x8s = nullptr);
// X8 quantizer (qf8_i8_x8): n a positive multiple of 32
int launch_x8(const float *x, int8_t *q, float *sc, int n, hipStream_t s);
// y = sum_k wts[k] * down_k(hidden[k]) (+ gamma * shared_down(hidden[nexp]) when
// sh != nullptr: the shared expert's hidden vector follows the routed ones),
// gamma = sigmoid(*gdot) when gdot != nullptr, 1 otherwise. Writes y32 and/or ybf.
int launch_i8_down_m1(const Qf4ExpCache *c, const float *hidden, const float *wts, const int *sel,
                      int nexp, const ShPtrs *sh, const float *gdot, float *y32, uint16_t *ybf, hipStream_t s);

// Multi-row decode (1 <= M <= 8), after launch_router_shared with its selection
// tail (sel/wts [M][K], INT8: the fp16 activation chunks in xh16): gate/up
// keyed by pair (k_csr_gateup: the first pair of each distinct expert reads
// the expert's rows once for all its pairs; hidden row = pair id), down
// partials per (pair, row block) (k_csr_down), whose last M grid rows sum each
// output's partials (the combine) and whose first grid rows are the shared
// expert's down rows. Partials travel as 64-bit words (fp32 bits | tag << 32,
// agent-scope stores) in pw [kTailRows][K+1][H], tag = ctl[0] as the selection
// tail left it (row 0's tag): one tag per call, larger than any tag a word left
// by an earlier call carries. fmt: QFM_FMT_INT8 or QFM_FMT_NVFP4 for the routed
// experts. hsh: shared hidden [M][I] (from launch_router_shared); hpair:
// [M*K][I] fp32; xh16 (INT8): M*H*2 + M*(H/16)*8 bytes, 16-byte aligned; pdsc:
// M*K 16-byte pair descriptors (NVFP4: written by the gate/up launch, read by
// the down launch).
int launch_csr_forward(const Qf4ExpCache *a, int fmt, const ShPtrs *sh, const uint16_t *x, const float *logits,
                       int ld, int gated, int M, float *hpair, const float *hsh, const int *sel, const float *wts,
                       int4 *pdsc, void *xh16, unsigned long long *pw, uint32_t *ctl, uint16_t *y, float *y32,
                       hipStream_t s);

// The fused forward on a caller-vouched workspace, without the section
// profiler (qfm_moe_forward minus its event marks): the no-allocation entry.
int forward_on_workspace(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y, void *ws, size_t ws_bytes,
                         hipStream_t s);

// Resolve the no-allocation entry's device array for the current device (qfm_init).
void noalloc_prepare_current_device();
// Resolve the one-launch pre-mixer's hand-off area for the current device (qfm_init).
void hc_prepare_current_device();

// Prefill (T > 8 rows): MFMA router + exact candidate selection, grouped
// MFMA gate/up and down over the routing inversion, owned-partial combine.
size_t prefill_ws_bytes(int T);
// y[t] = sum of the S owned partial slots part[t*S + k][H] in slot order (bf16 out,
// or fp32 into y32 when y32 != nullptr)
// ctr: {candidate overflows (tokens whose logits were all recomputed), gate/up items, down items}
void prefill_ws_view(void *ws, int T, float **lg_approx, int **sel, float **wts, int **ctr);
// y32 != nullptr: y is written as fp32 there instead of bf16 into y
int launch_prefill(const qfm_layer *L, const uint16_t *x, int T, uint16_t *y, float *y32, void *ws, int gated,
                   hipStream_t s);

}  // namespace qfm
