// qfm_api.cpp -- extern "C" boundary: configuration, error latch, the
// reference-named launchers, the fused per-layer forward and the harness
// utilities. Host code only; every kernel lives in the .hip files.
#include "qfm_internal.h"
#include "../../include/qf_store.h"

#include <array>
#include <cstdarg>
#include <vector>
#include <cstdio>
#include <cstddef>
#include <cstdlib>
#include <cstring>

namespace qfm {

Cfg g_cfg;

static thread_local int t_err_code = 0;
static thread_local char t_err_msg[512] = {0};

void set_error(int code, const char *fmt, ...) {
    if (t_err_code) return;   // keep the first error until it is read
    t_err_code = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err_msg, sizeof t_err_msg, fmt, ap);
    va_end(ap);
}

int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(-100 - (int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
        return -3;
    }
    return 0;
}

// The arena struct must stay byte-compatible with the reference's Qf4ExpCache
// (ocho/amd_server/qf_nvfp4_wave64.h:133-173) on LP64.
static_assert(offsetof(Qf4ExpCache, w_gate) == 8, "Qf4ExpCache layout");
static_assert(offsetof(Qf4ExpCache, i8_gate) == 80, "Qf4ExpCache layout");
static_assert(offsetof(Qf4ExpCache, nv_ring) == 128, "Qf4ExpCache layout");
static_assert(offsetof(Qf4ExpCache, s_gate) == 136, "Qf4ExpCache layout");
static_assert(offsetof(Qf4ExpCache, clock) == 184, "Qf4ExpCache layout");
static_assert(offsetof(Qf4ExpCache, fully_resident) == 216, "Qf4ExpCache layout");
static_assert(offsetof(Qf4ExpCache, s2g_dev) == 256, "Qf4ExpCache layout");
static_assert(offsetof(Qf4ExpCache, mb_dev) == 296, "Qf4ExpCache layout");
static_assert(sizeof(Qf4ExpCache) == 312, "Qf4ExpCache layout");
static_assert(sizeof(Qf8I8Mat) == 24, "Qf8I8Mat layout");
static_assert(sizeof(Qf5M8Route) == 56, "Qf5M8Route layout");

// ---- section profiler: hipEvent marks between the launches of a forward
// (eager launches only; the reference's QF8_PROFILE section marks play the
// same role). Sections: 0 router + shared gate/up, 1 routed gate/up (with the
// selection), 2 down + combine. Not thread-safe; one profiling stream.
struct Prof {
    bool on = false;
    std::vector<hipEvent_t> pool;
    size_t used = 0;
    std::vector<std::array<size_t, 4>> marks;   // event indices per forward
};
static Prof g_prof;
static size_t prof_event(hipStream_t s) {
    if (g_prof.used == g_prof.pool.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return (size_t)-1;
        g_prof.pool.push_back(e);
    }
    const size_t i = g_prof.used++;
    (void)hipEventRecord(g_prof.pool[i], s);
    return i;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// ---- memory preflight ------------------------------------------------------
static size_t g_hbm_budget = 0;        // bytes; 0: the device's own memory
static bool g_hbm_budget_set = false;  // set by qfm_set_hbm_budget (else QFM_HBM_BUDGET_MIB)
static size_t hbm_budget() {
    if (!g_hbm_budget_set) {
        const char *v = std::getenv("QFM_HBM_BUDGET_MIB");
        g_hbm_budget = v ? (size_t)std::strtoull(v, nullptr, 10) << 20 : 0;
        g_hbm_budget_set = true;
    }
    return g_hbm_budget;
}
int preflight_device_bytes(size_t bytes, const char *who) {
    size_t fr = 0, tot = 0;
    if (hipMemGetInfo(&fr, &tot) != hipSuccess) { set_error(-5, "%s: hipMemGetInfo failed", who); return -5; }
    const size_t budget = hbm_budget(), used = tot - fr;
    if (bytes > fr) {
        set_error(-4, "%s: needs %zu device bytes, %zu free (nothing allocated)", who, bytes, fr);
        return -4;
    }
    if (budget && used + bytes > budget) {
        set_error(-4, "%s: needs %zu device bytes; %zu in use, budget %zu (nothing allocated)", who, bytes, used,
                  budget);
        return -4;
    }
    return 0;
}

// Every workspace starts with the M <= 8 forward's tagged state, at the same
// offsets for every M (prefill included, whose own layout follows it): ctl =
// per-row tags (+ the count of bounded waits that ran out), lw =
// [kTailRows][E] tagged logit words (the router launch's selection tail), pw =
// [kTailRows][K+1][H] tagged partial words (the down launch's combine row).
// Zero is a valid start (the first tag is 1, and no zero word carries it);
// every later tag is larger than any tag a word already holds, so a workspace
// that is zeroed once stays valid across calls of any M.
static size_t ws_lw_bytes() { return align256((size_t)kTailRows * g_cfg.E * 8); }
static size_t ws_tag_bytes() {
    return 256 + ws_lw_bytes() + align256((size_t)kTailRows * (g_cfg.K + 1) * g_cfg.H * 8);
}

struct WsLayout {
    size_t ctl, lw, pw, logits, sel, wts, hidden, pdsc, xh16, total;
};
static WsLayout ws_layout(int M) {
    const Cfg &c = g_cfg;
    WsLayout w{};
    w.ctl = 0;
    w.lw = 256;
    w.pw = 256 + ws_lw_bytes();
    size_t off = ws_tag_bytes();
    w.logits = off; off += align256((size_t)M * (c.E + 1) * sizeof(float));
    w.sel = off;    off += align256((size_t)M * c.K * sizeof(int));
    w.wts = off;    off += align256((size_t)M * c.K * sizeof(float));
    w.hidden = off; off += align256((size_t)M * (c.K + 1) * c.I * sizeof(float));
    w.pdsc = off;   off += align256((size_t)M * c.K * 16);                      // per-pair descriptors (NVFP4)
    w.xh16 = off;   off += align256((size_t)M * c.H * 2 + (size_t)M * (c.H / 16) * 8);   // fp16 activations + chunk scales
    w.total = off;
    return w;
}

static bool layer_ok(const qfm_layer *L) {
    if (!L || !L->arena || !L->router) return false;
    const Qf4ExpCache *a = L->arena;
    // the fused forward addresses expert e at slot e: every expert resident
    if (a->slots < g_cfg.E || !a->fully_resident) {
        set_error(-1, "qfm_moe_forward: the arena must be fully resident (slots %d of %d, fully_resident %d)", a->slots,
                  g_cfg.E, a->fully_resident);
        return false;
    }
    if (L->fmt == QFM_FMT_INT8) {
        if (!a->i8_gate || !a->i8_up || !a->i8_down || !a->i8s_gate || !a->i8s_up || !a->i8s_down) return false;
    } else if (L->fmt == QFM_FMT_NVFP4) {
        if (!a->w_gate || !a->w_up || !a->w_down || !a->s_gate || !a->s_up || !a->s_down || !a->s2g_dev ||
            !a->s2u_dev || !a->s2d_dev || a->nv_ring)   // a staging ring holds only nv_ring NVFP4 slots
            return false;
    } else {
        return false;
    }
    if (L->sh_gate.w) {
        if (!L->sh_up.w || !L->sh_down.w || !L->sh_gate.s || !L->sh_up.s || !L->sh_down.s) return false;
        if (L->sh_gate.rows != g_cfg.I || L->sh_gate.K != g_cfg.H || L->sh_up.rows != g_cfg.I ||
            L->sh_up.K != g_cfg.H || L->sh_down.rows != g_cfg.H || L->sh_down.K != g_cfg.I)
            return false;
    }
    return true;
}

}  // namespace qfm

using namespace qfm;

extern "C" {

int qfm_init(const qfm_config *cfg) {
    if (!cfg) { set_error(-1, "qfm_init: null config"); return -1; }
    const bool shape = (cfg->hidden == 2048 && cfg->inter == 512) || (cfg->hidden == 2560 && cfg->inter == 640) ||
                       (cfg->hidden == 2048 && cfg->inter == 64);   // the tensor-parallel shard
    const int E = cfg->n_experts;
    const bool e_ok = E == 512;   // the reference's expert count; every path is built for it
    if (!shape || !e_ok || cfg->top_k < 1 || cfg->top_k > 16 || cfg->top_k > E) {
        set_error(-1, "qfm_init: unsupported configuration H=%d I=%d E=%d K=%d", cfg->hidden, cfg->inter, E, cfg->top_k);
        return -1;
    }
    g_cfg.H = cfg->hidden; g_cfg.I = cfg->inter; g_cfg.E = E; g_cfg.K = cfg->top_k;
    g_cfg.renorm = cfg->renorm ? 1 : 0; g_cfg.gated = cfg->shared_gated ? 1 : 0;
    noalloc_prepare_current_device();
    hc_prepare_current_device();
    return 0;
}

int qfm_get_config(qfm_config *cfg) {
    if (!cfg) return -1;
    cfg->hidden = g_cfg.H; cfg->inter = g_cfg.I; cfg->n_experts = g_cfg.E; cfg->top_k = g_cfg.K;
    cfg->renorm = g_cfg.renorm; cfg->shared_gated = g_cfg.gated;
    return 0;
}

const char *qfm_last_error(void) {
    static thread_local char out[512];
    std::strncpy(out, t_err_msg, sizeof out - 1);
    out[sizeof out - 1] = 0;
    t_err_code = 0; t_err_msg[0] = 0;
    return out;
}

int qfm_status(void) {
    check_launch("qfm_status");
    return t_err_code;
}

const char *qfm_version(void) { return "qfm 0.1 gfx950"; }

int qfm_set_hbm_budget(size_t bytes) {
    g_hbm_budget = bytes;
    g_hbm_budget_set = true;
    return 0;
}
size_t qfm_get_hbm_budget(void) { return hbm_budget(); }

size_t qfm_sizeof(int which) {
    switch (which) {
    case 0: return sizeof(Qf4ExpCache);
    case 1: return sizeof(qfm_layer);
    case 2: return sizeof(qfm_synth_layer);
    case 3: return sizeof(Qf8I8Mat);
    case 4: return sizeof(Qf5M8Route);
    case 5: return sizeof(qfm_config);
    case 6: return sizeof(qfm_ws_view);
    case 7: return sizeof(QfEntry);
    case 8: return sizeof(QfStore);
    case 9: return sizeof(Qf4ExpXfer);
    case 10: return sizeof(QfRouteMailbox);
    default: return 0;
    }
}

// ---- router ----------------------------------------------------------------
// Every reference-named void launcher has an _ex twin returning 0 or a
// negative code (-1 rejected argument, -2 unsupported shape, -3 launch
// failure); the void form calls it and leaves the code in the error latch.
int qf_rtr_gemv_launch_ex(const uint16_t *router, const float *x, float *logits, hipStream_t s) {
    if (!router || !x || !logits) { set_error(-1, "qf_rtr_gemv_launch: null pointer"); return -1; }
    return launch_router_bf16w(router, x, logits, s);
}
void qf_rtr_gemv_launch(const uint16_t *router, const float *x, float *logits, hipStream_t s) {
    (void)qf_rtr_gemv_launch_ex(router, x, logits, s);
}
int qf_rtr_topk10_launch_ex(const float *logits, int *sel_ids, float *wts, hipStream_t s) {
    if (!logits || !sel_ids || !wts) { set_error(-1, "qf_rtr_topk10_launch: null pointer"); return -1; }
    return launch_topk(logits, g_cfg.E, 1, sel_ids, wts, s);
}
void qf_rtr_topk10_launch(const float *logits, int *sel_ids, float *wts, hipStream_t s) {
    (void)qf_rtr_topk10_launch_ex(logits, sel_ids, wts, s);
}
int qf_rtr_topk10_rows_launch_ex(const float *logits, int *sel_ids, float *wts, int T, hipStream_t s) {
    if (!logits || !sel_ids || !wts || T < 1) { set_error(-1, "qf_rtr_topk10_rows_launch: bad arguments"); return -1; }
    return launch_topk(logits, g_cfg.E, T, sel_ids, wts, s);
}
void qf_rtr_topk10_rows_launch(const float *logits, int *sel_ids, float *wts, int T, hipStream_t s) {
    (void)qf_rtr_topk10_rows_launch_ex(logits, sel_ids, wts, T, s);
}
int qfm_router_logits(const float *W, const float *bias, const uint16_t *x, int M, float *logits, hipStream_t s) {
    if (!W || !x || !logits || M < 1) { set_error(-1, "qfm_router_logits: bad arguments"); return -1; }
    return launch_router_shared(W, bias, nullptr, nullptr, x, M, logits, g_cfg.E, nullptr, 0, s);
}
int qfm_topk(const float *logits, int M, int *sel, float *wts, hipStream_t s) {
    if (!logits || !sel || !wts || M < 1) { set_error(-1, "qfm_topk: bad arguments"); return -1; }
    return launch_topk(logits, g_cfg.E, M, sel, wts, s);
}

// ---- INT8 M=1 (reference signatures) ------------------------------------------
// gate/up reads its activations as X8 rows (x8q: H int8 codes, x8s: H/32 fp32
// scales), as the reference does (qf8_moe_i8.hip:416-421): quant_x != 0
// quantizes x into them first, quant_x == 0 uses what the caller left there
// (x is not read and may be null).
int qf8_i8_gateup_m1_ex(const Qf4ExpCache *c, const float *x, int8_t *x8q, float *x8s, float *hidden,
                        const int *sel_ids, int nexp, int quant_x, hipStream_t s) {
    if (!x8q || !x8s || (quant_x && !x)) {
        set_error(-1, "qf8_i8_gateup_m1: needs x8q/x8s (and x when quant_x)"); return -1;
    }
    if (quant_x) {
        const int rc = launch_x8(x, x8q, x8s, g_cfg.H, s);
        if (rc) return rc;
    }
    return launch_i8_gateup_m1(c, nullptr, nullptr, nullptr, const_cast<int *>(sel_ids), nullptr, nexp, hidden, s,
                               nullptr, nullptr, x8q, x8s);
}
void qf8_i8_gateup_m1(const Qf4ExpCache *c, const float *x, int8_t *x8q, float *x8s, float *hidden,
                      const int *sel_ids, int nexp, int quant_x, hipStream_t s) {
    (void)qf8_i8_gateup_m1_ex(c, x, x8q, x8s, hidden, sel_ids, nexp, quant_x, s);
}
int qf8_i8_down_m1_ex(const Qf4ExpCache *c, const float *hidden, int8_t *h8q, float *h8s, const float *wts,
                      const int *sel_ids, float *y, int nexp, hipStream_t s) {
    (void)h8q; (void)h8s;
    return launch_i8_down_m1(c, hidden, wts, sel_ids, nexp, nullptr, nullptr, y, nullptr, s);
}
void qf8_i8_down_m1(const Qf4ExpCache *c, const float *hidden, int8_t *h8q, float *h8s, const float *wts,
                    const int *sel_ids, float *y, int nexp, hipStream_t s) {
    (void)qf8_i8_down_m1_ex(c, hidden, h8q, h8s, wts, sel_ids, y, nexp, s);
}

// ---- fused layer ---------------------------------------------------------------
size_t qfm_workspace_bytes(int M) {
    if (M < 1) return 0;
    return M <= 8 ? ws_layout(M).total : ws_tag_bytes() + prefill_ws_bytes(M);
}

int qfm_workspace_view(void *ws, int M, qfm_ws_view *v) {
    if (!ws || !v || M < 1) return -1;
    if (M > 8) {
        prefill_ws_view(static_cast<char *>(ws) + ws_tag_bytes(), M, &v->logits, &v->sel, &v->wts, &v->counters);
        v->hidden = nullptr;
        return 0;
    }
    const WsLayout w = ws_layout(M);
    char *b = static_cast<char *>(ws);
    v->logits = reinterpret_cast<float *>(b + w.logits);
    v->sel = reinterpret_cast<int *>(b + w.sel);
    v->wts = reinterpret_cast<float *>(b + w.wts);
    v->hidden = reinterpret_cast<float *>(b + w.hidden);
    v->counters = nullptr;
    return 0;
}

static int forward_impl(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y, float *y32, void *ws,
                        size_t ws_bytes, int mask, hipStream_t s, bool prof = true);


int qfm_moe_forward(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y, void *ws, size_t ws_bytes,
                    hipStream_t s) {
    if (!y) { set_error(-1, "qfm_moe_forward: bad arguments (null y)"); return -1; }
    return forward_impl(L, x, M, y, nullptr, ws, ws_bytes, 7, s);
}

int qfm_moe_forward_f32(const qfm_layer *L, const uint16_t *x, int M, float *y, void *ws, size_t ws_bytes,
                        hipStream_t s) {
    if (!y) { set_error(-1, "qfm_moe_forward_f32: bad arguments (null y)"); return -1; }
    return forward_impl(L, x, M, nullptr, y, ws, ws_bytes, 7, s);
}

int qfm_moe_forward_sections(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y, void *ws, size_t ws_bytes,
                             int mask, hipStream_t s) {
    if (M != 1 || mask < 1 || mask > 7) { set_error(-1, "qfm_moe_forward_sections: M=1 and mask 1..7 only"); return -1; }
    if (!y) { set_error(-1, "qfm_moe_forward_sections: bad arguments (null y)"); return -1; }
    return forward_impl(L, x, M, y, nullptr, ws, ws_bytes, mask, s);
}

static int forward_impl(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y, float *y32, void *ws,
                        size_t ws_bytes, int mask, hipStream_t s, bool prof) {
    if (!layer_ok(L) || !x || (!y && !y32) || !ws || M < 1) { set_error(-1, "qfm_moe_forward: bad arguments"); return -1; }
    if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) { set_error(-1, "qfm_moe_forward: workspace not 256-byte aligned"); return -1; }
    if (ws_bytes < qfm_workspace_bytes(M)) {
        set_error(-1, "qfm_moe_forward: workspace too small (%zu < %zu)", ws_bytes, qfm_workspace_bytes(M)); return -1;
    }
    // a gated shared expert needs its gate vector on every path (prefill included)
    if (L->sh_gate.w && g_cfg.gated && !L->sh_gate_inp) {
        set_error(-1, "qfm_moe_forward: gated shared expert needs sh_gate_inp"); return -1;
    }
    if (M > 8) return launch_prefill(L, x, M, y, y32, static_cast<char *>(ws) + ws_tag_bytes(), g_cfg.gated, s);
    const WsLayout w = ws_layout(M);
    const Cfg &c = g_cfg;
    char *b = static_cast<char *>(ws);
    float *logits = reinterpret_cast<float *>(b + w.logits);
    int *sel = reinterpret_cast<int *>(b + w.sel);
    float *wts = reinterpret_cast<float *>(b + w.wts);
    float *hidden = reinterpret_cast<float *>(b + w.hidden);
    const bool has_sh = L->sh_gate.w != nullptr;
    const float *g = (has_sh && c.gated) ? L->sh_gate_inp : nullptr;
    ShPtrs shp{};
    if (has_sh) {
        shp.qg = L->sh_gate.w; shp.qu = L->sh_up.w; shp.qd = L->sh_down.w;
        shp.sg = L->sh_gate.s; shp.su = L->sh_up.s; shp.sd = L->sh_down.s;
    }
    const ShPtrs *sp = has_sh ? &shp : nullptr;
    const int ld = c.E + 1;
    std::array<size_t, 4> pm{};
    const bool marks = prof && g_prof.on;
    if (marks) pm[0] = prof_event(s);
    if (M == 1 && L->fmt == QFM_FMT_INT8 && c.E == 512) {
        // per row: K routed hidden vectors, then the shared one (read as one block by the down kernel)
        float *hsh = hidden + (size_t)c.K * c.I;
        // 1. router logits (+ shared gate dot): depend on x only
        int rc = 0;
        void *x16 = b + w.xh16;                    // x as scaled fp16 + (sum, 2^-k), written by the router launch
        if (mask & 1) rc = launch_router_shared(L->router, L->router_bias, g, nullptr, x, 1, logits, ld, hsh, c.I, s, x16);
        if (marks) pm[1] = prof_event(s);
        // 2. top-K inside the gate/up kernel, whose last grid row computes the shared
        // expert's hidden (no selection needed there); 3. down + combine (+ shared) -> y bf16
        if (!rc && (mask & 2)) rc = launch_i8_gateup_m1(L->arena, x, nullptr, logits, sel, wts, c.K, hidden, s, sp, x16);
        if (marks) pm[2] = prof_event(s);
        if (!rc && (mask & 4))
            rc = launch_i8_down_m1(L->arena, hidden, wts, sel, c.K, sp, g ? logits + c.E : nullptr, y32, y, s);
        if (marks) { pm[3] = prof_event(s); g_prof.marks.push_back(pm); }
        return rc;
    }
    if (M <= 8) {
        float *hsh = hidden + (size_t)M * c.K * c.I;
        // the router launch also ranks every row (its selection tail) and, for
        // INT8, writes the rows as fp16 chunks for the fork-row dots
        RouteTail tail{};
        tail.lw = reinterpret_cast<unsigned long long *>(b + w.lw);
        tail.ctl = reinterpret_cast<uint32_t *>(b + w.ctl);
        tail.sel = sel;
        tail.wts = wts;
        if (L->fmt == QFM_FMT_INT8) {
            tail.xh = reinterpret_cast<uint4 *>(b + w.xh16);
            tail.xci = reinterpret_cast<float2 *>(tail.xh + (size_t)M * c.H / 8);
        }
        tail.K = c.K;
        tail.renorm = c.renorm;
        int rc = launch_router_shared(L->router, L->router_bias, g, sp, x, M, logits, ld, hsh, c.I, s, nullptr, &tail);
        if (!rc) rc = launch_csr_forward(L->arena, L->fmt, sp, x, logits, ld, g ? 1 : 0, M, hidden, hsh, sel, wts,
                                         reinterpret_cast<int4 *>(b + w.pdsc), b + w.xh16,
                                         reinterpret_cast<unsigned long long *>(b + w.pw),
                                         reinterpret_cast<uint32_t *>(b + w.ctl), y, y32, s);
        return rc;
    }
    return launch_prefill(L, x, M, y, y32, b + ws_tag_bytes(), c.gated, s);
}

int qfm_moe_forward_layers(const qfm_layer *layers, int nl, const uint16_t *x, long x_stride, int M, uint16_t *y,
                           long y_stride, void *ws, size_t ws_bytes, hipStream_t s) {
    if (!layers || nl < 1 || x_stride < 0 || y_stride < 0) { set_error(-1, "qfm_moe_forward_layers: bad arguments"); return -1; }
    for (int l = 0; l < nl; l++) {
        const int rc = qfm_moe_forward(&layers[l], x + (size_t)l * x_stride, M, y + (size_t)l * y_stride, ws, ws_bytes, s);
        if (rc) return rc;
    }
    return 0;
}

int qfm_profile_enable(int on) {
    g_prof.on = on != 0;
    g_prof.used = 0;
    g_prof.marks.clear();
    return 0;
}

int qfm_profile_read(double *ms, int n, int *calls) {
    if (!ms || n < 1) return -1;
    for (int i = 0; i < n; i++) ms[i] = 0.0;
    if (calls) *calls = (int)g_prof.marks.size();
    if (g_prof.marks.empty()) return 0;
    if (hipEventSynchronize(g_prof.pool[g_prof.marks.back()[3]]) != hipSuccess) return -1;
    for (const auto &m : g_prof.marks)
        for (int i = 0; i < 3 && i < n; i++) {
            float t = 0.0f;
            if (hipEventElapsedTime(&t, g_prof.pool[m[i]], g_prof.pool[m[i + 1]]) != hipSuccess) return -1;
            ms[i] += t;
        }
    return 0;
}

// ---- graphs ----------------------------------------------------------------------
int qfm_graph_capture_begin(void *stream) {
    const hipError_t e = hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeGlobal);
    if (e != hipSuccess) { set_error(-5, "hipStreamBeginCapture: %s", hipGetErrorString(e)); return -5; }
    return 0;
}
void *qfm_graph_capture_end(void *stream) {
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g);
    if (e != hipSuccess || !g) { set_error(-5, "hipStreamEndCapture: %s", hipGetErrorString(e)); return nullptr; }
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) { set_error(-5, "hipGraphInstantiate: %s", hipGetErrorString(e)); return nullptr; }
    return x;
}
int qfm_graph_launch(void *graph_exec, void *stream) {
    const hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), static_cast<hipStream_t>(stream));
    if (e != hipSuccess) { set_error(-5, "hipGraphLaunch: %s", hipGetErrorString(e)); return -5; }
    return 0;
}
int qfm_graph_destroy(void *graph_exec) {
    return hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)) == hipSuccess ? 0 : -1;
}

// ---- generator -------------------------------------------------------------------
int qfm_gen_fill(void *out, int kind, uint64_t n0, uint64_t cnt, uint32_t seed, uint32_t layer, uint32_t tensor,
                 float scale, hipStream_t s) {
    return launch_gen_fill(out, kind, n0, cnt, seed, layer, tensor, scale, s);
}
int qfm_fill_f32(float *out, uint64_t cnt, float value, hipStream_t s) { return launch_fill_f32(out, cnt, value, s); }

// ---- harness utilities -------------------------------------------------------------
void *qfm_dev_malloc(size_t bytes) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) { set_error(-4, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e)); return nullptr; }
    // zeroed (a workspace must start zeroed), and finished before the return:
    // the fill runs on the null stream, which a non-blocking stream does not
    // wait for, so work the caller then queues there could run first
    e = hipMemsetAsync(p, 0, bytes ? bytes : 1, nullptr);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) { (void)hipFree(p); set_error(-4, "hipMemset(%zu): %s", bytes, hipGetErrorString(e)); return nullptr; }
    return p;
}
int qfm_dev_free(void *p) { return hipFree(p) == hipSuccess ? 0 : -1; }
int qfm_memcpy_h2d(void *dst, const void *src, size_t n) { return hipMemcpy(dst, src, n, hipMemcpyHostToDevice) == hipSuccess ? 0 : -1; }
int qfm_memcpy_d2h(void *dst, const void *src, size_t n) { return hipMemcpy(dst, src, n, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1; }
int qfm_memcpy_d2d(void *dst, const void *src, size_t n) { return hipMemcpy(dst, src, n, hipMemcpyDeviceToDevice) == hipSuccess ? 0 : -1; }
int qfm_memset(void *dst, int v, size_t n) {   // finished before the return (as qfm_dev_malloc's fill)
    return hipMemsetAsync(dst, v, n, nullptr) == hipSuccess && hipStreamSynchronize(nullptr) == hipSuccess ? 0 : -1;
}
void *qfm_stream_create(void) {
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    return s;
}
int qfm_stream_destroy(void *s) { return hipStreamDestroy(static_cast<hipStream_t>(s)) == hipSuccess ? 0 : -1; }
int qfm_stream_sync(void *s) {
    const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(s));
    if (e != hipSuccess) { set_error(-100 - (int)e, "hipStreamSynchronize: %s", hipGetErrorString(e)); return -1; }
    return 0;
}
int qfm_device_sync(void) {
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) { set_error(-100 - (int)e, "hipDeviceSynchronize: %s", hipGetErrorString(e)); return -1; }
    return 0;
}
void *qfm_event_create(void) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
int qfm_event_destroy(void *e) { return hipEventDestroy(static_cast<hipEvent_t>(e)) == hipSuccess ? 0 : -1; }
int qfm_event_record(void *e, void *s) {
    return hipEventRecord(static_cast<hipEvent_t>(e), static_cast<hipStream_t>(s)) == hipSuccess ? 0 : -1;
}
float qfm_event_elapsed_ms(void *e0, void *e1) {
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, static_cast<hipEvent_t>(e0), static_cast<hipEvent_t>(e1)) != hipSuccess) return -1.0f;
    return ms;
}
int qfm_device_info(char *name, int name_len, int *n_cu, size_t *mem_bytes, int *arch_major, int *arch_minor) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) return -1;
    if (name && name_len > 0) { std::strncpy(name, p.gcnArchName, (size_t)name_len - 1); name[name_len - 1] = 0; }
    if (n_cu) *n_cu = p.multiProcessorCount;
    if (mem_bytes) *mem_bytes = p.totalGlobalMem;
    if (arch_major) *arch_major = p.major;
    if (arch_minor) *arch_minor = p.minor;
    return 0;
}

}  // extern "C"

// the forward on a workspace the caller vouches for, never touching the
// section profiler (whose event pool may create events): the no-allocation entry
int qfm::forward_on_workspace(const qfm_layer *L, const uint16_t *x, int M, uint16_t *y, void *ws, size_t ws_bytes,
                              hipStream_t s) {
    return forward_impl(L, x, M, y, nullptr, ws, ws_bytes, 7, s, false);
}
