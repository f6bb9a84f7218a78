// qfm_arena.cpp -- resident expert arenas and synthetic layers.
//
// The arena is the reference's fully resident layout (slot == expert;
// ocho/amd_server/qf_expert_slots.cpp:332-365 fills every slot at init):
// one device blob per projection, experts back to back, so expert e's gate
// rows start at e * I * H. Synthetic layers fill every tensor with the
// counter-based generator: element n of tensor t in layer L is a pure
// function of (seed, L, t, n), with n the row-major index over the whole
// [experts][rows][cols] blob and the shared expert at expert index E.
#include "qfm_internal.h"
#include "../../include/qf_store.h"

#include <cstring>
#include <type_traits>

namespace qfm {
enum {
    T_QG = 1, T_QU = 2, T_QD = 3, T_SG = 4, T_SU = 5, T_SD = 6,
    T_ROUTER = 7, T_X = 8, T_SHGATE = 9, T_BIAS = 10,
    T_FG = 11, T_FU = 12, T_FD = 13, T_FSG = 14, T_FSU = 15, T_FSD = 16
};

template <typename T>
static bool dmalloc(T **p, size_t n) {
    *p = nullptr;
    const hipError_t e = hipMalloc(reinterpret_cast<void **>(p), n ? n : 1);
    if (e != hipSuccess) {
        set_error(-4, "hipMalloc(%zu) failed: %s", n, hipGetErrorString(e));
        *p = nullptr;
        return false;
    }
    return true;
}
template <typename T>
static void dfree(T **p) {
    if (*p) (void)hipFree(reinterpret_cast<void *>(const_cast<typename std::remove_const<T>::type *>(*p)));
    *p = nullptr;
}
}  // namespace qfm

using namespace qfm;

extern "C" {

size_t qfm_arena_bytes(int fmt) {
    const size_t E = (size_t)g_cfg.E, I = (size_t)g_cfg.I, H = (size_t)g_cfg.H;
    if (fmt == QFM_FMT_INT8) return 3 * E * I * H + E * (2 * I + H) * 4;
    if (fmt == QFM_FMT_NVFP4) return 3 * (E * I * H / 2 + E * I * H / 16) + 3 * E * 4;
    return 0;
}

int qfm_arena_init(Qf4ExpCache *c, int fmt, int layer) {
    if (!c || (fmt != QFM_FMT_INT8 && fmt != QFM_FMT_NVFP4)) { set_error(-1, "qfm_arena_init: bad arguments"); return -1; }
    std::memset(c, 0, sizeof *c);
    if (const int rc = preflight_device_bytes(qfm_arena_bytes(fmt), "qfm_arena_init")) return rc;
    const size_t E = (size_t)g_cfg.E, I = (size_t)g_cfg.I, H = (size_t)g_cfg.H;
    c->layer = layer;
    c->slots = (int)E;
    c->fully_resident = 1;
    bool ok = true;
    if (fmt == QFM_FMT_INT8) {
        ok = ok && dmalloc(&c->i8_gate, E * I * H) && dmalloc(&c->i8_up, E * I * H) && dmalloc(&c->i8_down, E * H * I);
        ok = ok && dmalloc(&c->i8s_gate, E * I * 4) && dmalloc(&c->i8s_up, E * I * 4) && dmalloc(&c->i8s_down, E * H * 4);
    } else {
        ok = ok && dmalloc(&c->w_gate, E * I * H / 2) && dmalloc(&c->w_up, E * I * H / 2) && dmalloc(&c->w_down, E * H * I / 2);
        ok = ok && dmalloc(&c->s_gate, E * I * H / 16) && dmalloc(&c->s_up, E * I * H / 16) && dmalloc(&c->s_down, E * H * I / 16);
        ok = ok && dmalloc(&c->s2g_dev, E * 4) && dmalloc(&c->s2u_dev, E * 4) && dmalloc(&c->s2d_dev, E * 4);
    }
    if (!ok) {
        dfree(&c->i8_gate); dfree(&c->i8_up); dfree(&c->i8_down);
        dfree(&c->i8s_gate); dfree(&c->i8s_up); dfree(&c->i8s_down);
        dfree(&c->w_gate); dfree(&c->w_up); dfree(&c->w_down);
        dfree(&c->s_gate); dfree(&c->s_up); dfree(&c->s_down);
        dfree(&c->s2g_dev); dfree(&c->s2u_dev); dfree(&c->s2d_dev);
        return -4;
    }
    return 0;
}

// also releases what qfm_expcache_init allocates (host maps, routing state, mailbox)
void qfm_arena_free(Qf4ExpCache *c) { qf4_expcache_free(c); }

int qfm_arena_generate(Qf4ExpCache *c, uint32_t seed, uint32_t layer, hipStream_t s) {
    if (!c) { set_error(-1, "qfm_arena_generate: null arena"); return -1; }
    const uint64_t E = (uint64_t)g_cfg.E, I = (uint64_t)g_cfg.I, H = (uint64_t)g_cfg.H;
    int rc = 0;
    if (c->i8_gate) {
        rc |= launch_gen_fill(c->i8_gate, QFM_GEN_I8, 0, E * I * H, seed, layer, T_QG, 0.f, s);
        rc |= launch_gen_fill(c->i8_up, QFM_GEN_I8, 0, E * I * H, seed, layer, T_QU, 0.f, s);
        rc |= launch_gen_fill(c->i8_down, QFM_GEN_I8, 0, E * H * I, seed, layer, T_QD, 0.f, s);
        rc |= launch_gen_fill(c->i8s_gate, QFM_GEN_ROWSCALE, 0, E * I, seed, layer, T_SG, 0.f, s);
        rc |= launch_gen_fill(c->i8s_up, QFM_GEN_ROWSCALE, 0, E * I, seed, layer, T_SU, 0.f, s);
        rc |= launch_gen_fill(c->i8s_down, QFM_GEN_ROWSCALE, 0, E * H, seed, layer, T_SD, 0.f, s);
    }
    if (c->w_gate) {
        rc |= launch_gen_fill(c->w_gate, QFM_GEN_FP4BYTE, 0, E * I * H / 2, seed, layer, T_FG, 0.f, s);
        rc |= launch_gen_fill(c->w_up, QFM_GEN_FP4BYTE, 0, E * I * H / 2, seed, layer, T_FU, 0.f, s);
        rc |= launch_gen_fill(c->w_down, QFM_GEN_FP4BYTE, 0, E * H * I / 2, seed, layer, T_FD, 0.f, s);
        rc |= launch_gen_fill(c->s_gate, QFM_GEN_E4M3SCALE, 0, E * I * H / 16, seed, layer, T_FSG, 0.f, s);
        rc |= launch_gen_fill(c->s_up, QFM_GEN_E4M3SCALE, 0, E * I * H / 16, seed, layer, T_FSU, 0.f, s);
        rc |= launch_gen_fill(c->s_down, QFM_GEN_E4M3SCALE, 0, E * H * I / 16, seed, layer, T_FSD, 0.f, s);
        rc |= launch_fill_f32(c->s2g_dev, E, 0.01f, s);
        rc |= launch_fill_f32(c->s2u_dev, E, 0.01f, s);
        rc |= launch_fill_f32(c->s2d_dev, E, 0.01f, s);
    }
    return rc ? -3 : 0;
}

int qfm_synth_layer_create(qfm_synth_layer *out, int fmt, uint32_t seed, uint32_t layer, int with_bias,
                           hipStream_t s) {
    if (!out) { set_error(-1, "qfm_synth_layer_create: null output"); return -1; }
    std::memset(out, 0, sizeof *out);
    const size_t E = (size_t)g_cfg.E, I = (size_t)g_cfg.I, H = (size_t)g_cfg.H;
    // the whole layer is priced before anything is allocated
    const size_t plan = qfm_arena_bytes(fmt) + E * H * 4 + (with_bias ? E * 4 : 0) + H * 4 + 3 * I * H +
                        (2 * I + H) * 4;
    if (fmt != QFM_FMT_INT8 && fmt != QFM_FMT_NVFP4) { set_error(-1, "qfm_synth_layer_create: bad format"); return -1; }
    if (int rc = preflight_device_bytes(plan, "qfm_synth_layer_create")) return rc;
    int rc = qfm_arena_init(&out->arena, fmt, (int)layer);
    if (rc) return rc;
    qfm_layer &L = out->layer;
    L.arena = &out->arena;
    L.fmt = fmt;
    float *router = nullptr, *bias = nullptr, *g = nullptr;
    int8_t *qg = nullptr, *qu = nullptr, *qd = nullptr;
    float *sg = nullptr, *su = nullptr, *sd = nullptr;
    bool ok = dmalloc(&router, E * H * 4) && dmalloc(&g, H * 4) && dmalloc(&qg, I * H) && dmalloc(&qu, I * H) &&
              dmalloc(&qd, H * I) && dmalloc(&sg, I * 4) && dmalloc(&su, I * 4) && dmalloc(&sd, H * 4);
    if (ok && with_bias) ok = dmalloc(&bias, E * 4);
    L.router = router; L.router_bias = bias; L.sh_gate_inp = g;
    L.sh_gate = Qf8I8Mat{qg, sg, (int)I, (int)H};
    L.sh_up = Qf8I8Mat{qu, su, (int)I, (int)H};
    L.sh_down = Qf8I8Mat{qd, sd, (int)H, (int)I};
    if (!ok) { qfm_synth_layer_destroy(out); return -4; }
    rc = qfm_arena_generate(&out->arena, seed, layer, s);
    rc |= launch_gen_fill(router, QFM_GEN_GAUSS_F32, 0, E * H, seed, layer, T_ROUTER, 0.02f, s);
    rc |= launch_gen_fill(g, QFM_GEN_GAUSS_F32, 0, H, seed, layer, T_SHGATE, 0.02f, s);
    if (bias) rc |= launch_gen_fill(bias, QFM_GEN_GAUSS_F32, 0, E, seed, layer, T_BIAS, 1.5f, s);
    // shared expert = generator expert index E (always INT8)
    rc |= launch_gen_fill(qg, QFM_GEN_I8, E * I * H, I * H, seed, layer, T_QG, 0.f, s);
    rc |= launch_gen_fill(qu, QFM_GEN_I8, E * I * H, I * H, seed, layer, T_QU, 0.f, s);
    rc |= launch_gen_fill(qd, QFM_GEN_I8, E * H * I, H * I, seed, layer, T_QD, 0.f, s);
    rc |= launch_gen_fill(sg, QFM_GEN_ROWSCALE, E * I, I, seed, layer, T_SG, 0.f, s);
    rc |= launch_gen_fill(su, QFM_GEN_ROWSCALE, E * I, I, seed, layer, T_SU, 0.f, s);
    rc |= launch_gen_fill(sd, QFM_GEN_ROWSCALE, E * H, H, seed, layer, T_SD, 0.f, s);
    return rc ? -3 : 0;
}

void qfm_synth_layer_destroy(qfm_synth_layer *l) {
    if (!l) return;
    qfm_arena_free(&l->arena);
    qfm_layer &L = l->layer;
    dfree(&L.router); dfree(&L.router_bias); dfree(&L.sh_gate_inp);
    dfree(&L.sh_gate.w); dfree(&L.sh_up.w); dfree(&L.sh_down.w);
    dfree(&L.sh_gate.s); dfree(&L.sh_up.s); dfree(&L.sh_down.s);
    std::memset(l, 0, sizeof *l);
}

int qfm_gen_input_rows(uint16_t *x, int M, uint32_t seed, uint32_t x_layer, int row0, hipStream_t s) {
    if (!x || M < 1 || row0 < 0) { set_error(-1, "qfm_gen_input_rows: bad arguments"); return -1; }
    const uint64_t H = (uint64_t)g_cfg.H;
    return launch_gen_fill(x, QFM_GEN_GAUSS_BF16, (uint64_t)row0 * H, (uint64_t)M * H, seed, x_layer, T_X, 0.f, s);
}

}  // extern "C"
