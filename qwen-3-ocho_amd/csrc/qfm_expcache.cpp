// qfm_expcache.cpp -- expert arenas filled from the weight store: full
// residency, the host-side LRU, and the host half of the device dispatch.
//
// Transfers follow one pipeline. The expert's six checkpoint tensors
// (gate/up/down packed e2m1 weights and e4m3 block scales) are gathered from
// the mapped store into one of two pinned staging buffers (after that
// buffer's previous transfer has finished: its event), copied to the slot on
// the transfer stream, and the compute stream is made to wait on the buffer's
// event; the host never blocks on compute. In INT8-only residency the NVFP4
// arrays are a two-slot ring: the expert lands in ring slot b (b = the staging
// buffer used) and is converted into its INT8 slot on the transfer stream
// before the buffer's event, so the next transfer through buffer b (which
// waits on that event) cannot overwrite the ring slot early. In FP8 mode the
// expert is packed on the host into the lane-chunk E4M3 form in the staging
// buffer instead.
#include "qfm_internal.h"
#include "../../include/qf_store.h"

#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

using namespace qfm;

namespace qfm {
int launch_quant_rows_bf16(const uint16_t *W, int rows, int K, int8_t *q, float *s, hipStream_t st);
}

namespace {

const char *const kProj[3] = {"gate_proj", "up_proj", "down_proj"};

// One staging buffer holds one expert in the largest form at the largest
// supported shape (H 2560, I 640): FP8 lane-chunk 3*I*H bytes + (2I + H) * 64
// fp32 scales = 5,898,240 bytes (NVFP4 needs 2,764,800).
constexpr size_t kStageBytes = (size_t)3 * 2560 * 640 + (size_t)(2 * 640 + 2560) * 64 * 4;
static_assert(kStageBytes == 5898240, "staging size");
static_assert(kStageBytes >= (size_t)3 * 2560 * 640 / 2 + (size_t)3 * 2560 * 640 / 16, "NVFP4 expert fits the staging buffer");
static_assert(kStageBytes >= (size_t)3 * 2048 * 512 + (size_t)(2 * 512 + 2048) * 64 * 4, "FP8 expert at 2048/512 fits");
constexpr int kLanes = 64;

std::atomic<unsigned long long> g_calls{0}, g_miss{0}, g_bytes{0};

struct Geo {
    size_t wb, sb;   // NVFP4 bytes per projection: packed weights, block scales
    int H, I, E, K;
};
Geo geo() {
    Geo g;
    g.H = g_cfg.H; g.I = g_cfg.I; g.E = g_cfg.E; g.K = g_cfg.K;
    g.wb = (size_t)g.I * g.H / 2;
    g.sb = (size_t)g.I * g.H / 16;
    return g;
}
size_t nv_slot_bytes(const Geo &g) { return 3 * (g.wb + g.sb); }
size_t fp8_slot_bytes(const Geo &g) { return (size_t)3 * g.I * g.H + (size_t)(2 * g.I + g.H) * kLanes * 4; }

const uint8_t *entry_bytes(const QfStore *st, const QfEntry *e) {
    return static_cast<const uint8_t *>(qfm_store_data(st, e));
}

// The six checkpoint tensors of one expert, with the reference's size checks
// (qf_expert_slots.cpp:230-251).
int find_expert(const QfStore *st, int layer, int expert, const QfEntry *we[3], const QfEntry *se[3]) {
    const Geo g = geo();
    char nm[QF_MAX_NAME];
    for (int p = 0; p < 3; p++) {
        std::snprintf(nm, sizeof nm, "model.language_model.layers.%d.mlp.experts.%d.%s.weight", layer, expert, kProj[p]);
        we[p] = qf_find(st, nm);
        std::snprintf(nm, sizeof nm, "model.language_model.layers.%d.mlp.experts.%d.%s.weight_scale", layer, expert,
                      kProj[p]);
        se[p] = qf_find(st, nm);
        if (!we[p] || !se[p] || we[p]->rec.nbytes != g.wb || se[p]->rec.nbytes != g.sb || !entry_bytes(st, we[p]) ||
            !entry_bytes(st, se[p])) {
            set_error(-1, "invalid routed expert tensor L%d E%d %s (need %zu weight and %zu scale bytes)", layer, expert,
                      kProj[p], g.wb, g.sb);
            return -1;
        }
    }
    return 0;
}

// Per-expert scale_2 of one projection for every expert (qf_expert_slots.cpp:78-89).
int load_s2(const QfStore *st, int layer, int proj, float *dst) {
    char nm[QF_MAX_NAME];
    for (int e = 0; e < g_cfg.E; e++) {
        std::snprintf(nm, sizeof nm, "model.language_model.layers.%d.mlp.experts.%d.%s.weight_scale_2", layer, e,
                      kProj[proj]);
        const QfEntry *en = qf_find(st, nm);
        if (!en || en->rec.nbytes != 4 || !entry_bytes(st, en)) {
            set_error(-1, "missing or mis-sized %s (need 4 bytes)", nm);
            return -1;
        }
        std::memcpy(dst + e, entry_bytes(st, en), 4);
    }
    return 0;
}

template <typename T>
bool dalloc(T **p, size_t bytes) {
    *p = nullptr;
    if (hipMalloc(reinterpret_cast<void **>(p), bytes ? bytes : 1) != hipSuccess) {
        *p = nullptr;
        set_error(-4, "expert cache: hipMalloc(%zu) failed", bytes);
        return false;
    }
    return true;
}
template <typename T>
void dfree(T **p) {
    if (*p) (void)hipFree((void *)*p);
    *p = nullptr;
}

// ---- FP8 lane-chunk packing (qf8_moe_fp8.hip:19-37, :217-246) ---------------
float e2m1_value(uint32_t nib) {
    const uint32_t mag = nib & 7u, e = mag >> 1, m = mag & 1u;
    uint32_t bits = ((e + 126u) << 23) | (m << 22);
    float v;
    std::memcpy(&v, &bits, 4);
    if (!e) v = m ? 0.5f : 0.0f;
    return (nib & 8u) ? -v : v;
}
// block scale byte read as an unsigned 5-bit exponent / 3-bit mantissa
float ue4m3_block(uint32_t b) {
    const uint32_t e = b >> 3, m = b & 7u;
    if (!e) return (float)m * 0.001953125f;
    const uint32_t bits = ((e + 120u) << 23) | (m << 20);
    float v;
    std::memcpy(&v, &bits, 4);
    return v;
}
// float -> E4M3 code as the reference's packer does it: magnitudes below
// 2^-9 flush to signed zero, subnormals truncate, normals round to nearest
// even, and everything from 2^8 up saturates to 0x7E (448).
uint8_t e4m3_pack(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    const uint32_t sgn = (u >> 24) & 0x80u;
    int e = (int)((u >> 23) & 0xFFu) - 127;
    const uint32_t m = u & 0x7FFFFFu;
    if (e < -9) return (uint8_t)sgn;
    if (e >= 8) return (uint8_t)(sgn | 0x7Eu);
    if (e < -6) return (uint8_t)(sgn | (((m | 0x800000u) >> (-6 - e + 20)) & 7u));
    uint32_t mm = m >> 20;
    const uint32_t rem = m & 0xFFFFFu;
    if (rem > 0x80000u || (rem == 0x80000u && (mm & 1u))) {
        if (++mm == 8u) {
            mm = 0;
            if (++e >= 8) return (uint8_t)(sgn | 0x7Eu);
        }
    }
    return (uint8_t)(sgn | (uint32_t)((e + 7) << 3) | mm);
}

}  // namespace

extern "C" {

int qf8_fp8_pack_expert(const uint8_t *nv_w, const uint8_t *nv_s, float s2, int rows, int in, uint8_t *w8,
                        float *sc) {
    if (!nv_w || !nv_s || !w8 || !sc || rows < 1 || in < kLanes || in % kLanes || in % 16) {
        set_error(-1, "qf8_fp8_pack_expert: bad arguments (rows %d, in %d)", rows, in);
        return -1;
    }
    const int ch = in / kLanes;   // values per lane chunk
    std::vector<float> v((size_t)ch);
    for (int r = 0; r < rows; r++) {
        const uint8_t *wr = nv_w + (size_t)r * (in / 2);
        const uint8_t *sr = nv_s + (size_t)r * (in / 16);
        for (int l = 0; l < kLanes; l++) {
            float amax = 0.0f;
            for (int c = 0; c < ch; c++) {
                const int k = l * ch + c;
                const uint32_t nib = (k & 1) ? (wr[k / 2] >> 4) : (wr[k / 2] & 15u);
                const float bs = ue4m3_block(sr[k / 16]);
                v[c] = e2m1_value(nib) * (bs * s2);
                amax = std::fmax(amax, std::fabs(v[c]));
            }
            const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
            sc[(size_t)r * kLanes + l] = scale;
            for (int c = 0; c < ch; c++) w8[(size_t)r * in + (size_t)l * ch + c] = e4m3_pack(v[c] / scale);
        }
    }
    return 0;
}

int qf4_expxfer_init(Qf4ExpXfer *xf) {
    if (!xf) { set_error(-1, "qf4_expxfer_init: null context"); return -1; }
    std::memset(xf, 0, sizeof *xf);
    for (int b = 0; b < 2; b++) {
        if (hipHostMalloc(&xf->buf[b], kStageBytes, hipHostMallocDefault) != hipSuccess) {
            xf->buf[b] = nullptr;
            set_error(-4, "qf4_expxfer_init: pinned staging allocation (%zu bytes) failed", kStageBytes);
            qf4_expxfer_free(xf);
            return -1;
        }
        if (hipEventCreateWithFlags(&xf->ev[b], hipEventDisableTiming) != hipSuccess) {
            xf->ev[b] = nullptr;
            set_error(-4, "qf4_expxfer_init: event creation failed");
            qf4_expxfer_free(xf);
            return -1;
        }
    }
    if (hipStreamCreateWithFlags(&xf->xfer, hipStreamNonBlocking) != hipSuccess) {
        xf->xfer = nullptr;
        set_error(-4, "qf4_expxfer_init: stream creation failed");
        qf4_expxfer_free(xf);
        return -1;
    }
    // both buffers start free: their events complete immediately
    for (int b = 0; b < 2; b++) (void)hipEventRecord(xf->ev[b], xf->xfer);
    return 0;
}

void qf4_expxfer_free(Qf4ExpXfer *xf) {
    if (!xf) return;
    if (xf->xfer) (void)hipStreamSynchronize(xf->xfer);
    for (int b = 0; b < 2; b++) {
        if (xf->buf[b]) (void)hipHostFree(xf->buf[b]);
        if (xf->ev[b]) (void)hipEventDestroy(xf->ev[b]);
    }
    if (xf->xfer) (void)hipStreamDestroy(xf->xfer);
    std::memset(xf, 0, sizeof *xf);
}

void qf4_expcache_free(Qf4ExpCache *c) {
    if (!c) return;
    dfree(&c->w_gate); dfree(&c->w_up); dfree(&c->w_down);
    dfree(&c->s_gate); dfree(&c->s_up); dfree(&c->s_down);
    dfree(&c->w8_gate); dfree(&c->w8_up); dfree(&c->w8_down);
    dfree(&c->sc_gate); dfree(&c->sc_up); dfree(&c->sc_down);
    dfree(&c->i8_gate); dfree(&c->i8_up); dfree(&c->i8_down);
    dfree(&c->i8s_gate); dfree(&c->i8s_up); dfree(&c->i8s_down);
    dfree(&c->slot_for_expert_dev); dfree(&c->expert_in_slot_dev);
    dfree(&c->age_dev); dfree(&c->clock_dev); dfree(&c->route_slot_dev);
    dfree(&c->s2g_dev); dfree(&c->s2u_dev); dfree(&c->s2d_dev);
    if (c->mb_host) (void)hipHostFree((void *)c->mb_host);
    std::free(c->slot_for_expert); std::free(c->expert_in_slot); std::free(c->age);
    std::free(c->s2g); std::free(c->s2u); std::free(c->s2d);
    std::memset(c, 0, sizeof *c);
}

static bool modes_ok(int modes) {
    const bool fp8 = modes & QFM_EXPCACHE_FP8, nv = modes & QFM_EXPCACHE_NVFP4, i8 = modes & QFM_EXPCACHE_INT8,
               ring = modes & QFM_EXPCACHE_INT8_ONLY;
    return !((modes & ~15) || (fp8 && (nv || i8 || ring)) || (!fp8 && !nv) || (ring && !i8));
}

size_t qfm_expcache_bytes(int slots, int modes) {
    const Geo g = geo();
    if (!modes_ok(modes) || slots < 1 || slots > g.E) return 0;
    const size_t S = (size_t)slots, n = (size_t)g.I * g.H;
    size_t b = 0;
    if (modes & QFM_EXPCACHE_FP8) {
        b += 3 * S * n + S * ((size_t)2 * g.I + g.H) * kLanes * 4;
    } else {
        const size_t nvs = (modes & QFM_EXPCACHE_INT8_ONLY) ? 2 : S;
        b += 3 * nvs * (g.wb + g.sb);
        if (modes & QFM_EXPCACHE_INT8) b += 3 * S * n + S * ((size_t)2 * g.I + g.H) * 4;
    }
    // device routing state: slot maps, ages, clock, route slots, global scales
    return b + (size_t)g.E * 4 + S * 4 + S * 8 + 8 + QF_ROUTE_MB_CAP * 4 + 3 * (size_t)g.E * 4;
}

int qfm_expcache_init(Qf4ExpCache *c, const QfStore *st, int layer, int slots, int modes) {
    if (!c || !st || layer < 0) { set_error(-1, "qfm_expcache_init: bad arguments"); return -1; }
    std::memset(c, 0, sizeof *c);
    const Geo g = geo();
    const bool fp8 = modes & QFM_EXPCACHE_FP8, i8 = modes & QFM_EXPCACHE_INT8, ring = modes & QFM_EXPCACHE_INT8_ONLY;
    if (!modes_ok(modes)) {
        set_error(-1, "qfm_expcache_init: invalid modes 0x%x (FP8 alone, or NVFP4 [+ INT8 [+ INT8_ONLY]])", modes);
        return -1;
    }
    if (slots < g.K || slots > g.E) {   // fewer than K slots would evict experts of the same token
        set_error(-1, "qfm_expcache_init: slots = %d outside [top_k %d, %d]", slots, g.K, g.E);
        return -1;
    }
    if (const int rc = preflight_device_bytes(qfm_expcache_bytes(slots, modes), "qfm_expcache_init")) return rc;
    if (g.K > QF_ROUTE_MB_CAP) {
        set_error(-1, "qfm_expcache_init: top_k %d exceeds the mailbox capacity %d", g.K, QF_ROUTE_MB_CAP);
        return -1;
    }
    c->layer = layer;
    c->slots = slots;
    const size_t S = (size_t)slots, n = (size_t)g.I * g.H;
    bool ok = true;
    if (fp8) {
        ok = ok && dalloc(&c->w8_gate, S * n) && dalloc(&c->w8_up, S * n) && dalloc(&c->w8_down, S * n);
        ok = ok && dalloc(&c->sc_gate, S * g.I * kLanes * 4) && dalloc(&c->sc_up, S * g.I * kLanes * 4) &&
             dalloc(&c->sc_down, S * g.H * kLanes * 4);
    } else {
        c->nv_ring = ring ? 2 : 0;
        const size_t nvs = ring ? 2 : S;
        ok = ok && dalloc(&c->w_gate, nvs * g.wb) && dalloc(&c->w_up, nvs * g.wb) && dalloc(&c->w_down, nvs * g.wb);
        ok = ok && dalloc(&c->s_gate, nvs * g.sb) && dalloc(&c->s_up, nvs * g.sb) && dalloc(&c->s_down, nvs * g.sb);
        if (i8) {
            ok = ok && dalloc(&c->i8_gate, S * n) && dalloc(&c->i8_up, S * n) && dalloc(&c->i8_down, S * n);
            ok = ok && dalloc(&c->i8s_gate, S * g.I * 4) && dalloc(&c->i8s_up, S * g.I * 4) &&
                 dalloc(&c->i8s_down, S * g.H * 4);
        }
    }
    c->slot_for_expert = (int *)std::malloc((size_t)g.E * sizeof(int));
    c->expert_in_slot = (int *)std::malloc(S * sizeof(int));
    c->age = (uint64_t *)std::calloc(S, sizeof(uint64_t));
    c->s2g = (float *)std::malloc((size_t)g.E * 4);
    c->s2u = (float *)std::malloc((size_t)g.E * 4);
    c->s2d = (float *)std::malloc((size_t)g.E * 4);
    if (!c->slot_for_expert || !c->expert_in_slot || !c->age || !c->s2g || !c->s2u || !c->s2d) {
        set_error(-4, "qfm_expcache_init: out of host memory");
        ok = false;
    }
    if (!ok) { qf4_expcache_free(c); return -4; }
    for (int e = 0; e < g.E; e++) c->slot_for_expert[e] = -1;
    for (size_t i = 0; i < S; i++) c->expert_in_slot[i] = -1;
    if (load_s2(st, layer, 0, c->s2g) || load_s2(st, layer, 1, c->s2u) || load_s2(st, layer, 2, c->s2d)) {
        qf4_expcache_free(c);
        return -1;
    }
    // device routing state, seeded empty (qf_expert_slots.cpp:170-198)
    ok = dalloc(&c->slot_for_expert_dev, (size_t)g.E * 4) && dalloc(&c->expert_in_slot_dev, S * 4) &&
         dalloc(&c->age_dev, S * 8) && dalloc(&c->clock_dev, 8) && dalloc(&c->route_slot_dev, QF_ROUTE_MB_CAP * 4) &&
         dalloc(&c->s2g_dev, (size_t)g.E * 4) && dalloc(&c->s2u_dev, (size_t)g.E * 4) && dalloc(&c->s2d_dev, (size_t)g.E * 4);
    ok = ok && hipMemcpy(c->slot_for_expert_dev, c->slot_for_expert, (size_t)g.E * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(c->expert_in_slot_dev, c->expert_in_slot, S * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemset(c->age_dev, 0, S * 8) == hipSuccess && hipMemset(c->clock_dev, 0, 8) == hipSuccess &&
         hipMemset(c->route_slot_dev, 0xFF, QF_ROUTE_MB_CAP * 4) == hipSuccess &&
         hipMemcpy(c->s2g_dev, c->s2g, (size_t)g.E * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(c->s2u_dev, c->s2u, (size_t)g.E * 4, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(c->s2d_dev, c->s2d, (size_t)g.E * 4, hipMemcpyHostToDevice) == hipSuccess;
    void *mb = nullptr;
    ok = ok && hipHostMalloc(&mb, sizeof(QfRouteMailbox), hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess;
    if (ok) {
        c->mb_host = static_cast<QfRouteMailbox *>(mb);
        std::memset(mb, 0, sizeof(QfRouteMailbox));
        void *dp = nullptr;
        ok = hipHostGetDevicePointer(&dp, mb, 0) == hipSuccess && dp;
        c->mb_dev = static_cast<QfRouteMailbox *>(dp);
    }
    if (!ok) {
        set_error(-4, "qfm_expcache_init: device routing state or mailbox set-up failed for layer %d", layer);
        qf4_expcache_free(c);
        return -4;
    }
    c->expected_seq = 0;
    return 0;
}

int qf4_expcache_init(Qf4ExpCache *c, const QfStore *st, int layer, int slots) {
    auto on = [](const char *v) { const char *s = std::getenv(v); return s && s[0] == '1'; };
    if (slots <= 0) {
        const char *s = std::getenv("QF_EXPERT_CACHE_SLOTS");
        slots = s ? std::atoi(s) : 192;
    }
    if (slots <= 0 || slots > g_cfg.E) slots = g_cfg.E;
    int modes;
    if (on("QF8_MOE_FP8")) modes = QFM_EXPCACHE_FP8;
    else {
        modes = QFM_EXPCACHE_NVFP4;
        if (on("QF_M1_INT8")) modes |= QFM_EXPCACHE_INT8 | (on("QF_M1_INT8_ONLY") ? QFM_EXPCACHE_INT8_ONLY : 0);
    }
    return qfm_expcache_init(c, st, layer, slots, modes);
}

}  // extern "C"

namespace {

// Upload `expert` into `slot` (see the file comment for the pipeline).
// after_compute: the slot still holds an expert that kernels already queued on
// `compute` may read, so the transfer stream first waits for everything queued
// there (write after read). The mailbox service needs no such wait: its host
// side runs after the dispatch kernel, and so after every earlier kernel of
// the stream, has executed.
int xfer_expert(Qf4ExpCache *c, const QfStore *st, Qf4ExpXfer *xf, int expert, int slot, hipStream_t compute,
                bool after_compute = false) {
    const Geo g = geo();
    if (!xf || !xf->xfer || !xf->buf[0] || !xf->buf[1]) { set_error(-1, "expert upload: transfer context not initialised"); return -1; }
    if (expert < 0 || expert >= g.E || slot < 0 || slot >= c->slots) {
        set_error(-1, "expert upload: expert %d / slot %d out of range", expert, slot);
        return -1;
    }
    const QfEntry *we[3], *se[3];
    if (find_expert(st, c->layer, expert, we, se)) return -1;
    const int b = xf->cur;
    xf->cur ^= 1;
    if (hipEventSynchronize(xf->ev[b]) != hipSuccess) { set_error(-3, "expert upload: staging wait failed"); return -1; }
    uint8_t *buf = static_cast<uint8_t *>(xf->buf[b]);
    hipStream_t xs = xf->xfer;
    // ev[b] is free here (synchronized above) and is recorded again on xs
    // below; the wait enqueued now keeps the state of this record
    if (after_compute && (hipEventRecord(xf->ev[b], compute) != hipSuccess ||
                          hipStreamWaitEvent(xs, xf->ev[b], 0) != hipSuccess)) {
        set_error(-3, "expert upload: ordering after the compute stream failed L%d E%d", c->layer, expert);
        return -1;
    }
    bool ok = true;
    if (c->w8_gate) {
        // FP8 lane-chunk: gate/up are [I][H], down [H][I]
        const float s2[3] = {c->s2g[expert], c->s2u[expert], c->s2d[expert]};
        uint8_t *dw[3] = {c->w8_gate, c->w8_up, c->w8_down};
        float *ds[3] = {c->sc_gate, c->sc_up, c->sc_down};
        size_t off = 0;
        for (int p = 0; p < 3 && ok; p++) {
            const int rows = p == 2 ? g.H : g.I, in = p == 2 ? g.I : g.H;
            const size_t wbytes = (size_t)rows * in, sbytes = (size_t)rows * kLanes * 4;
            uint8_t *w8 = buf + off;
            float *sc = reinterpret_cast<float *>(buf + off + wbytes);
            ok = qf8_fp8_pack_expert(entry_bytes(st, we[p]), entry_bytes(st, se[p]), s2[p], rows, in, w8, sc) == 0 &&
                 hipMemcpyAsync(dw[p] + (size_t)slot * wbytes, w8, wbytes, hipMemcpyHostToDevice, xs) == hipSuccess &&
                 hipMemcpyAsync(ds[p] + (size_t)slot * rows * kLanes, sc, sbytes, hipMemcpyHostToDevice, xs) == hipSuccess;
            off += wbytes + sbytes;
        }
    } else {
        for (int p = 0; p < 3; p++) {
            std::memcpy(buf + p * g.wb, entry_bytes(st, we[p]), g.wb);
            std::memcpy(buf + 3 * g.wb + p * g.sb, entry_bytes(st, se[p]), g.sb);
        }
        const int nslot = c->nv_ring ? b : slot;   // ring slot = staging buffer index
        uint8_t *dw[3] = {c->w_gate, c->w_up, c->w_down};
        uint8_t *ds[3] = {c->s_gate, c->s_up, c->s_down};
        for (int p = 0; p < 3 && ok; p++)
            ok = hipMemcpyAsync(dw[p] + (size_t)nslot * g.wb, buf + p * g.wb, g.wb, hipMemcpyHostToDevice, xs) == hipSuccess &&
                 hipMemcpyAsync(ds[p] + (size_t)nslot * g.sb, buf + 3 * g.wb + p * g.sb, g.sb, hipMemcpyHostToDevice,
                                xs) == hipSuccess;
        if (ok && c->nv_ring) ok = qf8_i8_build_slot(c, nslot, slot, expert, xs) == 0;
    }
    if (!ok) {
        set_error(-3, "expert upload failed L%d E%d", c->layer, expert);
        return -1;
    }
    if (hipEventRecord(xf->ev[b], xs) != hipSuccess || hipStreamWaitEvent(compute, xf->ev[b], 0) != hipSuccess) {
        set_error(-3, "expert upload: event ordering failed L%d E%d", c->layer, expert);
        return -1;
    }
    return 0;
}

}  // namespace

extern "C" {

int qf4_expcache_prefill(Qf4ExpCache *c, const QfStore *st, Qf4ExpXfer *xf, hipStream_t compute) {
    if (!c || !st || !xf || !c->slot_for_expert) { set_error(-1, "qf4_expcache_prefill: bad arguments"); return -1; }
    const int E = g_cfg.E;
    if (c->slots < E) return 0;
    for (int e = 0; e < E; e++) {
        if (xfer_expert(c, st, xf, e, e, compute)) return -1;
        c->slot_for_expert[e] = e;
        c->expert_in_slot[e] = e;
        c->age[e] = 1;
    }
    if (hipMemcpy(c->slot_for_expert_dev, c->slot_for_expert, (size_t)E * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(c->expert_in_slot_dev, c->expert_in_slot, (size_t)c->slots * 4, hipMemcpyHostToDevice) != hipSuccess) {
        set_error(-3, "qf4_expcache_prefill: slot map upload failed");
        return -1;
    }
    c->fully_resident = 1;
    return 1;
}

int qf4_expcache_prepare(Qf4ExpCache *c, const QfStore *st, Qf4ExpXfer *xf, int expert, hipStream_t compute) {
    if (!c || !st || !c->slot_for_expert || expert < 0 || expert >= g_cfg.E || c->slots <= 0) {
        set_error(-1, "qf4_expcache_prepare: bad arguments");
        return -1;
    }
    int slot = c->slot_for_expert[expert];
    if (slot >= 0) {
        c->age[slot] = ++c->clock;
        return slot;
    }
    slot = 0;   // first empty slot, else the smallest age (first of equals)
    for (int i = 0; i < c->slots; i++) {
        if (c->expert_in_slot[i] < 0) { slot = i; break; }
        if (c->age[i] < c->age[slot]) slot = i;
    }
    const int evicted = c->expert_in_slot[slot];
    if (xfer_expert(c, st, xf, expert, slot, compute, evicted >= 0)) return -1;
    if (evicted >= 0) c->slot_for_expert[evicted] = -1;
    c->expert_in_slot[slot] = expert;
    c->slot_for_expert[expert] = slot;
    c->age[slot] = ++c->clock;
    return slot;
}

int qf4_expcache_service(Qf4ExpCache *c, const QfStore *st, Qf4ExpXfer *xf, hipStream_t compute) {
    if (!c || !c->mb_host || !st || !xf) { set_error(-1, "qf4_expcache_service: bad arguments"); return -1; }
    QfRouteMailbox *mb = c->mb_host;
    const uint32_t want = c->expected_seq;
    // bounded wait on the stamp the dispatch kernel writes last
    const auto t0 = std::chrono::steady_clock::now();
    for (uint64_t spins = 0; mb->seq != want; spins++) {
        if ((spins & 4095) == 0 && std::chrono::steady_clock::now() - t0 > std::chrono::seconds(30)) {
            set_error(-5, "qf4_expcache_service: mailbox timeout L%d (want seq %u, have %u)", c->layer, want,
                      (unsigned)mb->seq);
            return -1;
        }
    }
    std::atomic_thread_fence(std::memory_order_acquire);
    uint32_t nmiss = mb->miss_n;
    if (nmiss > (uint32_t)g_cfg.K) nmiss = (uint32_t)g_cfg.K;
    g_calls += (unsigned long long)g_cfg.K;
    g_miss += nmiss;
    g_bytes += (unsigned long long)nmiss * (c->w8_gate ? fp8_slot_bytes(geo()) : nv_slot_bytes(geo()));
    for (uint32_t i = 0; i < nmiss; i++) {
        const int expert = mb->miss_expert[i], slot = mb->miss_slot[i];
        if (expert < 0 || expert >= g_cfg.E || slot < 0 || slot >= c->slots) {
            set_error(-5, "qf4_expcache_service: mailbox entry %u corrupt L%d (expert %d, slot %d)", i, c->layer, expert, slot);
            mb->miss_n = 0;
            return -1;
        }
        if (xfer_expert(c, st, xf, expert, slot, compute)) {
            mb->miss_n = 0;
            return -1;
        }
    }
    mb->miss_n = 0;
    return 0;
}

void qf4_expcache_stats(unsigned long long *calls, unsigned long long *miss, unsigned long long *bytes) {
    if (calls) *calls = g_calls.load();
    if (miss) *miss = g_miss.load();
    if (bytes) *bytes = g_bytes.load();
}

}  // extern "C"

// ---- whole MoE layer ----------------------------------------------------------
namespace {

const QfEntry *find_dense(const QfStore *st, const char *fmt, int layer, size_t elems, bool accept_f32 = true) {
    char nm[QF_MAX_NAME];
    std::snprintf(nm, sizeof nm, fmt, layer);
    const QfEntry *e = qf_find(st, nm);
    if (!e || !entry_bytes(st, e) || !(e->rec.nbytes == elems * 2 || (accept_f32 && e->rec.nbytes == elems * 4))) {
        set_error(-1, "missing or mis-sized %s (need %zu bf16 or fp32 values)", nm, elems);
        return nullptr;
    }
    return e;
}

const char *const kRouter = "model.language_model.layers.%d.mlp.gate.weight";
const char *const kShexp[3] = {"model.language_model.layers.%d.mlp.shared_expert.gate_proj.weight",
                               "model.language_model.layers.%d.mlp.shared_expert.up_proj.weight",
                               "model.language_model.layers.%d.mlp.shared_expert.down_proj.weight"};
const char *const kShGate = "model.language_model.layers.%d.mlp.shared_expert_gate.weight";

// dense tensor -> fp32 device [elems] (bf16 widened exactly; fp32 copied)
float *upload_f32(const QfStore *st, const QfEntry *e, size_t elems) {
    std::vector<float> h(elems);
    const uint8_t *src = entry_bytes(st, e);
    if (e->rec.nbytes == elems * 4) std::memcpy(h.data(), src, elems * 4);
    else
        for (size_t i = 0; i < elems; i++) {
            uint16_t b;
            std::memcpy(&b, src + 2 * i, 2);
            const uint32_t u = (uint32_t)b << 16;
            std::memcpy(&h[i], &u, 4);
        }
    float *d = nullptr;
    if (!dalloc(&d, elems * 4)) return nullptr;
    if (hipMemcpy(d, h.data(), elems * 4, hipMemcpyHostToDevice) != hipSuccess) {
        dfree(&d);
        set_error(-3, "layer load: upload of %s failed", e->name);
        return nullptr;
    }
    return d;
}

// dense tensor -> INT8 per-row matrix (fp32 entries rounded to bf16 first, nearest even)
int quant_dense(const QfStore *st, const QfEntry *e, int rows, int K, Qf8I8Mat *m, hipStream_t s) {
    const size_t n = (size_t)rows * K;
    const uint16_t *src = reinterpret_cast<const uint16_t *>(entry_bytes(st, e));
    std::vector<uint16_t> tmp;
    if (e->rec.nbytes == n * 4) {
        tmp.resize(n);
        const uint8_t *f = entry_bytes(st, e);
        for (size_t i = 0; i < n; i++) {
            uint32_t u;
            std::memcpy(&u, f + 4 * i, 4);
            u += 0x7FFFu + ((u >> 16) & 1u);
            tmp[i] = (uint16_t)(u >> 16);
        }
        src = tmp.data();
    }
    return qf8_i8_quant_bf16_host(src, rows, K, m, s);
}

}  // namespace

extern "C" {

int qfm_store_check_layer(const QfStore *st, int layer) {
    if (!st || layer < 0) { set_error(-1, "qfm_store_check_layer: bad arguments"); return -1; }
    const Geo g = geo();
    if (!find_dense(st, kRouter, layer, (size_t)g.E * g.H)) return -1;
    for (int p = 0; p < 3; p++)
        if (!find_dense(st, kShexp[p], layer, (size_t)g.I * g.H)) return -1;
    if (!find_dense(st, kShGate, layer, (size_t)g.H)) return -1;
    for (int e = 0; e < g.E; e++) {
        const QfEntry *we[3], *se[3];
        if (find_expert(st, layer, e, we, se)) return -1;
    }
    std::vector<float> s2((size_t)g.E);
    for (int p = 0; p < 3; p++)
        if (load_s2(st, layer, p, s2.data())) return -1;
    return 0;
}

int qfm_layer_load(qfm_synth_layer *out, const QfStore *st, int layer, int fmt, Qf4ExpXfer *xf, hipStream_t s) {
    if (!out || !st || !xf || (fmt != QFM_FMT_INT8 && fmt != QFM_FMT_NVFP4)) {
        set_error(-1, "qfm_layer_load: bad arguments");
        return -1;
    }
    std::memset(out, 0, sizeof *out);
    if (qfm_store_check_layer(st, layer)) return -1;
    const Geo g = geo();
    {   // the whole layer is priced before anything is allocated: router, gate
        // vector, the INT8 shared expert and the expert arena
        const int modes = fmt == QFM_FMT_INT8 ? (QFM_EXPCACHE_NVFP4 | QFM_EXPCACHE_INT8 | QFM_EXPCACHE_INT8_ONLY)
                                              : QFM_EXPCACHE_NVFP4;
        const size_t plan = (size_t)g.E * g.H * 4 + (size_t)g.H * 4 + (size_t)3 * g.I * g.H +
                            ((size_t)2 * g.I + g.H) * 4 + qfm_expcache_bytes(g.E, modes);
        if (const int rc = preflight_device_bytes(plan, "qfm_layer_load")) return rc;
    }
    qfm_layer &L = out->layer;
    L.fmt = fmt;
    L.arena = &out->arena;
    int rc = 0;
    const QfEntry *er = find_dense(st, kRouter, layer, (size_t)g.E * g.H);
    const QfEntry *eg = find_dense(st, kShGate, layer, (size_t)g.H);
    float *router = upload_f32(st, er, (size_t)g.E * g.H);
    float *gvec = router ? upload_f32(st, eg, (size_t)g.H) : nullptr;
    L.router = router;
    L.sh_gate_inp = gvec;
    if (!router || !gvec) rc = -3;
    Qf8I8Mat *mats[3] = {&L.sh_gate, &L.sh_up, &L.sh_down};
    for (int p = 0; p < 3 && !rc; p++) {
        const int rows = p == 2 ? g.H : g.I, K = p == 2 ? g.I : g.H;
        if (quant_dense(st, find_dense(st, kShexp[p], layer, (size_t)rows * K), rows, K, mats[p], s)) rc = -3;
    }
    if (!rc) {
        const int modes = fmt == QFM_FMT_INT8 ? (QFM_EXPCACHE_NVFP4 | QFM_EXPCACHE_INT8 | QFM_EXPCACHE_INT8_ONLY)
                                              : QFM_EXPCACHE_NVFP4;
        rc = qfm_expcache_init(&out->arena, st, layer, g.E, modes);
        if (!rc && qf4_expcache_prefill(&out->arena, st, xf, s) != 1) rc = -3;
    }
    if (!rc && hipStreamSynchronize(s) != hipSuccess) {
        set_error(-3, "qfm_layer_load: stream synchronize failed");
        rc = -3;
    }
    if (rc) qfm_synth_layer_destroy(out);
    return rc;
}

}  // extern "C"
