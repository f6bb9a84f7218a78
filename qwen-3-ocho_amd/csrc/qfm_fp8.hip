// qfm_fp8.hip -- MoE over the FP8 lane-chunk arena (format and contract in
// include/qf_fp8.h; semantics of ocho/amd_server/qf8_moe_fp8.hip:45-213).
//
// k_fp8_build_desc: one wave. The routing is staged in LDS, the selected
// experts are marked in a bitmap (descriptor index = rank of the expert id),
// and one pass over the tokens in order appends each (row, weight) to its
// expert's descriptor through per-expert counters.
// k_fp8_gateup / k_fp8_downacc: a fixed grid of 256-thread workgroups; wave w
// of workgroup b takes items b*4 + w, then strides by 4 * gridDim.x, until
// the device-side item count ctl[0] * tiles is exhausted (every wave reaches
// that bound). An item is (descriptor, tile of output rows); the wave loads
// all of the tile's weight chunks first (lane l owns chunk l of every row),
// decodes them with the gfx950 E4M3 convert, then for each of the
// descriptor's rows forms the chunk dot products, scales by the chunk scale
// and sums across the wave (DPP). Gate/up writes silu(g) * u; down adds
// wt * a into y with one atomic per (row, output).
#include "qfm_internal.h"
#include "qfm_dev.h"
#include "../../include/qf_fp8.h"

namespace qfm {

constexpr int kF8Grid = 1024;          // workgroups of the item walks (4 per CU)
constexpr int kF8MaxExperts = 512;
constexpr int kF8RowsGu = 4;           // gate/up output rows per item
constexpr int kF8RowsDn = 8;           // down output rows per item

// Routing of up to kF8LdsPairs (row, k) pairs is staged in LDS; larger
// batches are read from global memory in the same order.
constexpr int kF8LdsPairs = 2048;

__global__ void __launch_bounds__(64)
k_fp8_build_desc(const int *__restrict__ sel, const float *__restrict__ wt, int M, int K, int slot_base,
                 Qf8MoeDesc *__restrict__ desc, int *__restrict__ ctl, int n_experts) {
    __shared__ unsigned bits[kF8MaxExperts / 32];
    __shared__ int wpre[kF8MaxExperts / 32];            // set bits in the words before
    __shared__ int cnt[kF8MaxExperts];                  // rows seen per expert so far
    __shared__ int s_sel[kF8LdsPairs];
    __shared__ float s_wt[kF8LdsPairs];
    const int lane = threadIdx.x;
    const int nw = (n_experts + 31) / 32, P = M * K;
    const bool staged = P <= kF8LdsPairs;
    for (int i = lane; i < nw; i += 64) bits[i] = 0u;
    for (int i = lane; i < n_experts; i += 64) cnt[i] = 0;
    if (staged)
        for (int i = lane; i < P; i += 64) {
            s_sel[i] = sel[i];
            s_wt[i] = wt[i];
        }
    __syncthreads();
    const int *ss = staged ? s_sel : sel;
    const float *sw = staged ? s_wt : wt;
    for (int i = lane; i < P; i += 64) {
        const int e = ss[i];
        if (e >= 0 && e < n_experts) atomicOr(&bits[e >> 5], 1u << (e & 31));
    }
    __syncthreads();
    if (lane == 0) {
        int acc = 0;
        for (int w = 0; w < nw; w++) {
            wpre[w] = acc;
            acc += __popc(bits[w]);
        }
        ctl[0] = acc;
        ctl[1] = 0;
        ctl[2] = 0;
    }
    __syncthreads();
    // rows in token order, lane k holding selection k of the token; a repeated
    // expert within one token keeps only its first k (as the reference's
    // first-match search does), so the lanes of one step touch distinct counters
    for (int t = 0; t < M; t++) {
        const int e = lane < K ? ss[t * K + lane] : -1;
        bool first = e >= 0 && e < n_experts;
        for (int j = 0; j < K; j++) {
            const int ej = __shfl(e, j, 64);
            if (j < lane && ej == e) first = false;
        }
        if (first) {
            const int di = wpre[e >> 5] + __popc(bits[e >> 5] & ((1u << (e & 31)) - 1u));
            const int c = cnt[e];
            cnt[e] = c + 1;
            if (c < QF8_FP8_MAXROW) {
                desc[di].row[c] = t;
                desc[di].wt[c] = sw[t * K + lane];
            }
        }
        __syncthreads();
    }
    for (int e = lane; e < n_experts; e += 64) {
        if (!((bits[e >> 5] >> (e & 31)) & 1u)) continue;
        const int di = wpre[e >> 5] + __popc(bits[e >> 5] & ((1u << (e & 31)) - 1u));
        desc[di].slot = slot_base + e;
        desc[di].nrow = min(cnt[e], QF8_FP8_MAXROW);
    }
}

// a byte of w whose low seven bits are all set (0x7F or 0xFF)
__device__ __forceinline__ bool has_f8_top_code(uint32_t w) {
    const uint32_t v = ~(w | 0x80808080u);             // that byte of v is zero, every other byte nonzero
    return ((v - 0x01010101u) & ~v & 0x80808080u) != 0u;
}
// decode 8 E4M3 codes (one uint2) into out[0..7]: the gfx950 OCP convert, which
// matches the reference's integer decode (qf8_moe_fp8.hip:19-26) on every code
// but 0x7F / 0xFF; those read +-480 there (exponent 15, mantissa 7, no NaN) and
// NaN here, so a lane holding one takes the integer value instead
__device__ __forceinline__ void f8x8(uint2 q, float *out) {
    const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8(q.x, false), b = __builtin_amdgcn_cvt_pk_f32_fp8(q.x, true);
    const f32x2_t c = __builtin_amdgcn_cvt_pk_f32_fp8(q.y, false), d = __builtin_amdgcn_cvt_pk_f32_fp8(q.y, true);
    out[0] = a.x; out[1] = a.y; out[2] = b.x; out[3] = b.y;
    out[4] = c.x; out[5] = c.y; out[6] = d.x; out[7] = d.y;
    if (__builtin_expect(has_f8_top_code(q.x) || has_f8_top_code(q.y), 0)) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
            if ((byte & 0x7Fu) == 0x7Fu) out[i] = (byte & 0x80u) ? -480.0f : 480.0f;
        }
    }
}

// CH = H / 64 code bytes per lane and row (32 at H 2048, 40 at H 2560)
template <int CH>
__global__ void __launch_bounds__(256)
k_fp8_gateup(const uint8_t *__restrict__ Wg, const float *__restrict__ Sg, const uint8_t *__restrict__ Wu,
             const float *__restrict__ Su, const float *__restrict__ x, float *__restrict__ hidden,
             const Qf8MoeDesc *__restrict__ desc, const int *__restrict__ ctl, int I) {
    constexpr int H = CH * 64, NW = CH / 8, R = kF8RowsGu;
    const int lane = threadIdx.x & 63;
    const int tiles = I / R;
    const int total = ctl[0] * tiles;
    for (int item = blockIdx.x * 4 + (threadIdx.x >> 6); item < total; item += gridDim.x * 4) {
        const int di = item / tiles, o0 = (item % tiles) * R;
        const int slot = desc[di].slot, nrow = desc[di].nrow;
        const size_t wb = (size_t)slot * I * H + (size_t)o0 * H + (size_t)lane * CH;
        const size_t sb = ((size_t)slot * I + o0) * 64 + lane;
        uint2 gq[R][NW], uq[R][NW];
        float sg[R], su[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint2 *pg = reinterpret_cast<const uint2 *>(Wg + wb + (size_t)r * H);
            const uint2 *pu = reinterpret_cast<const uint2 *>(Wu + wb + (size_t)r * H);
#pragma unroll
            for (int j = 0; j < NW; j++) {
                gq[r][j] = pg[j];
                uq[r][j] = pu[j];
            }
            sg[r] = Sg[sb + r * 64];
            su[r] = Su[sb + r * 64];
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            float gv[CH], uv[CH];
#pragma unroll
            for (int j = 0; j < NW; j++) {
                f8x8(gq[r][j], gv + 8 * j);
                f8x8(uq[r][j], uv + 8 * j);
            }
            for (int t = 0; t < nrow; t++) {
                const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)desc[di].row[t] * H + (size_t)lane * CH);
                float ag = 0.0f, au = 0.0f;
#pragma unroll
                for (int j = 0; j < CH / 4; j++) {
                    const float4 xv = xr[j];
                    ag = fmaf(gv[4 * j + 3], xv.w, fmaf(gv[4 * j + 2], xv.z, fmaf(gv[4 * j + 1], xv.y, fmaf(gv[4 * j], xv.x, ag))));
                    au = fmaf(uv[4 * j + 3], xv.w, fmaf(uv[4 * j + 2], xv.z, fmaf(uv[4 * j + 1], xv.y, fmaf(uv[4 * j], xv.x, au))));
                }
                const float g = group_sum<64>(ag * sg[r]), u = group_sum<64>(au * su[r]);
                if (lane == 0) hidden[((size_t)di * QF8_FP8_MAXROW + t) * I + o0 + r] = silu(g) * u;
            }
        }
    }
}

// CHD = I / 64 code bytes per lane and row (8 at I 512, 10 at I 640)
template <int CHD>
__global__ void __launch_bounds__(256)
k_fp8_downacc(const uint8_t *__restrict__ Wd, const float *__restrict__ Sd, const float *__restrict__ hidden,
              float *__restrict__ y, const Qf8MoeDesc *__restrict__ desc, const int *__restrict__ ctl, int H) {
    constexpr int I = CHD * 64, R = kF8RowsDn;
    const int lane = threadIdx.x & 63;
    const int tiles = H / R;
    const int total = ctl[0] * tiles;
    for (int item = blockIdx.x * 4 + (threadIdx.x >> 6); item < total; item += gridDim.x * 4) {
        const int di = item / tiles, o0 = (item % tiles) * R;
        const int slot = desc[di].slot, nrow = desc[di].nrow;
        const size_t wb = (size_t)slot * H * I + (size_t)o0 * I + (size_t)lane * CHD;
        const size_t sb = ((size_t)slot * H + o0) * 64 + lane;
        float w[R][CHD], sd[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            if constexpr (CHD == 8) {
                f8x8(*reinterpret_cast<const uint2 *>(Wd + wb + (size_t)r * I), w[r]);
            } else {
                const uint16_t *p = reinterpret_cast<const uint16_t *>(Wd + wb + (size_t)r * I);
#pragma unroll
                for (int j = 0; j < CHD / 2; j++) {
                    const f32x2_t v = __builtin_amdgcn_cvt_pk_f32_fp8((uint32_t)p[j], false);
                    w[r][2 * j] = v.x;
                    w[r][2 * j + 1] = v.y;
                }
            }
            sd[r] = Sd[sb + r * 64];
        }
        for (int t = 0; t < nrow; t++) {
            const float *hr = hidden + ((size_t)di * QF8_FP8_MAXROW + t) * I + (size_t)lane * CHD;
            float h[CHD];
#pragma unroll
            for (int j = 0; j < CHD / 2; j++) {
                const float2 v = reinterpret_cast<const float2 *>(hr)[j];
                h[2 * j] = v.x;
                h[2 * j + 1] = v.y;
            }
            const int yrow = desc[di].row[t];
            const float wt = desc[di].wt[t];
#pragma unroll
            for (int r = 0; r < R; r++) {
                float a = 0.0f;
#pragma unroll
                for (int j = 0; j < CHD; j++) a = fmaf(w[r][j], h[j], a);
                a = group_sum<64>(a * sd[r]);
                if (lane == 0) atomicAdd(&y[(size_t)yrow * H + o0 + r], wt * a);
            }
        }
    }
}

static bool fp8_shape_ok(const char *who) {
    if (!shape_2048() && !shape_2560()) {
        set_error(-2, "%s: unsupported shape H %d I %d", who, g_cfg.H, g_cfg.I);
        return false;
    }
    return true;
}

}  // namespace qfm

using namespace qfm;

extern "C" {

int qf8_fp8_build_desc_ex(const int *sel_dev, const float *wt_dev, int M, int K, int slot_base, Qf8MoeDesc *desc,
                          int *ctl, hipStream_t s) {
    if (!sel_dev || !wt_dev || !desc || !ctl) { set_error(-1, "qf8_fp8_build_desc: null argument"); return -1; }
    if (M < 1 || K < 1 || K > 64 || M > (1 << 20) / K || slot_base < 0 || g_cfg.E > kF8MaxExperts) {
        set_error(-2, "qf8_fp8_build_desc: M %d, K %d, slot_base %d out of range", M, K, slot_base);
        return -2;
    }
    hipLaunchKernelGGL(k_fp8_build_desc, dim3(1), dim3(64), 0, s, sel_dev, wt_dev, M, K, slot_base, desc, ctl, g_cfg.E);
    return check_launch("qf8_fp8_build_desc") ? -3 : 0;
}

int qf8_fp8_gateup_ex(const uint8_t *Wg, const float *Sg, const uint8_t *Wu, const float *Su, const float *x,
                      float *hidden, const Qf8MoeDesc *desc, int *ctl, hipStream_t s) {
    if (!Wg || !Sg || !Wu || !Su || !x || !hidden || !desc || !ctl) { set_error(-1, "qf8_fp8_gateup: null argument"); return -1; }
    if (!fp8_shape_ok("qf8_fp8_gateup")) return -2;
    if (shape_2048())
        hipLaunchKernelGGL(k_fp8_gateup<32>, dim3(kF8Grid), dim3(256), 0, s, Wg, Sg, Wu, Su, x, hidden, desc, ctl, g_cfg.I);
    else
        hipLaunchKernelGGL(k_fp8_gateup<40>, dim3(kF8Grid), dim3(256), 0, s, Wg, Sg, Wu, Su, x, hidden, desc, ctl, g_cfg.I);
    return check_launch("qf8_fp8_gateup") ? -3 : 0;
}

int qf8_fp8_downacc_ex(const uint8_t *Wd, const float *Sd, const float *hidden, float *y, const Qf8MoeDesc *desc,
                       int *ctl, hipStream_t s) {
    if (!Wd || !Sd || !hidden || !y || !desc || !ctl) { set_error(-1, "qf8_fp8_downacc: null argument"); return -1; }
    if (!fp8_shape_ok("qf8_fp8_downacc")) return -2;
    if (shape_2048())
        hipLaunchKernelGGL(k_fp8_downacc<8>, dim3(kF8Grid), dim3(256), 0, s, Wd, Sd, hidden, y, desc, ctl, g_cfg.H);
    else
        hipLaunchKernelGGL(k_fp8_downacc<10>, dim3(kF8Grid), dim3(256), 0, s, Wd, Sd, hidden, y, desc, ctl, g_cfg.H);
    return check_launch("qf8_fp8_downacc") ? -3 : 0;
}

void qf8_fp8_build_desc(const int *sel_dev, const float *wt_dev, int M, int K, int slot_base, Qf8MoeDesc *desc,
                        int *ctl, hipStream_t s) {
    (void)qf8_fp8_build_desc_ex(sel_dev, wt_dev, M, K, slot_base, desc, ctl, s);
}
void qf8_fp8_gateup(const uint8_t *Wg, const float *Sg, const uint8_t *Wu, const float *Su, const float *x,
                    float *hidden, const Qf8MoeDesc *desc, int *ctl, hipStream_t s) {
    (void)qf8_fp8_gateup_ex(Wg, Sg, Wu, Su, x, hidden, desc, ctl, s);
}
void qf8_fp8_downacc(const uint8_t *Wd, const float *Sd, const float *hidden, float *y, const Qf8MoeDesc *desc,
                     int *ctl, hipStream_t s) {
    (void)qf8_fp8_downacc_ex(Wd, Sd, hidden, y, desc, ctl, s);
}

}  // extern "C"
