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
// then for each of the descriptor's rows decodes them with the gfx950 E4M3
// convert, forms the chunk dot products, scales by the chunk scale and sums
// the tile's outputs across the wave together (one reduce-scatter). Gate/up
// writes silu(g) * u; down adds wt * a into y, the tile's outputs in one
// atomic instruction (one lane per output).
#include "qfm_internal.h"
#include "qfm_dev.h"
#include "../../include/qf_fp8.h"

namespace qfm {

constexpr int kF8Grid = 1024;          // workgroups of the item walks (4 per CU)
constexpr int kF8MaxExperts = 512;
// output rows per item, measured over 8 layers at H 2048 (M = 1 / M = 8 us per
// layer): gate/up 2 rows and down 8 rows 25.6-25.9 / 102.5-102.7; gate/up 1
// row 26.3-26.8 / 129-134; gate/up 4 rows 30.6-34.4 / 124-142; down 4 or 16
// rows 26.2-29.6 / 107-118 with 2 gate/up rows
#ifndef QFM_F8_GU_ROWS
#define QFM_F8_GU_ROWS 2
#endif
#ifndef QFM_F8_DN_ROWS
#define QFM_F8_DN_ROWS 8
#endif
constexpr int kF8RowsGu = QFM_F8_GU_ROWS;   // gate/up output rows per item
constexpr int kF8RowsDn = QFM_F8_DN_ROWS;   // down output rows per item

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

// CH = H / 64 code bytes per lane and row (32 at H 2048, 40 at H 2560), loaded
// as 16-byte words when CH allows (8-byte words otherwise)
template <int CH>
struct F8Row {
    static constexpr bool W16 = CH % 16 == 0;
    static constexpr int NQ = W16 ? CH / 16 : CH / 8;
    uint4 q[W16 ? NQ : 1];
    uint2 d[W16 ? 1 : NQ];
    __device__ __forceinline__ void load(const uint8_t *p) {
        if constexpr (W16) {
#pragma unroll
            for (int j = 0; j < NQ; j++) q[j] = reinterpret_cast<const uint4 *>(p)[j];
        } else {
#pragma unroll
            for (int j = 0; j < NQ; j++) d[j] = reinterpret_cast<const uint2 *>(p)[j];
        }
    }
    // the codes as opaque to the compiler: a decode inside a loop is then not
    // hoisted out of it (R rows decoded at once would not fit the registers)
    __device__ __forceinline__ void opaque() {
        if constexpr (W16) {
#pragma unroll
            for (int j = 0; j < NQ; j++) asm volatile("" : "+v"(q[j].x), "+v"(q[j].y), "+v"(q[j].z), "+v"(q[j].w));
        } else {
#pragma unroll
            for (int j = 0; j < NQ; j++) asm volatile("" : "+v"(d[j].x), "+v"(d[j].y));
        }
    }
    __device__ __forceinline__ void decode(float *out) const {
        if constexpr (W16) {
#pragma unroll
            for (int j = 0; j < NQ; j++) {
                f8x8(make_uint2(q[j].x, q[j].y), out + 16 * j);
                f8x8(make_uint2(q[j].z, q[j].w), out + 16 * j + 8);
            }
        } else {
#pragma unroll
            for (int j = 0; j < NQ; j++) f8x8(d[j], out + 8 * j);
        }
    }
};

// gate/up: item = (descriptor, R output rows); the wave loads the R gate and
// up rows' chunks (lane l owns bytes [l CH, l CH + CH) of each row) and their
// chunk scales, and for each descriptor row decodes and dots them with the
// lane's slice of x (loaded once per row, not per output row), the 2R
// sums reduced across the wave together (reduce-scatter: lane 2 r + m holds
// output r's gate (m = 0) or up (m = 1) sum)
template <int CH>
__global__ void __launch_bounds__(256)
k_fp8_gateup(const uint8_t *__restrict__ Wg, const float *__restrict__ Sg, const uint8_t *__restrict__ Wu,
             const float *__restrict__ Su, const float *__restrict__ x, float *__restrict__ hidden,
             const Qf8MoeDesc *__restrict__ desc, const int *__restrict__ ctl, int I) {
    constexpr int H = CH * 64, R = kF8RowsGu;
    static_assert(2 * R <= 32 && (R & (R - 1)) == 0, "2R sums per lane, a power of two");
    const int lane = threadIdx.x & 63;
    const int tiles = I / R;
    const int total = ctl[0] * tiles;
    for (int item = blockIdx.x * 4 + (threadIdx.x >> 6); item < total; item += gridDim.x * 4) {
        const int di = item / tiles, o0 = (item % tiles) * R;
        const Qf8MoeDesc &D = desc[di];
        const int slot = D.slot, nrow = D.nrow;
        const size_t wb = (size_t)slot * I * H + (size_t)o0 * H + (size_t)lane * CH;
        const size_t sb = ((size_t)slot * I + o0) * 64 + lane;
        F8Row<CH> gq[R], uq[R];
        float sg[R], su[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            gq[r].load(Wg + wb + (size_t)r * H);
            uq[r].load(Wu + wb + (size_t)r * H);
            sg[r] = Sg[sb + r * 64];
            su[r] = Su[sb + r * 64];
        }
        for (int t = 0; t < nrow; t++) {
            const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)D.row[t] * H + (size_t)lane * CH);
            float xv[CH];
#pragma unroll
            for (int j = 0; j < CH / 4; j++) {
                const float4 v = xr[j];
                xv[4 * j] = v.x; xv[4 * j + 1] = v.y; xv[4 * j + 2] = v.z; xv[4 * j + 3] = v.w;
            }
            float s[2 * R];
#pragma unroll
            for (int r = 0; r < R; r++) {          // codes decoded per row of x (one row on average)
                float wv[CH], ag = 0.0f, au = 0.0f;
                gq[r].opaque();
                uq[r].opaque();
                gq[r].decode(wv);
#pragma unroll
                for (int j = 0; j < CH; j++) ag = fmaf(wv[j], xv[j], ag);
                uq[r].decode(wv);
#pragma unroll
                for (int j = 0; j < CH; j++) au = fmaf(wv[j], xv[j], au);
                s[2 * r] = ag * sg[r];
                s[2 * r + 1] = au * su[r];
                __builtin_amdgcn_sched_barrier(0);   // one row's decode at a time (registers)
            }
            const float v = canon_scatter_level<2 * R, 1>(s, lane);     // lane l: sum l & (2R - 1)
            const float u = lane_xor<1>(v);                             // the partner's (up, at odd lanes)
            if (lane < 2 * R && (lane & 1) == 0)
                hidden[((size_t)di * QF8_FP8_MAXROW + t) * I + o0 + (lane >> 1)] = silu(v) * u;
        }
    }
}

// CHD = I / 64 code bytes per lane and row (8 at I 512, 10 at I 640); item =
// (descriptor, R output rows), the R sums of a descriptor row reduced together
// (lane r holds output r) and added into y by R lanes of one atomic instruction
template <int CHD>
__global__ void __launch_bounds__(256)
k_fp8_downacc(const uint8_t *__restrict__ Wd, const float *__restrict__ Sd, const float *__restrict__ hidden,
              float *__restrict__ y, const Qf8MoeDesc *__restrict__ desc, const int *__restrict__ ctl, int H) {
    constexpr int I = CHD * 64, R = kF8RowsDn;
    static_assert(R <= 32 && (R & (R - 1)) == 0, "R sums per lane, a power of two");
    const int lane = threadIdx.x & 63;
    const int tiles = H / R;
    const int total = ctl[0] * tiles;
    for (int item = blockIdx.x * 4 + (threadIdx.x >> 6); item < total; item += gridDim.x * 4) {
        const int di = item / tiles, o0 = (item % tiles) * R;
        const Qf8MoeDesc &D = desc[di];
        const int slot = D.slot, nrow = D.nrow;
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
                    const uint32_t b0 = p[j] & 0xFFu, b1 = p[j] >> 8;
                    if (__builtin_expect((b0 & 0x7Fu) == 0x7Fu, 0)) w[r][2 * j] = (b0 & 0x80u) ? -480.0f : 480.0f;
                    if (__builtin_expect((b1 & 0x7Fu) == 0x7Fu, 0)) w[r][2 * j + 1] = (b1 & 0x80u) ? -480.0f : 480.0f;
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
            const int yrow = D.row[t];
            const float wt = D.wt[t];
            float s[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                float a = 0.0f;
#pragma unroll
                for (int j = 0; j < CHD; j++) a = fmaf(w[r][j], h[j], a);
                s[r] = a * sd[r];
            }
            const float a = canon_scatter_level<R, 1>(s, lane);          // lane l: output l & (R - 1)
            if (lane < R) atomicAdd(&y[(size_t)yrow * H + o0 + lane], wt * a);
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
