// qfm_compat.hip -- the reference-named launchers that the fused layer
// forward (qfm_moe_forward) does not route through: the X8 activation
// quantizer, the chunk (CSR) INT8 expert tier, the NVFP4 M=1 and M=8 tiers,
// the INT8 shared expert and the NVFP4 -> INT8 arena build. They keep the
// reference's argument lists and buffer contracts (y seeded / pre-zeroed /
// overwritten exactly where the reference does) so an engine call site links
// against them unchanged.
//
// Differences from the reference, all in the direction of more exact
// arithmetic: hidden vectors are kept in fp32 between gate/up and down (the
// reference re-quantizes them to X8; h8q/h8s/e8q/e8s are accepted and not
// written). E4M3 block scales are decoded from the byte with integer ops
// exactly as the reference does (e4m3_scale: e = byte >> 3, so bytes >= 0x80
// are large unsigned scales, and 0x7F is +inf), not by the OCP fp8 convert.
//
// Every reference-named void launcher has an _ex twin that returns 0, -1 (a
// rejected argument: nothing launched), -2 (unsupported shape) or -3 (launch
// failure); the void form calls it and leaves the code in the error latch.
#include "qfm_dev.h"
#include "qfm_internal.h"

namespace qfm {

constexpr int kMaxSel = 16;       // top_k upper bound (qfm_init validates it)

// ---- X8: per 32-block scale absmax/127 (1 for an all-zero block), q = rint(v/s)
// clamped to +-127 (ocho/amd_server/qf8_moe_i8.hip:58-70, qf8_dense_i8.hip k_d8_x8).
__global__ void __launch_bounds__(256)
k_x8(const float *__restrict__ x, int8_t *__restrict__ q, float *__restrict__ s, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const float v = i < n ? x[i] : 0.0f;
    float mx = fabsf(v);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, WAVE));
    if (i >= n) return;
    const float sc = mx > 0.0f ? mx * (1.0f / 127.0f) : 1.0f;
    int qi = (int)rintf(v / sc);
    qi = qi > 127 ? 127 : (qi < -127 ? -127 : qi);
    q[i] = (int8_t)qi;
    if ((i & 31) == 0) s[i >> 5] = sc;
}

// ---- routing inversion for any T (qf8_i8_csr_build semantics,
// qf8_moe_i8.hip:323-362): experts ascending, an expert's pairs in pair order
// p = t*K + k, pair_tok = p / K; counts = {n_exp, n_pairs}. Deterministic.
// Pass 1 (one block): per-expert counts in LDS, scans, distinct compaction.
__global__ void __launch_bounds__(1024)
k_cb_count(const int *__restrict__ sel, int P, int E, int *__restrict__ exp_slot, int *__restrict__ exp_ptr,
           int *__restrict__ counts) {
    __shared__ int cnt[1024], sc[1024], nz[1024];
    const int t = threadIdx.x;
    cnt[t] = 0;
    __syncthreads();
    for (int p = t; p < P; p += 1024) {
        const int e = sel[p];
        if ((unsigned)e < (unsigned)E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    const int c = cnt[t], f = c > 0 ? 1 : 0;
    sc[t] = c;
    nz[t] = f;
    __syncthreads();
    for (int st = 1; st < 1024; st <<= 1) {          // inclusive scans (Hillis-Steele)
        const int a = t >= st ? sc[t - st] : 0, b = t >= st ? nz[t - st] : 0;
        __syncthreads();
        sc[t] += a;
        nz[t] += b;
        __syncthreads();
    }
    if (f) { exp_slot[nz[t] - 1] = t; exp_ptr[nz[t] - 1] = sc[t] - c; }
    if (t == 1023) { exp_ptr[nz[t]] = sc[t]; counts[0] = nz[t]; counts[1] = sc[t]; }
}
// Pass 2 (one block per 256 pairs): position = start of the expert's range +
// #{earlier blocks' pairs of that expert} (histogram of the prefix in LDS) +
// #{earlier pairs of this block with that expert}.
__global__ void __launch_bounds__(256)
k_cb_scatter(const int *__restrict__ sel, const float *__restrict__ wt, int P, int K, int E,
             const int *__restrict__ exp_slot, const int *__restrict__ exp_ptr, const int *__restrict__ counts,
             int *__restrict__ pair_tok, float *__restrict__ pair_wt) {
    __shared__ int h[1024];
    __shared__ int ts[256];
    const int t = threadIdx.x, p0 = blockIdx.x * 256, p = p0 + t;
    for (int i = t; i < E; i += 256) h[i] = 0;
    __syncthreads();
    for (int q = t; q < p0; q += 256) {
        const int e = sel[q];
        if ((unsigned)e < (unsigned)E) atomicAdd(&h[e], 1);
    }
    const int e = p < P ? sel[p] : -1;
    ts[t] = e;
    __syncthreads();
    if (p >= P || (unsigned)e >= (unsigned)E) return;
    int r = 0;
    for (int j = 0; j < t; j++) r += ts[j] == e ? 1 : 0;
    int lo = 0, hi = counts[0] - 1;                   // exp_slot is ascending: find e
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (exp_slot[mid] < e) lo = mid + 1; else hi = mid;
    }
    const int pos = exp_ptr[lo] + h[e] + r;
    pair_tok[pos] = p / K;
    pair_wt[pos] = wt[p];
}

// ---- M=8 tier routing inversion restricted to one expert range
// (qf_moe_m8_wave64.hip:261-311): experts [lo, lo + epc) only, ascending;
// exp_slot = slot_base + (e - lo); pairs in (token, k) order. One block,
// one thread per pair (M*K <= 1024), E <= 1024.
__global__ void __launch_bounds__(1024)
k_m8_csr(const int *__restrict__ sel, const float *__restrict__ wt, int P, int K, int lo, int hi, int slot_base,
         int *__restrict__ exp_slot, int *__restrict__ exp_ptr, int *__restrict__ pair_tok,
         float *__restrict__ pair_wt, int *__restrict__ counts) {
    __shared__ int se[1024];
    __shared__ uint32_t bits[32];
    const int p = threadIdx.x;
    if (p < 32) bits[p] = 0u;
    const int e = p < P ? sel[p] : -1;
    const bool own = e >= lo && e < hi;
    se[p] = own ? e : -1;
    __syncthreads();
    if (own) atomicOr(&bits[e >> 5], 1u << (e & 31));
    int less = 0, before = 0;
    if (own)
        for (int q = 0; q < P; q++) {
            const int f = se[q];
            less += (f >= 0 && f < e) ? 1 : 0;
            before += (f == e && q < p) ? 1 : 0;
        }
    const int n_pairs = __syncthreads_count(own ? 1 : 0);
    if (own) {
        int first_less = __popc(bits[e >> 5] & ((1u << (e & 31)) - 1u));
        for (int w = 0; w < (e >> 5); w++) first_less += __popc(bits[w]);
        pair_tok[less + before] = p / K;
        pair_wt[less + before] = wt[p];
        if (before == 0) { exp_slot[first_less] = slot_base + (e - lo); exp_ptr[first_less] = less; }
    }
    if (p == 0) {
        int n = 0;
        for (int w = 0; w < 32; w++) n += __popc(bits[w]);
        exp_ptr[n] = n_pairs;
        counts[0] = n;
        counts[1] = n_pairs;
    }
}

// ---- INT8 weights x X8 activations: exact integer dot of 16 values
__device__ __forceinline__ int dot16_i8i8(uint4 w, uint4 x) {
    int a = __builtin_amdgcn_sdot4((int)w.x, (int)x.x, 0, false);
    a = __builtin_amdgcn_sdot4((int)w.y, (int)x.y, a, false);
    a = __builtin_amdgcn_sdot4((int)w.z, (int)x.z, a, false);
    return __builtin_amdgcn_sdot4((int)w.w, (int)x.w, a, false);
}
// INT8 weights x fp32 values: offset-binary dot with the -128*sum correction.
__device__ __forceinline__ float dot16_i8f(uint4 w, const float *x, float acc) {
    float sx = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) sx += x[i];
    return dot16_u8(w, x, fmaf(-128.0f, sx, acc));
}
__device__ __forceinline__ void ld_f32x16(const float *p, float *v) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 a = reinterpret_cast<const float4 *>(p)[i];
        v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
    }
}

// ---- chunk tier gate/up: INT8 arena x X8 token rows (qf8_moe_i8.hip:196-262).
// grid (I / RPB, n_exp_max); each lane group keeps its gate and up row in
// registers and dots them with TX tokens at a time.
template <int H, int I>
__global__ void __launch_bounds__(256)
k_cx_gateup_i8x8(const int8_t *__restrict__ Wg, const float *__restrict__ Sg, const int8_t *__restrict__ Wu,
                 const float *__restrict__ Su, const int8_t *__restrict__ xq, const float *__restrict__ xs,
                 float *__restrict__ hidden, const int *__restrict__ exp_slot, const int *__restrict__ exp_ptr,
                 const int *__restrict__ pair_tok, const int *__restrict__ n_exp_dev) {
    constexpr int CPR = H / 16, LPR = lpr_of(CPR), NST = CPR / LPR, RPB = 256 / LPR, TX = 4;
    const int e = blockIdx.y;
    if (e >= *n_exp_dev) return;
    const int l = threadIdx.x % LPR, row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int slot = exp_slot[e], base = exp_ptr[e], n = exp_ptr[e + 1] - base;
    const size_t woff = ((size_t)slot * I + row) * H;
    uint4 wg[NST], wu[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        wg[st] = ld_nt16(Wg + woff + (st * LPR + l) * 16);
        wu[st] = ld_nt16(Wu + woff + (st * LPR + l) * 16);
    }
    const float sg = Sg[(size_t)slot * I + row], su = Su[(size_t)slot * I + row];
    for (int j0 = 0; j0 < n; j0 += TX) {
        int tk[TX];
#pragma unroll
        for (int j = 0; j < TX; j++) tk[j] = pair_tok[base + (j0 + j < n ? j0 + j : j0)];
        uint4 xv[TX][NST];
        float sc[TX][NST];
#pragma unroll
        for (int j = 0; j < TX; j++)
#pragma unroll
            for (int st = 0; st < NST; st++) {
                const int c = st * LPR + l;
                xv[j][st] = *reinterpret_cast<const uint4 *>(xq + (size_t)tk[j] * H + c * 16);
                sc[j][st] = xs[(size_t)tk[j] * (H / 32) + (c >> 1)];
            }
#pragma unroll
        for (int j = 0; j < TX; j++) {
            float ag = 0.0f, au = 0.0f;
#pragma unroll
            for (int st = 0; st < NST; st++) {
                ag = fmaf((float)dot16_i8i8(wg[st], xv[j][st]), sc[j][st], ag);
                au = fmaf((float)dot16_i8i8(wu[st], xv[j][st]), sc[j][st], au);
            }
            ag = group_sum<LPR>(ag);
            au = group_sum<LPR>(au);
            if (l == 0 && j0 + j < n) hidden[(size_t)(base + j0 + j) * I + row] = silu(ag * sg) * (au * su);
        }
    }
}

// ---- chunk tier down: owned partials part[(tok*K + k)][H] = wt * sd * <Wd, h>
// with k the position of the expert in the token's selection
// (qf8_moe_i8.hip:263-311). grid (H / RPB, n_exp_max).
template <int H, int I>
__global__ void __launch_bounds__(256)
k_cx_down_part_i8(const int8_t *__restrict__ Wd, const float *__restrict__ Sd, const float *__restrict__ hidden,
                  const float *__restrict__ pair_wt, const int *__restrict__ pair_tok,
                  const int *__restrict__ exp_slot, const int *__restrict__ exp_ptr,
                  const int *__restrict__ n_exp_dev, const int *__restrict__ sel, int K, float *__restrict__ part) {
    constexpr int CPR = I / 16, LPR = lpr_of(CPR), NST = CPR / LPR, RPB = 256 / LPR, TX = NST == 1 ? 4 : 1;
    const int e = blockIdx.y;
    if (e >= *n_exp_dev) return;
    const int l = threadIdx.x % LPR, row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int slot = exp_slot[e], base = exp_ptr[e], n = exp_ptr[e + 1] - base;
    uint4 w[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) w[st] = ld_nt16(Wd + ((size_t)slot * H + row) * I + (st * LPR + l) * 16);
    const float sd = Sd[(size_t)slot * H + row];
    for (int j0 = 0; j0 < n; j0 += TX) {
        float hv[TX][NST][16];
#pragma unroll
        for (int j = 0; j < TX; j++) {
            const int pj = base + (j0 + j < n ? j0 + j : j0);
#pragma unroll
            for (int st = 0; st < NST; st++) ld_f32x16(hidden + (size_t)pj * I + (st * LPR + l) * 16, hv[j][st]);
        }
#pragma unroll
        for (int j = 0; j < TX; j++) {
            float acc = 0.0f;
#pragma unroll
            for (int st = 0; st < NST; st++) acc = dot16_i8f(w[st], hv[j][st], acc);
            acc = group_sum<LPR>(acc);
            if (l == 0 && j0 + j < n) {
                const int pj = base + j0 + j, tok = pair_tok[pj];
                int k = 0;
                for (int kk = 0; kk < K; kk++)
                    if (sel[(size_t)tok * K + kk] == slot) { k = kk; break; }
                part[((size_t)tok * K + k) * H + row] = pair_wt[pj] * sd * acc;
            }
        }
    }
}

// y[t][i] = sum_k part[t*K + k][i], fixed k order (qf8_moe_i8.hip:312-322).
__global__ void __launch_bounds__(256)
k_cx_combine(const float *__restrict__ part, int K, int H, float *__restrict__ y) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= H) return;
    const float *pt = part + (size_t)t * K * H + i;
    float a = 0.0f;
    for (int k = 0; k < K; k++) a += pt[(size_t)k * H];
    y[(size_t)t * H + i] = a;
}

// Four-card combine: y[i] = ((y0[i] + y1[i]) + y2[i]) + y3[i] (the
// left-to-right sum of k_m8_reduce4, qf_moe_m8_wave64.hip:216-221). VEC: four
// elements per thread in 16-byte accesses (every pointer 16-byte aligned);
// the n % 4 tail elements are done by the first threads of the vector grid.
template <bool VEC>
__global__ void __launch_bounds__(256)
k_cx_reduce4(float *y, const float *y0, const float *y1, const float *y2, const float *y3, int n) {   // y may alias an input
    const int i = blockIdx.x * 256 + threadIdx.x;
    if constexpr (VEC) {
        const int n4 = n >> 2;
        if (i < n4) {
            const float4 a = reinterpret_cast<const float4 *>(y0)[i], b = reinterpret_cast<const float4 *>(y1)[i];
            const float4 c = reinterpret_cast<const float4 *>(y2)[i], d = reinterpret_cast<const float4 *>(y3)[i];
            reinterpret_cast<float4 *>(y)[i] = make_float4(((a.x + b.x) + c.x) + d.x, ((a.y + b.y) + c.y) + d.y,
                                                           ((a.z + b.z) + c.z) + d.z, ((a.w + b.w) + c.w) + d.w);
        }
        const int t = n4 * 4 + i;
        if (i < (n & 3)) y[t] = ((y0[t] + y1[t]) + y2[t]) + y3[t];
    } else {
        if (i < n) y[i] = ((y0[i] + y1[i]) + y2[i]) + y3[i];
    }
}

// ---- NVFP4 weights x fp32 activations -------------------------------------------
// Pair groups: group g covers pairs [ptr[g], ptr[g+1]) of weight slot slot[g];
// ptr == nullptr makes group g the single pair g on activation row 0 (the M=1
// form). s2 tables are indexed by s2_idx[g] when given, else by the slot.
struct PairGroups {
    const int *slot, *ptr, *tok, *n_dev, *s2_idx;
};

// gate/up (qf_nvfp4_wave64.hip:376-404 for M=1, qf_moe_m8_wave64.hip:72-146 for
// M=8): hidden[pair][I] = silu(s2g * Wg.x) * (s2u * Wu.x); slot < 0 -> zeros.
template <int H, int I>
__global__ void __launch_bounds__(256)
k_cx_gateup_f4(const uint8_t *__restrict__ Wg, const uint8_t *__restrict__ Sg, const uint8_t *__restrict__ Wu,
               const uint8_t *__restrict__ Su, const float *__restrict__ s2g, const float *__restrict__ s2u,
               const float *__restrict__ x, float *__restrict__ hidden, PairGroups pg) {
    constexpr int CPR = H / 32, LPR = lpr_of(CPR), NST = CPR / LPR, RPB = 256 / LPR;
    const int g = blockIdx.y;
    if (pg.n_dev && g >= *pg.n_dev) return;
    const int l = threadIdx.x % LPR, row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int slot = pg.slot[g];
    const int base = pg.ptr ? pg.ptr[g] : g, n = pg.ptr ? pg.ptr[g + 1] - base : 1;
    if (slot < 0) {
        if (l == 0)
            for (int j = 0; j < n; j++) hidden[(size_t)(base + j) * I + row] = 0.0f;
        return;
    }
    const int si = pg.s2_idx ? pg.s2_idx[g] : slot;
    const size_t woff = ((size_t)slot * I + row) * (H / 2), soff = ((size_t)slot * I + row) * (H / 16);
    uint4 wg[NST], wu[NST];
    uint32_t bg[NST], bu[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        const int c = st * LPR + l;
        wg[st] = ld_nt16(Wg + woff + c * 16);
        wu[st] = ld_nt16(Wu + woff + c * 16);
        bg[st] = *reinterpret_cast<const uint16_t *>(Sg + soff + c * 2);
        bu[st] = *reinterpret_cast<const uint16_t *>(Su + soff + c * 2);
    }
    const float fg = s2g[si], fu = s2u[si];
    for (int j = 0; j < n; j++) {
        const int tok = pg.tok ? pg.tok[base + j] : 0;
        float ag = 0.0f, au = 0.0f;
#pragma unroll
        for (int st = 0; st < NST; st++) {
            float xv[32];
            const float *xp = x + (size_t)tok * H + (st * LPR + l) * 32;
            ld_f32x16(xp, xv);
            ld_f32x16(xp + 16, xv + 16);
            ag += f4_chunk(wg[st], bg[st], xv);
            au += f4_chunk(wu[st], bu[st], xv);
        }
        ag = group_sum<LPR>(ag);
        au = group_sum<LPR>(au);
        if (l == 0) hidden[(size_t)(base + j) * I + row] = silu(ag * fg) * (au * fu);
    }
}

// M=8 down + weighted accumulate into a pre-zeroed y_partial with atomics
// (qf_moe_m8_wave64.hip:148-211). grid (H / RPB, n_exp_max).
template <int H, int I>
__global__ void __launch_bounds__(256)
k_cx_down_atomic_f4(const uint8_t *__restrict__ Wd, const uint8_t *__restrict__ Sd, const float *__restrict__ s2d,
                    const float *__restrict__ hidden, const float *__restrict__ pair_wt, float *__restrict__ y,
                    PairGroups pg) {
    constexpr int CPR = I / 32, LPR = lpr_of(CPR), NST = CPR / LPR, RPB = 256 / LPR;
    const int g = blockIdx.y;
    if (pg.n_dev && g >= *pg.n_dev) return;
    const int l = threadIdx.x % LPR, row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int slot = pg.slot[g], base = pg.ptr[g], n = pg.ptr[g + 1] - base;
    if (slot < 0) return;
    const size_t woff = ((size_t)slot * H + row) * (I / 2), soff = ((size_t)slot * H + row) * (I / 16);
    uint4 w[NST];
    uint32_t b[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        const int c = st * LPR + l;
        w[st] = ld_nt16(Wd + woff + c * 16);
        b[st] = *reinterpret_cast<const uint16_t *>(Sd + soff + c * 2);
    }
    const float fd = s2d[pg.s2_idx ? pg.s2_idx[g] : slot];
    for (int j = 0; j < n; j++) {
        float acc = 0.0f;
#pragma unroll
        for (int st = 0; st < NST; st++) {
            float hv[32];
            const float *hp = hidden + (size_t)(base + j) * I + (st * LPR + l) * 32;
            ld_f32x16(hp, hv);
            ld_f32x16(hp + 16, hv + 16);
            acc += f4_chunk(w[st], b[st], hv);
        }
        acc = group_sum<LPR>(acc);
        if (l == 0) atomicAdd(&y[(size_t)pg.tok[base + j] * H + row], pair_wt[base + j] * acc * fd);
    }
}

// M=1 down: one writer per output row looping the nexp experts in fixed order,
// y SEEDED (qf_nvfp4_wave64.hip:406-454). The hidden rows are staged in LDS;
// every expert's weight chunk is loaded before the first is used.
template <int H, int I>
__global__ void __launch_bounds__(256)
k_cx_down_seed_f4(const uint8_t *__restrict__ Wd, const uint8_t *__restrict__ Sd, const float *__restrict__ s2d,
                  const float *__restrict__ hidden, const float *__restrict__ wts, float *__restrict__ y,
                  const int *__restrict__ sel, const int *__restrict__ slot_ids, int nexp) {
    constexpr int CPR = I / 32, LPR = lpr_of(CPR), NST = CPR / LPR, RPB = 256 / LPR;
    constexpr int KB = NST == 1 ? kMaxSel : 2;        // experts whose weight chunks are loaded together
    __shared__ __align__(16) float sh[kMaxSel * I];
    const int l = threadIdx.x % LPR, row = blockIdx.x * RPB + threadIdx.x / LPR;
    for (int i = threadIdx.x; i < nexp * I / 4; i += 256)
        reinterpret_cast<float4 *>(sh)[i] = reinterpret_cast<const float4 *>(hidden)[i];
    float total = 0.0f;
    for (int k0 = 0; k0 < nexp; k0 += KB) {
        uint4 w[KB][NST];
        uint32_t b[KB][NST];
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int k = k0 + kb;
            const int sl = k < nexp ? slot_ids[k] : -1, s = sl < 0 ? 0 : sl;
            const size_t woff = ((size_t)s * H + row) * (I / 2), soff = ((size_t)s * H + row) * (I / 16);
#pragma unroll
            for (int st = 0; st < NST; st++) {
                const int c = st * LPR + l;
                w[kb][st] = ld_nt16(Wd + woff + c * 16);
                b[kb][st] = *reinterpret_cast<const uint16_t *>(Sd + soff + c * 2);
            }
        }
        if (k0 == 0) __syncthreads();                 // hidden rows staged
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            const int k = k0 + kb;
            if (k >= nexp) break;
            if (slot_ids[k] < 0) continue;
            float acc = 0.0f;
#pragma unroll
            for (int st = 0; st < NST; st++) acc += f4_chunk(w[kb][st], b[kb][st], sh + k * I + (st * LPR + l) * 32);
            acc = group_sum<LPR>(acc);
            total = fmaf(wts[k], acc * s2d[sel[k]], total);
        }
    }
    if (l == 0) y[row] = total;
}

// ---- INT8 shared expert over T rows of X8 activations (qf8_dense_i8.hip:283-296,
// :346-358). Pass 1, grid (I / RPB + 1, T): gate and up rows -> eg = silu(g)*u,
// eu = u; the last block column computes g1[t] = <gate_inp, x_t>.
template <int H, int I>
__global__ void __launch_bounds__(256)
k_cx_shexp_gu(Qf8I8Mat gate, Qf8I8Mat up, Qf8I8Mat gi, const int8_t *__restrict__ xq,
              const float *__restrict__ xs, float *__restrict__ eg, float *__restrict__ eu, float *__restrict__ g1) {
    constexpr int CPR = H / 16, LPR = lpr_of(CPR), NST = CPR / LPR, RPB = 256 / LPR;
    const int t = blockIdx.y, l = threadIdx.x % LPR, r = threadIdx.x / LPR;
    const bool gate_row = blockIdx.x == I / RPB;
    if (gate_row && r > 0) return;
    const int row = gate_row ? 0 : blockIdx.x * RPB + r;
    const int8_t *wa = gate_row ? gi.w : gate.w + (size_t)row * H;
    const int8_t *wb = gate_row ? gi.w : up.w + (size_t)row * H;
    uint4 va[NST], vb[NST], xv[NST];
    float sc[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        const int c = st * LPR + l;
        va[st] = ld_nt16(wa + c * 16);
        vb[st] = ld_nt16(wb + c * 16);
        xv[st] = *reinterpret_cast<const uint4 *>(xq + (size_t)t * H + c * 16);
        sc[st] = xs[(size_t)t * (H / 32) + (c >> 1)];
    }
    float a = 0.0f, bsum = 0.0f;
#pragma unroll
    for (int st = 0; st < NST; st++) {
        a = fmaf((float)dot16_i8i8(va[st], xv[st]), sc[st], a);
        bsum = fmaf((float)dot16_i8i8(vb[st], xv[st]), sc[st], bsum);
    }
    a = group_sum<LPR>(a);
    bsum = group_sum<LPR>(bsum);
    if (l != 0) return;
    if (gate_row) { g1[t] = a * gi.s[0]; return; }
    const float u = bsum * up.s[row];
    eg[(size_t)t * I + row] = silu(a * gate.s[row]) * u;
    eu[(size_t)t * I + row] = u;
}
// Pass 2, grid (H / RPB, T): ed = sd * <Wd, eg_t>; y[t] += sigmoid(g1[t]) * ed.
template <int H, int I>
__global__ void __launch_bounds__(256)
k_cx_shexp_down(Qf8I8Mat down, const float *__restrict__ eg, const float *__restrict__ g1, float *__restrict__ ed,
                float *__restrict__ y) {
    constexpr int CPR = I / 16, LPR = lpr_of(CPR), NST = CPR / LPR, RPB = 256 / LPR;
    const int t = blockIdx.y, l = threadIdx.x % LPR, row = blockIdx.x * RPB + threadIdx.x / LPR;
    uint4 w[NST];
    float hv[NST][16];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        const int c = st * LPR + l;
        w[st] = ld_nt16(down.w + (size_t)row * I + c * 16);
        ld_f32x16(eg + (size_t)t * I + c * 16, hv[st]);
    }
    float acc = 0.0f;
#pragma unroll
    for (int st = 0; st < NST; st++) acc = dot16_i8f(w[st], hv[st], acc);
    acc = group_sum<LPR>(acc);
    if (l == 0) {
        const float d = acc * down.s[row];
        ed[(size_t)t * H + row] = d;
        y[(size_t)t * H + row] += (1.0f / (1.0f + __expf(-g1[t]))) * d;
    }
}

// ---- NVFP4 -> INT8 arena conversion (semantics of qf8_moe_i8.hip:146-195):
// value k of a row = e2m1(code k) * ue4m3(block scale k/16) * s2, in that
// order; row scale = absmax * (1/127) (1 for an all-zero row); code =
// rint(value * (1/scale)) clamped to +-127. One wave per row: lane l takes the
// 16-byte chunks l, l + 64, ... of the packed row (32 codes and their two
// block scales each), decodes them with the gfx950 fp4 convert at unit scale
// (exact e2m1 values), reduces the row maximum with DPP and writes 32 codes
// per chunk as two 16-byte stores. CPL = chunks per lane (K <= 2048: 1).
template <int CPL>
__global__ void __launch_bounds__(256)
k_f4_rows_to_i8(const uint8_t *__restrict__ W, const uint8_t *__restrict__ S, const float *__restrict__ s2,
                int rows, int K, int8_t *__restrict__ Wo, float *__restrict__ So) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), slot = blockIdx.y;
    if (row >= rows) return;                              // wave-uniform
    const size_t rs = (size_t)slot * rows + row;          // row index in the slot-major arena
    const int nch = K / 32;
    const float gsc = s2[slot];
    float val[CPL][32];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        const int ch = c * 64 + lane;
        if (ch < nch) {
            const uint4 w = *reinterpret_cast<const uint4 *>(W + rs * (K / 2) + (size_t)ch * 16);
            const uint32_t sb = *reinterpret_cast<const uint16_t *>(S + rs * (K / 16) + (size_t)ch * 2);
            const float bs[2] = {e4m3_scale(sb & 0xFFu), e4m3_scale(sb >> 8)};
            const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {                 // word q holds codes 8q .. 8q + 7
                const f32x2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd[q], 1.0f, 0);
                const f32x2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd[q], 1.0f, 1);
                const f32x2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd[q], 1.0f, 2);
                const f32x2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd[q], 1.0f, 3);
                const float e[8] = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
                const float b = bs[q >> 1];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const float v = (e[u] * b) * gsc;
                    val[c][8 * q + u] = v;
                    amax = fmaxf(amax, fabsf(v));
                }
            }
        }
    }
    amax = group_max<64>(amax);
    const float scale = amax > 0.0f ? amax * (1.0f / 127.0f) : 1.0f;
    const float inv = 1.0f / scale;
#pragma unroll
    for (int c = 0; c < CPL; c++) {
        const int ch = c * 64 + lane;
        if (ch < nch) {
            uint32_t pk[8];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                uint32_t word = 0;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int code = min(127, max(-127, (int)rintf(val[c][4 * q + u] * inv)));
                    word |= ((uint32_t)code & 0xFFu) << (8 * u);
                }
                pk[q] = word;
            }
            uint4 *dst = reinterpret_cast<uint4 *>(Wo + rs * K + (size_t)ch * 32);
            dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
        }
    }
    if (lane == 0) So[rs] = scale;
}

// ---- host helpers ------------------------------------------------------------------
int launch_x8(const float *x, int8_t *q, float *sc, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_x8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, q, sc, n);
    return check_launch("qf8_i8_x8");
}

static bool shape_ok(const char *who) {
    if (shape_2048() || shape_2560()) return true;
    set_error(-2, "%s: (hidden, inter) must be (2048, 512) or (2560, 640)", who);
    return false;
}
#define QFM_SHAPE_DISPATCH(KERNEL_CALL)                 \
    do {                                                \
        if (shape_2048()) { constexpr int HH = 2048, II = 512; KERNEL_CALL; } \
        else { constexpr int HH = 2560, II = 640; KERNEL_CALL; }              \
    } while (0)

}  // namespace qfm

using namespace qfm;

extern "C" {

int qf8_i8_x8_ex(const float *x, int8_t *q, float *sc, int n, hipStream_t s) {
    if (!x || !q || !sc || n < 32 || n % 32) { set_error(-1, "qf8_i8_x8: need n a positive multiple of 32"); return -1; }
    return launch_x8(x, q, sc, n, s);
}

void qf8_i8_x8(const float *x, int8_t *q, float *sc, int n, hipStream_t s) {
    (void)qf8_i8_x8_ex(x, q, sc, n, s);
}

int qf8_i8_csr_build_ex(const int *sel, const float *wt, int T, int *exp_slot, int *exp_ptr, int *pair_tok,
                         float *pair_wt, int *counts, hipStream_t s) {
    const int K = g_cfg.K, E = g_cfg.E;
    if (!sel || !wt || !exp_slot || !exp_ptr || !pair_tok || !pair_wt || !counts || T < 1 || E > 1024 ||
        (long)T * K > (1L << 30)) {
        set_error(-1, "qf8_i8_csr_build: bad arguments"); return -1;
    }
    const int P = T * K;
    hipLaunchKernelGGL(k_cb_count, dim3(1), dim3(1024), 0, s, sel, P, E, exp_slot, exp_ptr, counts);
    hipLaunchKernelGGL(k_cb_scatter, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, s, sel, wt, P, K, E, exp_slot,
                       exp_ptr, counts, pair_tok, pair_wt);
    return check_launch("qf8_i8_csr_build");
}

void qf8_i8_csr_build(const int *sel, const float *wt, int T, int *exp_slot, int *exp_ptr, int *pair_tok,
                      float *pair_wt, int *counts, hipStream_t s) {
    (void)qf8_i8_csr_build_ex(sel, wt, T, exp_slot, exp_ptr, pair_tok, pair_wt, counts, s);
}

int qf8_i8_experts_chunk_ex(const Qf4ExpCache *c, const int8_t *xq, const float *xs, float *hidden, int8_t *h8q,
                             float *h8s, const int *exp_slot, const int *exp_ptr, const int *pair_tok,
                             const float *pair_wt, const int *n_exp_dev, int n_exp_max, int n_pairs_max, const int *sel,
                             float *part, int T, float *y, hipStream_t s) {
    (void)h8q; (void)h8s; (void)n_pairs_max;
    if (!shape_ok("qf8_i8_experts_chunk")) return -2;
    if (!c || !c->i8_gate || !c->i8_up || !c->i8_down || !xq || !xs || !hidden || !exp_slot || !exp_ptr ||
        !pair_tok || !pair_wt || !n_exp_dev || !sel || !part || !y || T < 1 || n_exp_max < 1 ||
        n_exp_max > c->slots) {
        set_error(-1, "qf8_i8_experts_chunk: bad arguments"); return -1;
    }
    const int K = g_cfg.K;
    QFM_SHAPE_DISPATCH({
        hipLaunchKernelGGL((k_cx_gateup_i8x8<HH, II>), dim3(II / (256 / lpr_of(HH / 16)), n_exp_max), dim3(256), 0,
                           s, c->i8_gate, c->i8s_gate, c->i8_up, c->i8s_up, xq, xs, hidden, exp_slot, exp_ptr,
                           pair_tok, n_exp_dev);
        hipLaunchKernelGGL((k_cx_down_part_i8<HH, II>), dim3(HH / (256 / lpr_of(II / 16)), n_exp_max), dim3(256), 0,
                           s, c->i8_down, c->i8s_down, hidden, pair_wt, pair_tok, exp_slot, exp_ptr, n_exp_dev, sel,
                           K, part);
        hipLaunchKernelGGL(k_cx_combine, dim3((HH + 255) / 256, T), dim3(256), 0, s, part, K, HH, y);
    });
    return check_launch("qf8_i8_experts_chunk");
}

void qf8_i8_experts_chunk(const Qf4ExpCache *c, const int8_t *xq, const float *xs, float *hidden, int8_t *h8q,
                          float *h8s, const int *exp_slot, const int *exp_ptr, const int *pair_tok,
                          const float *pair_wt, const int *n_exp_dev, int n_exp_max, int n_pairs_max, const int *sel,
                          float *part, int T, float *y, hipStream_t s) {
    (void)qf8_i8_experts_chunk_ex(c, xq, xs, hidden, h8q, h8s, exp_slot, exp_ptr, pair_tok, pair_wt, n_exp_dev, n_exp_max, n_pairs_max, sel, part, T, y, s);
}

int qf5_nvfp4_gateup_all_launch_ex(const uint8_t *Wg, const uint8_t *Sg, const uint8_t *Wu, const uint8_t *Su,
                                    const float *x, float *hidden, const float *s2g_dev, const float *s2u_dev,
                                    const int *sel_ids, const int *slot_ids, int nexp, hipStream_t stream) {
    if (!shape_ok("qf5_nvfp4_gateup_all_launch")) return -2;
    if (!Wg || !Sg || !Wu || !Su || !x || !hidden || !s2g_dev || !s2u_dev || !sel_ids || !slot_ids || nexp < 1 ||
        nexp > kMaxSel) {
        set_error(-1, "qf5_nvfp4_gateup_all_launch: bad arguments"); return -1;
    }
    const PairGroups pg{slot_ids, nullptr, nullptr, nullptr, sel_ids};
    QFM_SHAPE_DISPATCH(hipLaunchKernelGGL((k_cx_gateup_f4<HH, II>), dim3(II / (256 / lpr_of(HH / 32)), nexp),
                                          dim3(256), 0, stream, Wg, Sg, Wu, Su, s2g_dev, s2u_dev, x, hidden, pg));
    return check_launch("qf5_nvfp4_gateup_all_launch");
}

void qf5_nvfp4_gateup_all_launch(const uint8_t *Wg, const uint8_t *Sg, const uint8_t *Wu, const uint8_t *Su,
                                 const float *x, float *hidden, const float *s2g_dev, const float *s2u_dev,
                                 const int *sel_ids, const int *slot_ids, int nexp, hipStream_t stream) {
    (void)qf5_nvfp4_gateup_all_launch_ex(Wg, Sg, Wu, Su, x, hidden, s2g_dev, s2u_dev, sel_ids, slot_ids, nexp, stream);
}

int qf5_nvfp4_downacc_all_launch_ex(const uint8_t *Wd, const uint8_t *Sd, const float *hidden, const float *wts,
                                     float *y, const float *s2d_dev, const int *sel_ids, const int *slot_ids, int nexp,
                                     hipStream_t stream) {
    if (!shape_ok("qf5_nvfp4_downacc_all_launch")) return -2;
    if (!Wd || !Sd || !hidden || !wts || !y || !s2d_dev || !sel_ids || !slot_ids || nexp < 1 || nexp > kMaxSel) {
        set_error(-1, "qf5_nvfp4_downacc_all_launch: bad arguments"); return -1;
    }
    QFM_SHAPE_DISPATCH(hipLaunchKernelGGL((k_cx_down_seed_f4<HH, II>), dim3(HH / (256 / lpr_of(II / 32))), dim3(256),
                                          0, stream, Wd, Sd, s2d_dev, hidden, wts, y, sel_ids, slot_ids, nexp));
    return check_launch("qf5_nvfp4_downacc_all_launch");
}

void qf5_nvfp4_downacc_all_launch(const uint8_t *Wd, const uint8_t *Sd, const float *hidden, const float *wts,
                                  float *y, const float *s2d_dev, const int *sel_ids, const int *slot_ids, int nexp,
                                  hipStream_t stream) {
    (void)qf5_nvfp4_downacc_all_launch_ex(Wd, Sd, hidden, wts, y, s2d_dev, sel_ids, slot_ids, nexp, stream);
}

int qf5_nvfp4_moe_all_ex(const uint8_t *Wg, const uint8_t *Sg, const uint8_t *Wu, const uint8_t *Su,
                          const uint8_t *Wd, const uint8_t *Sd, const float *x, float *hidden, float *y,
                          const float *s2g_dev, const float *s2u_dev, const float *s2d_dev, const float *wts,
                          const int *sel_ids, const int *slot_ids, int nexp, hipStream_t stream) {
    const int rc = qf5_nvfp4_gateup_all_launch_ex(Wg, Sg, Wu, Su, x, hidden, s2g_dev, s2u_dev, sel_ids, slot_ids, nexp,
                                                  stream);
    if (rc) return rc;
    return qf5_nvfp4_downacc_all_launch_ex(Wd, Sd, hidden, wts, y, s2d_dev, sel_ids, slot_ids, nexp, stream);
}

void qf5_nvfp4_moe_all(const uint8_t *Wg, const uint8_t *Sg, const uint8_t *Wu, const uint8_t *Su,
                       const uint8_t *Wd, const uint8_t *Sd, const float *x, float *hidden, float *y,
                       const float *s2g_dev, const float *s2u_dev, const float *s2d_dev, const float *wts,
                       const int *sel_ids, const int *slot_ids, int nexp, hipStream_t stream) {
    (void)qf5_nvfp4_moe_all_ex(Wg, Sg, Wu, Su, Wd, Sd, x, hidden, y, s2g_dev, s2u_dev, s2d_dev, wts, sel_ids, slot_ids, nexp, stream);
}

int qf5_m8_gateup_ex(const uint8_t *Wg, const uint8_t *Sg, const uint8_t *Wu, const uint8_t *Su,
                      const float *s2g_res, const float *s2u_res, const float *x, float *hidden, const Qf5M8Route *rt,
                      hipStream_t stream) {
    if (!shape_ok("qf5_m8_gateup")) return -2;
    if (!Wg || !Sg || !Wu || !Su || !s2g_res || !s2u_res || !x || !hidden || !rt || !rt->n_exp_dev ||
        !rt->exp_slot || !rt->exp_ptr || !rt->pair_tok || rt->n_exp_max < 1 || rt->n_exp_max > 65535) {
        set_error(-1, "qf5_m8_gateup: bad arguments"); return -1;
    }
    const PairGroups pg{rt->exp_slot, rt->exp_ptr, rt->pair_tok, rt->n_exp_dev, nullptr};
    QFM_SHAPE_DISPATCH(hipLaunchKernelGGL((k_cx_gateup_f4<HH, II>), dim3(II / (256 / lpr_of(HH / 32)), rt->n_exp_max),
                                          dim3(256), 0, stream, Wg, Sg, Wu, Su, s2g_res, s2u_res, x, hidden, pg));
    return check_launch("qf5_m8_gateup");
}

void qf5_m8_gateup(const uint8_t *Wg, const uint8_t *Sg, const uint8_t *Wu, const uint8_t *Su,
                   const float *s2g_res, const float *s2u_res, const float *x, float *hidden, const Qf5M8Route *rt,
                   hipStream_t stream) {
    (void)qf5_m8_gateup_ex(Wg, Sg, Wu, Su, s2g_res, s2u_res, x, hidden, rt, stream);
}

int qf5_m8_downacc_ex(const uint8_t *Wd, const uint8_t *Sd, const float *s2d_res, const float *hidden,
                       float *y_partial, const Qf5M8Route *rt, hipStream_t stream) {
    if (!shape_ok("qf5_m8_downacc")) return -2;
    if (!Wd || !Sd || !s2d_res || !hidden || !y_partial || !rt || !rt->n_exp_dev || !rt->exp_slot || !rt->exp_ptr ||
        !rt->pair_tok || !rt->pair_wt || rt->n_exp_max < 1 || rt->n_exp_max > 65535) {
        set_error(-1, "qf5_m8_downacc: bad arguments"); return -1;
    }
    const PairGroups pg{rt->exp_slot, rt->exp_ptr, rt->pair_tok, rt->n_exp_dev, nullptr};
    QFM_SHAPE_DISPATCH(hipLaunchKernelGGL((k_cx_down_atomic_f4<HH, II>), dim3(HH / (256 / lpr_of(II / 32)),
                                          rt->n_exp_max), dim3(256), 0, stream, Wd, Sd, s2d_res, hidden, rt->pair_wt,
                                          y_partial, pg));
    return check_launch("qf5_m8_downacc");
}

void qf5_m8_downacc(const uint8_t *Wd, const uint8_t *Sd, const float *s2d_res, const float *hidden,
                    float *y_partial, const Qf5M8Route *rt, hipStream_t stream) {
    (void)qf5_m8_downacc_ex(Wd, Sd, s2d_res, hidden, y_partial, rt, stream);
}

int qf5_m8_reduce4_ex(float *y_out, const float *y0, const float *y1, const float *y2, const float *y3, int n,
                       hipStream_t s) {
    if (n < 0 || (n > 0 && (!y_out || !y0 || !y1 || !y2 || !y3))) { set_error(-1, "qf5_m8_reduce4: bad arguments"); return -1; }
    if (n == 0) return 0;
    const uintptr_t al = reinterpret_cast<uintptr_t>(y_out) | reinterpret_cast<uintptr_t>(y0) |
                         reinterpret_cast<uintptr_t>(y1) | reinterpret_cast<uintptr_t>(y2) |
                         reinterpret_cast<uintptr_t>(y3);
    if ((al & 15) == 0) {
        const int n4 = n >> 2, nb = (n4 > (n & 3) ? n4 : (n & 3)) + 255;
        hipLaunchKernelGGL(k_cx_reduce4<true>, dim3((unsigned)(nb / 256)), dim3(256), 0, s, y_out, y0, y1, y2, y3, n);
    } else {
        hipLaunchKernelGGL(k_cx_reduce4<false>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y_out, y0, y1, y2,
                           y3, n);
    }
    return check_launch("qf5_m8_reduce4");
}

void qf5_m8_reduce4(float *y_out, const float *y0, const float *y1, const float *y2, const float *y3, int n,
                    hipStream_t s) {
    (void)qf5_m8_reduce4_ex(y_out, y0, y1, y2, y3, n, s);
}

int qf5_m8_build_csr_ex(const int *sel_dev, const float *wt_dev, int M, int K, int card, int epc, int il, int *exp_slot,
                         int *exp_ptr, int *pair_tok, float *pair_wt, int *counts, hipStream_t s) {
    if (!sel_dev || !wt_dev || !exp_slot || !exp_ptr || !pair_tok || !pair_wt || !counts || M < 1 || K < 1 ||
        M * K > 1024 || card < 0 || epc < 1 || il < 0 || (card + 1) * epc > 1024) {
        set_error(-1, "qf5_m8_build_csr: bad arguments (M*K <= 1024, experts < 1024)"); return -1;
    }
    hipLaunchKernelGGL(k_m8_csr, dim3(1), dim3(1024), 0, s, sel_dev, wt_dev, M * K, K, card * epc, card * epc + epc,
                       il * epc, exp_slot, exp_ptr, pair_tok, pair_wt, counts);
    return check_launch("qf5_m8_build_csr");
}

void qf5_m8_build_csr(const int *sel_dev, const float *wt_dev, int M, int K, int card, int epc, int il, int *exp_slot,
                      int *exp_ptr, int *pair_tok, float *pair_wt, int *counts, hipStream_t s) {
    (void)qf5_m8_build_csr_ex(sel_dev, wt_dev, M, K, card, epc, il, exp_slot, exp_ptr, pair_tok, pair_wt, counts, s);
}

static bool mat_ok(const Qf8I8Mat *m, int rows, int K) {
    return m && m->w && m->s && m->rows >= rows && m->K == K;
}

int qf8_i8_shexp_rows(const Qf8I8Mat *gate, const Qf8I8Mat *up, const Qf8I8Mat *gate_inp, const Qf8I8Mat *down,
                      const int8_t *xq, const float *xs, float *eg, float *eu, float *g1, float *ed, int8_t *e8q,
                      float *e8s, float *y2560, int T, hipStream_t s) {
    (void)e8q; (void)e8s;
    if (!shape_ok("qf8_i8_shexp_rows")) return -2;
    const int H = g_cfg.H, I = g_cfg.I;
    if (!mat_ok(gate, I, H) || !mat_ok(up, I, H) || !mat_ok(gate_inp, 1, H) || !mat_ok(down, H, I) || !xq || !xs ||
        !eg || !eu || !g1 || !ed || !y2560 || T < 1 || T > 65535) {
        set_error(-1, "qf8_i8_shexp_rows: bad arguments"); return -1;
    }
    QFM_SHAPE_DISPATCH({
        hipLaunchKernelGGL((k_cx_shexp_gu<HH, II>), dim3(II / (256 / lpr_of(HH / 16)) + 1, T), dim3(256), 0, s,
                           *gate, *up, *gate_inp, xq, xs, eg, eu, g1);
        hipLaunchKernelGGL((k_cx_shexp_down<HH, II>), dim3(HH / (256 / lpr_of(II / 16)), T), dim3(256), 0, s, *down,
                           eg, g1, ed, y2560);
    });
    return check_launch("qf8_i8_shexp_rows");
}

int qf8_i8_shexp_m1_ex(const Qf8I8Mat *gate, const Qf8I8Mat *up, const Qf8I8Mat *gate_inp, const Qf8I8Mat *down,
                        const int8_t *xq, const float *xs, float *eg, float *eu, float *g1, float *ed, int8_t *e8q,
                        float *e8s, float *y2560, hipStream_t s) {
    return qf8_i8_shexp_rows(gate, up, gate_inp, down, xq, xs, eg, eu, g1, ed, e8q, e8s, y2560, 1, s);
}

void qf8_i8_shexp_m1(const Qf8I8Mat *gate, const Qf8I8Mat *up, const Qf8I8Mat *gate_inp, const Qf8I8Mat *down,
                     const int8_t *xq, const float *xs, float *eg, float *eu, float *g1, float *ed, int8_t *e8q,
                     float *e8s, float *y2560, hipStream_t s) {
    (void)qf8_i8_shexp_m1_ex(gate, up, gate_inp, down, xq, xs, eg, eu, g1, ed, e8q, e8s, y2560, s);
}

// one matrix of nslots slots: rows of K codes, four rows per block
static void f4_rows_to_i8(const uint8_t *W, const uint8_t *S, const float *s2, int rows, int K, int nslots,
                          int8_t *Wo, float *So, hipStream_t s) {
    const dim3 grid((unsigned)((rows + 3) / 4), (unsigned)nslots);
    if (K / 32 <= 64) hipLaunchKernelGGL(k_f4_rows_to_i8<1>, grid, dim3(256), 0, s, W, S, s2, rows, K, Wo, So);
    else hipLaunchKernelGGL(k_f4_rows_to_i8<2>, grid, dim3(256), 0, s, W, S, s2, rows, K, Wo, So);
}

static int i8_build_range(Qf4ExpCache *c, int src_slot, int dst_slot, int s2_index, int nslots, hipStream_t s) {
    const int H = g_cfg.H, I = g_cfg.I;
    const size_t gw = (size_t)I * H;                 // elements per matrix (all three)
    f4_rows_to_i8(c->w_gate + src_slot * (gw / 2), c->s_gate + src_slot * (gw / 16), c->s2g_dev + s2_index, I, H,
                  nslots, c->i8_gate + dst_slot * gw, c->i8s_gate + (size_t)dst_slot * I, s);
    f4_rows_to_i8(c->w_up + src_slot * (gw / 2), c->s_up + src_slot * (gw / 16), c->s2u_dev + s2_index, I, H, nslots,
                  c->i8_up + dst_slot * gw, c->i8s_up + (size_t)dst_slot * I, s);
    f4_rows_to_i8(c->w_down + src_slot * (gw / 2), c->s_down + src_slot * (gw / 16), c->s2d_dev + s2_index, H, I,
                  nslots, c->i8_down + dst_slot * gw, c->i8s_down + (size_t)dst_slot * H, s);
    return check_launch("qf8_i8_build") ? -1 : 0;
}

int qf8_i8_build(Qf4ExpCache *c, hipStream_t s) {
    if (!c || !c->i8_gate || !c->w_gate || !c->s2g_dev || !c->i8_up || !c->i8_down || !c->w_up || !c->w_down ||
        !c->s_gate || !c->s_up || !c->s_down || !c->s2u_dev || !c->s2d_dev || c->slots < 1 || c->slots > 65535 ||
        !shape_ok("qf8_i8_build"))
        return -1;
    if (c->nv_ring) {   // the NVFP4 arrays hold only the staging ring, not every slot
        set_error(-1, "qf8_i8_build: the arena's NVFP4 arrays are a %d-slot staging ring; use qf8_i8_build_slot",
                  c->nv_ring);
        return -1;
    }
    return i8_build_range(c, 0, 0, 0, c->slots, s);
}

int qf8_i8_build_slot(Qf4ExpCache *c, int src_slot, int dst_slot, int expert, hipStream_t s) {
    if (!c || !c->i8_gate || !c->w_gate || !c->s2g_dev || !c->i8_up || !c->i8_down || !c->w_up || !c->w_down ||
        !c->s_gate || !c->s_up || !c->s_down || !c->s2u_dev || !c->s2d_dev || src_slot < 0 || dst_slot < 0 ||
        src_slot >= (c->nv_ring ? c->nv_ring : c->slots) || dst_slot >= c->slots || expert < 0 || expert >= g_cfg.E ||
        !shape_ok("qf8_i8_build_slot"))
        return -1;
    return i8_build_range(c, src_slot, dst_slot, expert, 1, s);
}

}  // extern "C"
