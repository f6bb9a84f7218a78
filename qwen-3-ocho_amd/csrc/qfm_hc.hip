// qfm_hc.hip -- dense INT8 x X8 projections, the FFN-side hyper-connection
// pre-mixer and the residual-stream inject (contracts in include/qf_dense.h).
//
// k_gemv_i8x8<LPR, NST>: LPR lanes per weight row, NST 16-byte steps per
// lane (K = 16 * LPR * NST); each lane keeps its NST weight words in
// registers and reuses them for every activation row of its block's token
// tile. Block dots are exact int32 (sdot4), scaled by the 32-value block
// scale and accumulated in fp32, then summed over the LPR lanes with DPP.
//
// One row (T = 1) runs in one launch, k_hc_one: slice blocks, each of which
// norms one stream, X8-codes one K slice of it (1024 values, 512 at H = 2560)
// and publishes the partial dots of 16 (32) down / inject rows over that
// slice (and, in the first
// row group, the slice's normed values) as tagged words, followed by up blocks
// of 64 outputs that wait for those words, sum the partials in slice order and
// run the up GEMV, the combine and X8(mixed) (hc_up_body). T rows run in two
// launches:
//   k_hc_norm_down  one wave per down (silu(v/4)) or inject (2 sigmoid(v/4))
//                   row, 2 rows per block; every block recomputes the fused
//                   inject of the previous mixer, the zero-centred RMS norm
//                   and X8(normed) into LDS, block 0 stores them;
//   k_hc_up_combine one block per 32 outputs j: X8(hc_d) into LDS (every
//                   block; block 0 also stores it), the 4 x 32 up rows
//                   {c*H + j} of the up GEMV, the sigmoid-weighted mean over
//                   the 4 streams and X8(mixed) of the 32 values, and the
//                   residual's fused inject for those 4 x 32 entries.
#include <mutex>

#include "qfm_internal.h"
#include "qfm_dev.h"
#include "../../include/qf_dense.h"

namespace qfm {

struct GemvMat {
    const int8_t *w;
    const float *s;
    float *y;
    int rows, act;
};
struct GemvBatch {
    GemvMat d[4];
    int n, K;
};

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int dot16_i8i8(const i32x4 w, const i32x4 x) {
    int d = __builtin_amdgcn_sdot4(w.x, x.x, 0, false);
    d = __builtin_amdgcn_sdot4(w.y, x.y, d, false);
    d = __builtin_amdgcn_sdot4(w.z, x.z, d, false);
    return __builtin_amdgcn_sdot4(w.w, x.w, d, false);
}

__device__ __forceinline__ float gemv_act(float v, int act) {
    if (act == 1) {
        const float q = v * 0.25f;
        return q / (1.0f + expf(-q));
    }
    if (act == 2) return 2.0f / (1.0f + expf(-v * 0.25f));
    return v;
}

// X8 of one value per lane over aligned 32-lane groups (qf8_i8_x8's rule)
__device__ __forceinline__ int x8_code(float v, float &scale) {
    const float mx = group_max<32>(fabsf(v));
    scale = mx > 0.0f ? mx * (1.0f / 127.0f) : 1.0f;
    return min(127, max(-127, (int)rintf(v / scale)));
}

template <int LPR, int NST>
__global__ void __launch_bounds__(256)
k_gemv_i8x8(GemvBatch b, const int8_t *__restrict__ xq, const float *__restrict__ xs, int T, int tpb) {
    constexpr int K = LPR * 16 * NST, RPB = 256 / LPR;
    const int mi = blockIdx.y;                                   // select without indexing the argument block
    const GemvMat d = mi == 0 ? b.d[0] : mi == 1 ? b.d[1] : mi == 2 ? b.d[2] : b.d[3];
    if ((int)blockIdx.x * RPB >= d.rows) return;                 // block-uniform
    const int l = threadIdx.x % LPR;
    const int row = blockIdx.x * RPB + threadIdx.x / LPR;
    const bool live = row < d.rows;
    const int8_t *wr = d.w + (size_t)(live ? row : 0) * K + l * 16;
    i32x4 w[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) w[st] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wr + st * LPR * 16));
    const float rs = live ? d.s[row] : 0.0f;
    const int t_end = min(T, (int)(blockIdx.z + 1) * tpb);
    for (int t = blockIdx.z * tpb; t < t_end; t++) {
        const int8_t *xr = xq + (size_t)t * K;
        const float *sr = xs + (size_t)t * (K / 32);
        float acc = 0.0f;
#pragma unroll
        for (int st = 0; st < NST; st++) {
            const int e0 = st * LPR * 16 + l * 16;
            acc = fmaf((float)dot16_i8i8(w[st], *reinterpret_cast<const i32x4 *>(xr + e0)), sr[e0 >> 5], acc);
        }
        acc = group_sum<LPR>(acc);
        if (live && l == 0) d.y[(size_t)t * d.rows + row] = gemv_act(acc * rs, d.act);
    }
}

// ---- hand-off area of the one-launch pre-mixer (T = 1) -----------------------------
// 64-bit words (fp32 bits | tag << 32, agent-scope stores): [0, 20 * 324) the
// partial dots of the down / inject rows, slice s of row r at s * 324 + r
// (slices 0 .. NS - 1, NS = 4H / KS, at most 20), then normed [4H]. The call's tag is
// next_tag(epoch): every block reads epoch at its start and the last up block
// to finish reading its words advances it (arrivals counts them), so the next
// call, stream-ordered after this one, uses the next tag and no word needs
// clearing. The array starts zeroed (epoch 0, no live tag); timeouts counts
// the words whose bounded wait ran out (0 unless something is badly wrong).
// K slice of a slice block: 1024 values where H allows, else 512 (H = 2560)
__host__ __device__ constexpr int hc_slice_of(int H) { return H % 1024 == 0 ? 1024 : 512; }
constexpr int kHcRows = QF8_HCL + QF8_HCC;                 // partial words per slice
constexpr int kHcNormed = kHcRows * (4 * 2560 / 512);      // the most slices (H = 2560)
constexpr int kHcWordsMax = kHcNormed + 4 * 2560;
struct HcArea {
    uint32_t epoch, arrivals, timeouts, pad[61];
    unsigned long long w[kHcWordsMax];
};
static __device__ __align__(256) HcArea hc_area;

__device__ __forceinline__ unsigned long long hc_word(float v, uint32_t tag) {
    return (unsigned long long)__float_as_uint(v) | ((unsigned long long)tag << 32);
}

// Norm + X8 + down/inject GEMV in one launch. grid (rows / RB, T), 1024
// threads: block b owns weight rows RB b .. RB b + RB - 1 (down rows first,
// then the inject rows), the 16-byte steps of each row dealt round-robin to
// 16 / RB waves;
// each thread issues its residual loads and then its weight loads.
// Every block then recomputes the residual's norm and X8 codes for all 4
// streams into LDS: thread c * 256 + t owns elements i * 256 + t of stream c
// and sums them in order, then each wave and the four waves of a stream are
// reduced (the reference's partition and order, so every block gets the same
// codes); block 0 also stores normed / X8 (the API outputs); then the row's
// partial dots run against the LDS codes and are summed in wave order. The
// fused inject's updated residual is not stored here (other blocks still read
// R): k_hc_up_combine stores it.

template <int NV, int RB>
__global__ void __launch_bounds__(1024)
k_hc_norm_down(const float *__restrict__ R, const uint16_t *__restrict__ wn, const float *__restrict__ y_prev,
               const float *__restrict__ inj_prev, const int8_t *__restrict__ Wd, const float *__restrict__ Sd,
               const int8_t *__restrict__ Wi, const float *__restrict__ Si, float *__restrict__ hc_d,
               float *__restrict__ inj, float *__restrict__ normed, int8_t *__restrict__ q, float *__restrict__ sc) {
    constexpr int H = NV * 256, RS = 4 * H, NST = RS / 1024;
    __shared__ __align__(16) int8_t s_q[RS];
    __shared__ float s_s[RS / 32];
    __shared__ float red[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = tid >> 8, t256 = tid & 255;                  // stream, thread within the stream
    const size_t t = blockIdx.y;
    // RB rows per block, each row's 16-byte steps dealt round-robin to WPR waves
    constexpr int WPR = 16 / RB;
    constexpr int NSQ = (NST + WPR - 1) / WPR;                 // steps per wave (the last may be short)
    const int kq = wave % WPR, rloc = wave / WPR;
    const int row = blockIdx.x * RB + rloc;
    const int nrow = QF8_HCL + (Wi ? QF8_HCC : 0);
    const bool live = row < nrow;
    const bool is_inj = row >= QF8_HCL;
    const int8_t *wr = (is_inj ? Wi + (size_t)(live ? row - QF8_HCL : 0) * RS : Wd + (size_t)(live ? row : 0) * RS) +
                       lane * 16;
    // this thread's residual values (with the previous mixer's inject) and norm
    // weights first (memory retires loads in issue order, so the norm then
    // waits only for these), then the row's weights, which stream meanwhile
    const size_t base = t * RS + (size_t)c * H;
    float v[NV], yv[NV];
    uint16_t wb[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        v[i] = R[base + i * 256 + t256];
        wb[i] = wn[(size_t)c * H + i * 256 + t256];
    }
    const float sj = y_prev ? inj_prev[t * QF8_HCC + c] : 0.0f;
    if (y_prev)                                                // uniform
#pragma unroll
        for (int i = 0; i < NV; i++) yv[i] = y_prev[t * H + i * 256 + t256];
    i32x4 w[NSQ];
#pragma unroll
    for (int j = 0; j < NSQ; j++) {
        const int st = kq + WPR * j;
        if (st < NST) w[j] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wr + st * 1024));
    }
    if (y_prev)
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] = fmaf(sj, yv[i], v[i]);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) acc = fmaf(v[i], v[i], acc);
    acc = group_sum<64>(acc);
    if (lane == 0) red[wave] = acc;
    __syncthreads();
    const float rstd = rsqrtf((red[4 * c] + red[4 * c + 1] + red[4 * c + 2] + red[4 * c + 3]) / (float)H + 1e-6f);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int e = c * H + i * 256 + t256;                  // 32 consecutive e per half-wave
        const float nv = v[i] * rstd * (1.0f + bf16_to_f32(wb[i]));
        float s1;
        const int qi = x8_code(nv, s1);
        s_q[e] = (int8_t)qi;
        if ((tid & 31) == 0) s_s[e >> 5] = s1;
        if (blockIdx.x == 0) {
            normed[t * RS + e] = nv;
            q[t * RS + e] = (int8_t)qi;
            if ((tid & 31) == 0) sc[(t * RS + e) >> 5] = s1;
        }
    }
    __syncthreads();
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < NSQ; j++) {
        const int st = kq + WPR * j;
        if (st < NST) {
            const int e0 = st * 1024 + lane * 16;
            a = fmaf((float)dot16_i8i8(w[j], *reinterpret_cast<const i32x4 *>(s_q + e0)), s_s[e0 >> 5], a);
        }
    }
    a = group_sum<64>(a);
    __shared__ float part[RB][WPR];
    if (lane == 0) part[rloc][kq] = a;
    __syncthreads();
    if (tid < RB && blockIdx.x * RB + tid < nrow) {            // one lane per row: its WPR parts in order
        const int r = blockIdx.x * RB + tid;
        float sum = part[tid][0];
#pragma unroll
        for (int q = 1; q < WPR; q++) sum += part[tid][q];
        if (r >= QF8_HCL) inj[t * QF8_HCC + r - QF8_HCL] = gemv_act(sum * Si[r - QF8_HCL], 2);
        else hc_d[t * QF8_HCL + r] = gemv_act(sum * Sd[r], 1);
    }
}

// grid (H / 32, T), 512 threads: 8 waves x 16 row groups of 4 lanes = 128 up rows
template <int H>
__global__ void __launch_bounds__(512)
k_hc_up_combine(const int8_t *__restrict__ Wu, const float *__restrict__ Su, const float *__restrict__ hc_d,
                const float *__restrict__ normed, float *__restrict__ hcy, float *__restrict__ mixed,
                int8_t *__restrict__ xq_out, float *__restrict__ xs_out, int8_t *__restrict__ d8q,
                float *__restrict__ d8s, float *__restrict__ R, const float *__restrict__ y_prev,
                const float *__restrict__ inj_prev, uint16_t *__restrict__ xb_out) {
    constexpr int L = QF8_HCL, RS = 4 * H;
    __shared__ __align__(16) int8_t s_q[L];
    __shared__ float s_s[L / 32];
    __shared__ float s_h[4][32];
    const int tid = threadIdx.x;
    const size_t t = blockIdx.y;
    const int j0 = blockIdx.x * 32;
    // this block's up rows {c*H + j} and, for the combine, the normed values:
    // issued before the X8 prologue so their latency overlaps it
    const int lane = tid & 63, l = lane & 3;
    const int li = (tid >> 6) * 16 + (lane >> 2);             // 0..127
    const int c = li >> 5, jj = li & 31;
    const size_t row = (size_t)c * H + j0 + jj;
    const int8_t *wr = Wu + row * L + l * 16;
    i32x4 wv[L / 64];
#pragma unroll
    for (int st = 0; st < L / 64; st++) wv[st] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wr + st * 64));
    const float su = Su[row];
    float nrm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (tid < 32)
#pragma unroll
        for (int cc = 0; cc < 4; cc++) nrm[cc] = normed[t * RS + (size_t)cc * H + j0 + tid];
    // the previous mixer's inject into the residual (k_hc_norm_down read R unchanged)
    if (y_prev && tid < 128) {
        const int rc = tid >> 5, rj = j0 + (tid & 31);
        float *rp = R + t * RS + (size_t)rc * H + rj;
        *rp = fmaf(inj_prev[t * QF8_HCC + rc], y_prev[t * H + rj], *rp);
    }
    if (tid < L) {                                            // threads 0..319: five whole waves
        float s1;
        const int qi = x8_code(hc_d[t * L + tid], s1);
        s_q[tid] = (int8_t)qi;
        if ((tid & 31) == 0) s_s[tid >> 5] = s1;
        if (blockIdx.x == 0) {
            d8q[t * L + tid] = (int8_t)qi;
            if ((tid & 31) == 0) d8s[t * (L / 32) + (tid >> 5)] = s1;
        }
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int st = 0; st < L / 64; st++) {
        const int e0 = st * 64 + l * 16;
        acc = fmaf((float)dot16_i8i8(wv[st], *reinterpret_cast<const i32x4 *>(s_q + e0)), s_s[e0 >> 5], acc);
    }
    acc = group_sum<4>(acc);
    if (l == 0) {
        const float hv = acc * su;
        hcy[t * RS + row] = hv;
        s_h[c][jj] = hv;
    }
    __syncthreads();
    if (tid < 32) {
        const int j = j0 + tid;
        float sum = 0.0f;
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const float m = 1.0f / (1.0f + expf(-s_h[cc][tid]));
            sum = fmaf(m, nrm[cc], sum);
        }
        const float v = sum * 0.25f;
        mixed[t * H + j] = v;
        if (xb_out) xb_out[t * H + j] = f32_to_bf16(v);   // the fused MoE forward's input row
        float s1;
        xq_out[t * H + j] = (int8_t)x8_code(v, s1);
        if (tid == 0) xs_out[t * (H / 32) + blockIdx.x] = s1;
    }
}

// The down / inject role of the one-launch pre-mixer: block b owns K slice
// s = b % NS (the KS values KS k .. KS k + KS - 1 of stream c, s = c * H / KS
// + k; KS = 1024, or 512 at H = 2560) of the row group g = b / NS (RPB =
// 16384 / KS rows, RPB g .. RPB g + RPB - 1 of the 320 down rows followed by
// the 4 inject rows). Threads 0..255 hold stream c as k_hc_norm_down's stream
// threads do (thread t: elements i * 256 + t, with the previous mixer's
// inject), so the sum of squares, rstd and the slice's normed values and X8
// codes are theirs bit for bit; X8 runs over the slice only, one value per
// thread (threads 256..KS-1 load their slice element themselves). Each group
// of KS / 16 lanes then dots one row's KS codes (16 bytes a lane, one exact
// int32 block dot scaled by its X8 scale) and publishes the row's partial for
// slice s. Row group 0 stores the slice's normed, X8 codes and scales and
// publishes normed.
template <int NV>
__device__ __forceinline__ void hc_slice_body(int b, const float *__restrict__ R, const uint16_t *__restrict__ wn,
                                              const float *__restrict__ y_prev, const float *__restrict__ inj_prev,
                                              const int8_t *__restrict__ Wd, const int8_t *__restrict__ Wi,
                                              float *__restrict__ normed, int8_t *__restrict__ q,
                                              float *__restrict__ sc, HcArea *A) {
    constexpr int H = NV * 256, RS = 4 * H, KS = hc_slice_of(H), SPS = H / KS, NS = 4 * SPS;
    constexpr int LPR = KS / 16, RPB = 1024 / LPR;      // lanes per row, rows per block
    constexpr int SQ = KS / 256;                         // slice values per stream thread's i range
    __shared__ __align__(16) int8_t s_q[KS];
    __shared__ float s_s[KS / 32];
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int s = b % NS, g = b / NS;
    const int c = s / SPS, k = s - c * SPS;                    // stream, slice within the stream
    const uint32_t tag = next_tag(__hip_atomic_load(&A->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int rloc = tid / LPR, l = tid % LPR;
    const int row = g * RPB + rloc;
    const int nrow = QF8_HCL + (Wi ? QF8_HCC : 0);
    const bool live = row < nrow;
    const int8_t *wr = (row < QF8_HCL ? Wd + (size_t)row * RS : live ? Wi + (size_t)(row - QF8_HCL) * RS : Wd) +
                       s * KS + l * 16;
    // the stream's values (threads 0..255) and the slice's other elements
    // (threads 256..KS-1: element t of the slice, with the same inject fma)
    // and norm weights first (the norm waits only for these), then the
    // weights, which stream meanwhile
    const bool own = tid < 256, half2 = tid >= 256 && tid < KS;
    const int m = tid;                                         // element of the slice (tid < KS)
    const size_t e_own = (size_t)c * H + (size_t)k * KS + (tid & (KS - 1));
    float v[NV], yv[NV], v2 = 0.0f, y2 = 0.0f;
    uint16_t wb = 0;
    if (own) {
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] = R[(size_t)c * H + i * 256 + tid];
    } else if (half2) {
        v2 = R[e_own];
    }
    if (tid < KS) wb = wn[e_own];
    const float sj = y_prev ? inj_prev[c] : 0.0f;
    if (y_prev) {
        if (own)
#pragma unroll
            for (int i = 0; i < NV; i++) yv[i] = y_prev[i * 256 + tid];
        else if (half2)
            y2 = y_prev[e_own - (size_t)c * H];
    }
    const i32x4 w = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wr));
    if (own) {                                                 // waves 0..3
        if (y_prev)
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = fmaf(sj, yv[i], v[i]);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; i++) acc = fmaf(v[i], v[i], acc);
        acc = group_sum<64>(acc);
        if (lane == 0) red[wave] = acc;
    } else if (half2 && y_prev) {
        v2 = fmaf(sj, y2, v2);
    }
    __syncthreads();
    if (tid < KS) {                                      // one slice value per thread
        const float rstd = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + 1e-6f);
        float v0 = v[0];
#pragma unroll
        for (int i = 1; i < NV / SQ; i++)
            if (k == i) v0 = v[SQ * i];
        const float nv = (own ? v0 : v2) * rstd * (1.0f + bf16_to_f32(wb));
        float s1;
        const int qi = x8_code(nv, s1);
        s_q[m] = (int8_t)qi;
        if ((tid & 31) == 0) s_s[m >> 5] = s1;
        if (g == 0) {
            normed[e_own] = nv;
            q[e_own] = (int8_t)qi;
            if ((tid & 31) == 0) sc[e_own >> 5] = s1;
            st_agent_u64(&A->w[kHcNormed + e_own], hc_word(nv, tag));
        }
    }
    __syncthreads();
    float a = (float)dot16_i8i8(w, *reinterpret_cast<const i32x4 *>(s_q + l * 16)) * s_s[l >> 1];
    a = group_sum<LPR>(a);
    if (l == 0 && live) st_agent_u64(&A->w[s * kHcRows + row], hc_word(a, tag));
}

// The up / combine role of the one-launch pre-mixer: up block u owns the 64
// outputs j0 = 64 u .. j0 + 63 (up rows {c*H + j}, 4 lanes per row over the
// 320 codes, 1024 threads). It requests its weights, the row scales and the
// residual inject's operands, then waits for the words of the down blocks:
// the NS partials of down row tid (waves 0-4), of the inject rows (wave 5;
// once every partial carries the call's tag every down block has read R), and
// its 4 x 64 normed values (waves 6-9). hc_d / inject values are the
// partials summed in slice order, scaled and activated; from there on the
// arithmetic is k_hc_up_combine's, except that silu and the combine's sigmoid
// use the hardware exp and reciprocal (within 1e-6 of the IEEE forms).
template <int H>
__device__ __forceinline__ void
hc_up_body(int u, int nup, const float *__restrict__ Sd, const float *__restrict__ Si, bool has_inj,
           const int8_t *__restrict__ Wu, const float *__restrict__ Su, float *__restrict__ hc_d,
           float *__restrict__ inj, float *__restrict__ hcy, float *__restrict__ mixed, int8_t *__restrict__ xq_out,
           float *__restrict__ xs_out, int8_t *__restrict__ d8q, float *__restrict__ d8s, float *__restrict__ R,
           const float *__restrict__ y_prev, const float *__restrict__ inj_prev, uint16_t *__restrict__ xb_out,
           HcArea *A) {
    constexpr int L = QF8_HCL, NS = 4 * H / hc_slice_of(H);
    __shared__ __align__(16) int8_t s_q[L];
    __shared__ float s_s[L / 32];
    __shared__ float s_h[4][64], s_n[4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, l = lane & 3;
    const int j0 = u * 64;
    const uint32_t tag = next_tag(__hip_atomic_load(&A->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int li = tid >> 2, c = li >> 6, jj = li & 63;
    const size_t row = (size_t)c * H + j0 + jj;
    const int8_t *wr = Wu + row * L + l * 16;
    i32x4 wv[L / 64];
#pragma unroll
    for (int st = 0; st < L / 64; st++) wv[st] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wr + st * 64));
    const float su = Su[row];
    // the row whose partials this thread sums (down rows, then inject rows), or -1
    const int dr = wave < 5 ? tid : wave == 5 && has_inj && lane < QF8_HCC ? L + lane : -1;
    const float rsc = dr < 0 ? 0.0f : dr < L ? Sd[dr] : Si[dr - L];
    // the previous mixer's inject into R[rc][rj] (stored once the down blocks are done with R)
    const bool rup = y_prev && tid < 256;
    const int rc = tid >> 6, rj = j0 + lane;
    float rv = 0.0f, iv = 0.0f, yv = 0.0f;
    if (rup) {
        rv = R[(size_t)rc * H + rj];
        iv = inj_prev[rc];
        yv = y_prev[rj];
    }
    // the words: waves 0-5 the NS partials of row dr (lanes with dr < 0 read
    // row 0's and ignore them), all requested together and requested again
    // until every one carries the call's tag (by the time the loads above
    // have returned the slice blocks have mostly published); waves 6-9 one
    // normed value each
    float sum = 0.0f, w0 = 0.0f;
    uint32_t bad = 0u;
    // the first request only once the loads above have returned: one that
    // went out now would sample the words long before the slice blocks
    // publish, and its (useless) traffic would meet theirs
    __builtin_amdgcn_s_waitcnt(0);
    if (wave < 6) {
        const uint32_t off = (uint32_t)(dr < 0 ? 0 : dr);
        unsigned long long x[NS];
        for (int it = 0;;) {
            uint32_t o = off;
            asm volatile("" : "+v"(o));                        // addresses formed anew each pass, not kept live
            const unsigned long long *wp = A->w + o;
#pragma unroll
            for (int i = 0; i < NS; i++) x[i] = ld_agent_u64(wp + i * kHcRows);
            bad = 0u;
#pragma unroll
            for (int i = 0; i < NS; i++)
                if (dr >= 0 && (uint32_t)(x[i] >> 32) != tag) bad |= 1u << i;
            if (__builtin_amdgcn_ballot_w64(bad != 0u) == 0 || ++it >= kTailSpinMax) break;
            __builtin_amdgcn_s_sleep(2);
        }
        sum = __uint_as_float((uint32_t)x[0]);
#pragma unroll
        for (int i = 1; i < NS; i++) sum += __uint_as_float((uint32_t)x[i]);
    } else if (wave < 10) {
        const unsigned long long *wp = &A->w[kHcNormed + (wave - 6) * H + j0 + lane];
        unsigned long long x = ld_agent_u64(wp);
        for (int it = 0; (uint32_t)(x >> 32) != tag; it++) {   // (per lane; the wave leaves when all have)
            if (it == kTailSpinMax) { bad = 1u; break; }
            __builtin_amdgcn_s_sleep(2);
            x = ld_agent_u64(wp);
        }
        w0 = __uint_as_float((uint32_t)x);
    }
    if (bad) __hip_atomic_fetch_add(&A->timeouts, (uint32_t)__builtin_popcount(bad), __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    if (wave < 5) {                                            // hc_d and X8(hc_d): five whole waves
        const float q4 = sum * rsc * 0.25f;                    // silu(v / 4), hardware exp and reciprocal
        const float hv = q4 * __builtin_amdgcn_rcpf(1.0f + __expf(-q4));
        float s1;
        const int qi = x8_code(hv, s1);
        s_q[tid] = (int8_t)qi;
        if ((tid & 31) == 0) s_s[tid >> 5] = s1;
        if (u == 0) {
            hc_d[tid] = hv;
            d8q[tid] = (int8_t)qi;
            if ((tid & 31) == 0) d8s[tid >> 5] = s1;
        }
    } else if (wave == 5) {
        if (u == 0 && dr >= 0) inj[dr - L] = gemv_act(sum * rsc, 2);
    } else if (wave < 10) {
        s_n[wave - 6][lane] = w0;
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int st = 0; st < L / 64; st++) {
        const int e0 = st * 64 + l * 16;
        acc = fmaf((float)dot16_i8i8(wv[st], *reinterpret_cast<const i32x4 *>(s_q + e0)), s_s[e0 >> 5], acc);
    }
    acc = group_sum<4>(acc);
    if (l == 0) {
        const float hv = acc * su;
        hcy[row] = hv;
        s_h[c][jj] = hv;
    }
    if (rup) R[(size_t)rc * H + rj] = fmaf(iv, yv, rv);
    __syncthreads();
    if (tid == 64) {                                           // every word of this block is read (wave 1: no
                                                               // combine work waits on the round trip)
        const uint32_t old = __hip_atomic_fetch_add(&A->arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == (uint32_t)nup - 1u) {
            __hip_atomic_store(&A->arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&A->epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (tid < 64) {
        const int j = j0 + tid;
        float sm = 0.0f;
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const float m = __builtin_amdgcn_rcpf(1.0f + __expf(-s_h[cc][tid]));
            sm = fmaf(m, s_n[cc][tid], sm);
        }
        const float v = sm * 0.25f;
        mixed[j] = v;
        if (xb_out) xb_out[j] = f32_to_bf16(v);
        float s1;
        xq_out[j] = (int8_t)x8_code(v, s1);
        if ((tid & 31) == 0) xs_out[j >> 5] = s1;
    }
}

// The pre-mixer at T = 1 in one launch: grid (ndown + H / 64), 1024 threads;
// blocks below ndown = NS * ceil(rows / 32) are slice blocks (hc_slice_body),
// the rest up blocks (last in the grid, so every slice block is dispatched
// before any up block waits; the waits are bounded either way).
struct HcOneArgs {
    const float *R;
    const uint16_t *wn;
    const float *y_prev, *inj_prev;
    const int8_t *Wd;
    const float *Sd;
    const int8_t *Wi;
    const float *Si;
    float *hc_d, *inj, *normed;
    int8_t *n8q;
    float *n8s;
    const int8_t *Wu;
    const float *Su;
    float *hcy, *mixed;
    int8_t *xq_out;
    float *xs_out;
    int8_t *d8q;
    float *d8s;
    float *Rw;
    uint16_t *xb_out;
    HcArea *A;
    int ndown;
};

template <int NV>
__global__ void __launch_bounds__(1024) k_hc_one(HcOneArgs a) {
    const int bx = (int)blockIdx.x;
    if (bx < a.ndown)
        hc_slice_body<NV>(bx, a.R, a.wn, a.y_prev, a.inj_prev, a.Wd, a.Wi, a.normed, a.n8q, a.n8s, a.A);
    else
        hc_up_body<NV * 256>(bx - a.ndown, (int)gridDim.x - a.ndown, a.Sd, a.Si, a.Wi != nullptr, a.Wu, a.Su,
                             a.hc_d, a.inj, a.hcy, a.mixed, a.xq_out, a.xs_out, a.d8q, a.d8s, a.Rw, a.y_prev,
                             a.inj_prev, a.xb_out, a.A);
}

__global__ void __launch_bounds__(256) k_stream_inject(float *__restrict__ R, const float *__restrict__ y,
                                                       const float *__restrict__ inj, int H) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < 4 * H) R[i] = fmaf(inj[i / H], y[i % H], R[i]);
}

// ---- host side -------------------------------------------------------------------
// Device address of this device's hand-off area (hipGetSymbolAddress once per
// device, with that device current; host code never passes the array's name
// to a kernel). nullptr and an error latched on failure.
constexpr int kHcMaxDevices = 64;
static HcArea *g_hc_area[kHcMaxDevices];
static std::mutex g_hc_mu;

static HcArea *hc_area_for_current_device(const char *who, bool latch = true) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kHcMaxDevices) {
        if (latch) set_error(-5, "%s: no current device (or device index >= %d)", who, kHcMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_hc_mu);
    if (!g_hc_area[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(hc_area));
        if (e != hipSuccess || !p) {
            if (latch) set_error(-5, "%s: hipGetSymbolAddress: %s", who, hipGetErrorString(e));
            return nullptr;
        }
        g_hc_area[dev] = static_cast<HcArea *>(p);
    }
    return g_hc_area[dev];
}

// set-up from qfm_init: resolve the current device's area now (nothing done
// when the host has no device)
void hc_prepare_current_device() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) return;
    (void)hc_area_for_current_device("qfm_init", false);
}

static int fill_batch(const Qf8I8Multi *mm, GemvBatch *b, int *maxr, const char *who) {
    if (!mm || mm->n < 1 || mm->n > 4) { set_error(-1, "%s: 1..4 matrices", who); return -1; }
    *b = GemvBatch{};
    b->n = mm->n;
    *maxr = 0;
    for (int i = 0; i < mm->n; i++) {
        const Qf8I8Mat *m = mm->m[i];
        if (!m || !m->w || !m->s || !mm->y[i] || m->rows < 1 || mm->act[i] < 0 || mm->act[i] > 2) {
            set_error(-1, "%s: matrix %d: null pointer, no rows or act outside 0..2", who, i);
            return -1;
        }
        if (i == 0) b->K = m->K;
        if (m->K != b->K) { set_error(-2, "%s: mixed K (%d, %d)", who, b->K, m->K); return -2; }
        b->d[i] = GemvMat{m->w, m->s, mm->y[i], m->rows, mm->act[i]};
        *maxr = max(*maxr, m->rows);
    }
    return 0;
}

static int launch_gemv(const GemvBatch &b, int maxr, const int8_t *xq, const float *xs, int T, hipStream_t s,
                       const char *who) {
    const int tpb = T == 1 ? 1 : 8;
    const unsigned gz = (unsigned)((T + tpb - 1) / tpb);
#define QFM_GEMV(LPR, NST)                                                                                          \
    hipLaunchKernelGGL((k_gemv_i8x8<LPR, NST>), dim3((unsigned)((maxr + 256 / LPR - 1) / (256 / LPR)), b.n, gz),   \
                       dim3(256), 0, s, b, xq, xs, T, tpb)
    switch (b.K) {
        case 320: QFM_GEMV(4, 5); break;
        case 512: QFM_GEMV(8, 4); break;
        case 640: QFM_GEMV(8, 5); break;
        case 2048: QFM_GEMV(32, 4); break;
        case 2560: QFM_GEMV(32, 5); break;
        case 6144: QFM_GEMV(32, 12); break;
        case 8192: QFM_GEMV(64, 8); break;
        case 10240: QFM_GEMV(64, 10); break;
        default: set_error(-2, "%s: unsupported K = %d", who, b.K); return -2;
    }
#undef QFM_GEMV
    return check_launch(who) ? -3 : 0;
}

static int hc_impl(float *normed, float *hc_d, float *mixed, float *inj, float *R, const uint16_t *wn,
                   const Qf8I8Mat *down, const Qf8I8Mat *inject, const Qf8I8Mat *up, int8_t *n8q, float *n8s,
                   int8_t *d8q, float *d8s, float *hcy, const float *y_prev, const float *inj_prev, int8_t *xq_out,
                   float *xs_out, int T, hipStream_t s, const char *who, uint16_t *xb_out = nullptr) {
    const int H = g_cfg.H, RS = 4 * H;
    if (!normed || !hc_d || !mixed || !R || !wn || !down || !up || !n8q || !n8s || !d8q || !d8s || !hcy || !xq_out ||
        !xs_out || (inject && !inj) || (!y_prev) != (!inj_prev) || T < 1) {
        set_error(-1, "%s: null buffer (inject needs inj; y_prev and inj_prev go together)", who);
        return -1;
    }
    if (H != 2048 && H != 2560) { set_error(-2, "%s: hidden %d unsupported", who, H); return -2; }
    if (down->rows != QF8_HCL || down->K != RS || up->rows != RS || up->K != QF8_HCL ||
        (inject && (inject->rows != QF8_HCC || inject->K != RS))) {
        set_error(-2, "%s: expect down [%d][%d], inject [%d][%d], up [%d][%d]", who, QF8_HCL, RS, QF8_HCC, RS, RS,
                  QF8_HCL);
        return -2;
    }
    if (!down->w || !down->s || !up->w || !up->s || (inject && (!inject->w || !inject->s))) {
        set_error(-1, "%s: matrix without codes or scales", who);
        return -1;
    }
    const int nrow = QF8_HCL + (inject ? QF8_HCC : 0);
    // two rows per block (162 blocks at the 2048 shape): 10.6 us per layer
    // against 10.8 with four rows (81 blocks) and 12.6 with one (two launches)
    constexpr int RB = 2;
    const int ndown = (nrow + RB - 1) / RB;
    const int8_t *wi = inject ? inject->w : nullptr;
    const float *si = inject ? inject->s : nullptr;
    if (T == 1) {                                              // one launch, the up blocks last
        HcArea *A = hc_area_for_current_device(who);
        if (!A) return -5;
        const int ks = hc_slice_of(H), rpb = 16384 / ks;   // slice values, rows per slice block
        const int nslice = (4 * H / ks) * ((nrow + rpb - 1) / rpb);
        const HcOneArgs a{R,   wn,     y_prev, inj_prev, down->w, down->s, wi,     si, hc_d, inj,  normed, n8q,
                          n8s, up->w,  up->s,  hcy,      mixed,   xq_out,  xs_out, d8q, d8s,  R,   xb_out, A,
                          nslice};
        const dim3 g((unsigned)(nslice + H / 64));
        if (H == 2048) hipLaunchKernelGGL(k_hc_one<8>, g, dim3(1024), 0, s, a);
        else hipLaunchKernelGGL(k_hc_one<10>, g, dim3(1024), 0, s, a);
        return check_launch(who) ? -3 : 0;
    }
    const dim3 g1((unsigned)ndown, (unsigned)T);
    if (H == 2048)
        hipLaunchKernelGGL((k_hc_norm_down<8, RB>), g1, dim3(1024), 0, s, R, wn, y_prev, inj_prev, down->w, down->s, wi, si,
                           hc_d, inj, normed, n8q, n8s);
    else
        hipLaunchKernelGGL((k_hc_norm_down<10, RB>), g1, dim3(1024), 0, s, R, wn, y_prev, inj_prev, down->w, down->s, wi, si,
                           hc_d, inj, normed, n8q, n8s);
    if (check_launch(who)) return -3;
    const dim3 g((unsigned)(H / 32), (unsigned)T);
    if (H == 2048)
        hipLaunchKernelGGL(k_hc_up_combine<2048>, g, dim3(512), 0, s, up->w, up->s, hc_d, normed, hcy, mixed, xq_out,
                           xs_out, d8q, d8s, R, y_prev, inj_prev, xb_out);
    else
        hipLaunchKernelGGL(k_hc_up_combine<2560>, g, dim3(512), 0, s, up->w, up->s, hc_d, normed, hcy, mixed, xq_out,
                           xs_out, d8q, d8s, R, y_prev, inj_prev, xb_out);
    return check_launch(who) ? -3 : 0;
}

}  // namespace qfm

using namespace qfm;

extern "C" {

int qf8_i8_gemv_multi_ex(const Qf8I8Multi *mm, const int8_t *xq, const float *xs, hipStream_t s) {
    return qf8_i8_gemv_rows(mm, xq, xs, 1, s);
}

void qf8_i8_gemv_multi(const Qf8I8Multi *mm, const int8_t *xq, const float *xs, hipStream_t s) {
    (void)qf8_i8_gemv_multi_ex(mm, xq, xs, s);
}

int qf8_i8_gemv_rows(const Qf8I8Multi *mm, const int8_t *xq, const float *xs, int T, hipStream_t s) {
    GemvBatch b;
    int maxr;
    if (!xq || !xs || T < 1 || T > 65535 * 8) { set_error(-1, "qf8_i8_gemv: null activations or T = %d", T); return -1; }
    const int rc = fill_batch(mm, &b, &maxr, "qf8_i8_gemv");
    return rc ? rc : launch_gemv(b, maxr, xq, xs, T, s, "qf8_i8_gemv");
}

int qf8_i8_hc_m1_ex(float *normed, float *hc_d, float *mixed, float *inj, float *R, const uint16_t *wn,
                    const Qf8I8Mat *down, const Qf8I8Mat *inject, const Qf8I8Mat *up, int8_t *n8q, float *n8s,
                    int8_t *d8q, float *d8s, float *hcy, const float *y_prev, const float *inj_prev, int8_t *xq_out,
                    float *xs_out, hipStream_t s) {
    return hc_impl(normed, hc_d, mixed, inj, R, wn, down, inject, up, n8q, n8s, d8q, d8s, hcy, y_prev, inj_prev,
                   xq_out, xs_out, 1, s, "qf8_i8_hc_m1");
}

void qf8_i8_hc_m1(float *normed, float *hc_d, float *mixed, float *inj, float *R, const uint16_t *wn,
                  const Qf8I8Mat *down, const Qf8I8Mat *inject, const Qf8I8Mat *up, int8_t *n8q, float *n8s,
                  int8_t *d8q, float *d8s, float *hcy, const float *y_prev, const float *inj_prev, int8_t *xq_out,
                  float *xs_out, hipStream_t s) {
    (void)qf8_i8_hc_m1_ex(normed, hc_d, mixed, inj, R, wn, down, inject, up, n8q, n8s, d8q, d8s, hcy, y_prev,
                          inj_prev, xq_out, xs_out, s);
}

int qf8_i8_hc_rows(float *normed, float *hc_d, float *mixed, float *inj, float *R, const uint16_t *wn,
                   const Qf8I8Mat *down, const Qf8I8Mat *inject, const Qf8I8Mat *up, int8_t *n8q, float *n8s,
                   int8_t *d8q, float *d8s, float *hcy, const float *y_prev, const float *inj_prev, int8_t *xq_out,
                   float *xs_out, int T, hipStream_t s) {
    if (T < 1 || T > 65535) { set_error(-1, "qf8_i8_hc_rows: T = %d", T); return -1; }
    return hc_impl(normed, hc_d, mixed, inj, R, wn, down, inject, up, n8q, n8s, d8q, d8s, hcy, y_prev, inj_prev,
                   xq_out, xs_out, T, s, "qf8_i8_hc_rows");
}

int qfm_hc_premix(float *normed, float *hc_d, float *mixed, float *inj, float *R, const uint16_t *wn,
                  const Qf8I8Mat *down, const Qf8I8Mat *inject, const Qf8I8Mat *up, int8_t *n8q, float *n8s,
                  int8_t *d8q, float *d8s, float *hcy, const float *y_prev, const float *inj_prev, int8_t *xq_out,
                  float *xs_out, uint16_t *x_bf16, int T, hipStream_t s) {
    if (T < 1 || T > 65535 || !x_bf16) { set_error(-1, "qfm_hc_premix: T = %d or no bf16 output", T); return -1; }
    return hc_impl(normed, hc_d, mixed, inj, R, wn, down, inject, up, n8q, n8s, d8q, d8s, hcy, y_prev, inj_prev,
                   xq_out, xs_out, T, s, "qfm_hc_premix", x_bf16);
}

int qfm_hc_wait_timeouts(uint32_t *count) {
    if (!count) { set_error(-1, "qfm_hc_wait_timeouts: null count"); return -1; }
    HcArea *A = hc_area_for_current_device("qfm_hc_wait_timeouts");
    if (!A) return -5;
    if (hipMemcpy(count, &A->timeouts, sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess) {
        set_error(-3, "qfm_hc_wait_timeouts: hipMemcpy failed");
        return -3;
    }
    return 0;
}

int qf8_stream_inject_ex(float *R, const float *y, const float *inj, hipStream_t s) {
    if (!R || !y || !inj) { set_error(-1, "qf8_stream_inject: null argument"); return -1; }
    const int H = g_cfg.H;
    hipLaunchKernelGGL(k_stream_inject, dim3((unsigned)((4 * H + 255) / 256)), dim3(256), 0, s, R, y, inj, H);
    return check_launch("qf8_stream_inject") ? -3 : 0;
}

void qf8_stream_inject(float *R, const float *y, const float *inj, hipStream_t s) {
    (void)qf8_stream_inject_ex(R, y, inj, s);
}

}  // extern "C"
