// qfm_csr.hip -- multi-row decode (M <= 8 "Ocho" fork rows): routing
// inversion + weight-once-per-distinct-expert gate/up and down, INT8 and
// NVFP4 arenas.
//
// Reference behaviour: the M=8 CSR tier k_m8_build_csr / k_m8_gateup /
// k_m8_downacc (ocho/amd_server/qf_moe_m8_wave64.hip:72-211, :261-299) and the
// chunk path k_i8_csr_build / k_i8_gateup_csr / k_i8_downacc_csr /
// k_i8_combine (ocho/amd_server/qf8_moe_i8.hip:196-358): distinct experts in
// ascending id, the pairs of an expert in (token, k) order, every weight row
// read once per distinct expert and dotted against all rows routed to it,
// owned partials part[t][k][H] summed in k order (no atomics, deterministic).
//
// Launch sequence (all stream-ordered), after the router launch:
//   pair-keyed form (INT8 at every M, NVFP4 at M <= 7): the router launch's
//                  selection tail has written sel/wts (and, INT8, the fp16
//                  activation chunks);
//   CSR form (NVFP4 at M = 8, measured faster there):
//   k_topk_csr     one block: the top-K of all M rows (one wave per row), then
//                  the routing inversion in LDS (per-row expert bitmaps and
//                  their word prefix counts, P = M*K <= 128 pairs); publishes
//                  sel/wts/CSR. For INT8 a second set of waves meanwhile
//                  writes the activations as scaled fp16 chunks
//                  (chunk16_to_f16).
//   k_csr_gateup   grid (I/rows, M*K), 256 threads. Pair-keyed: grid row y is
//                  pair y; it works only if y is its expert's first pair, for
//                  all of the expert's pairs (ballots over sel, pairs_of);
//                  CSR: grid row y is the y-th distinct expert (a descriptor).
//                  One lane group per gate/up row: the row pair is loaded
//                  once, then dotted with the LDS-staged activation row of each
//                  routed token. hidden is written per pair (row = pair id /
//                  CSR position).
//   k_csr_down     grid (H/ROWS, M*K + shared + M), 256 threads: the
//                  expert's down rows [ROWS b, ROWS b + ROWS), its pairs'
//                  hidden vectors staged in LDS as scaled fp16 chunks; writes
//                  the partial w * <Wd_e[c], h_pair> * scale of (t, k) as a
//                  tagged word pw[t][k][c] (slots S = K + 1 with a shared
//                  expert). Grid rows [0, ceil(M/2)) are the shared expert
//                  (INT8), two tokens each, slot K:
//                  gamma_t * <Wd_sh[c], hsh_t> * sd_sh[c]. The last M grid
//                  rows are the combine: y[t][c] = the sum of the S slots of
//                  t in slot order, once every word carries the call's tag.
// The pair set of an expert is the same in both forms (ascending pair id =
// (token, k) order) and every sum runs in the same order: the two forms give
// identical bits.
// INT8 dots widen the codes to fp16 (dot16_i8h); NVFP4 gate/up converts e2m1
// to bf16 pairs against the bf16 activations, NVFP4 down to fp16 pairs.
#include "qfm_dev.h"
#include "qfm_internal.h"

namespace qfm {

constexpr int kMaxRows = 8;
constexpr int kMaxPairs = kMaxRows * 16;

// ---- weight-format policies ----------------------------------------------------
// A row of K values is K/VPB bytes; lanes read 16-byte chunks (VPC values).
struct FmtI8 {
    static constexpr int VPB = 1, VPC = 16;
};
struct FmtF4 {
    static constexpr int VPB = 2, VPC = 32;
};

// x slice for a chunk-strided lane layout: chunk q of a row covers values
// [q*VPC, q*VPC + VPC); lane l of an LPR group owns chunks st*LPR + l.
template <int K, int LPR, int VPC>
__device__ __forceinline__ void load_slice_bf16(const uint16_t *x, int l, float (&xs)[K / (LPR * VPC)][VPC]) {
    constexpr int NST = K / (LPR * VPC);
#pragma unroll
    for (int st = 0; st < NST; st++) {
        const uint16_t *p = x + (st * LPR + l) * VPC;
#pragma unroll
        for (int q = 0; q < VPC / 8; q++) {
            const uint4 a = *reinterpret_cast<const uint4 *>(p + q * 8);
            const uint32_t d[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int b = 0; b < 4; b++) { xs[st][q * 8 + 2 * b] = bf16_lo(d[b]); xs[st][q * 8 + 2 * b + 1] = bf16_hi(d[b]); }
        }
    }
}

// ---- routing inversion in LDS ---------------------------------------------------
struct CsrLds {
    int sel[kMaxPairs];
    float wts[kMaxPairs];
    int pair[kMaxPairs];      // CSR position -> original pair index t*K + k
    int exp_id[kMaxPairs];
    int exp_ptr[kMaxPairs + 1];
    uint32_t tbits[kMaxRows][512 / 32];   // per row: bitmap of its selected experts (E == 512)
    int tpre[kMaxRows][512 / 32];         // per row: its selected experts in bitmap words [0, w)
    uint32_t bits[512 / 32];              // union of the rows' bitmaps
    int gpre[512 / 32 + 1];               // distinct experts in words [0, w); [16] = all
    int n_exp;
    alignas(16) unsigned long long tk[8][kTopkLds];
};

// Called by all threads of the block after sel of the P = M K pairs is in LDS
// and tbits is zero; the K experts of a row are distinct (top-K). Position of
// pair p = (t, k) with expert e in (expert, token, k) order
//   #{q: e_q < e} + #{q < p: e_q == e}
//   = sum over rows u of #{experts of u below e} + #{rows u < t selecting e},
// and e's distinct index = #{distinct experts below e}: both read from the
// per-row bitmaps and their word prefix counts (no scan over the pairs).
__device__ __forceinline__ void csr_build_lds(CsrLds &c, int M, int K) {
    const int P = M * K, i = threadIdx.x, wave = i >> 6, lane = i & 63;
    if (i < P) {
        const int e = c.sel[i];
        atomicOr(&c.tbits[i / K][e >> 5], 1u << (e & 31));
    }
    __syncthreads();
    if (wave < M && lane < 32) {
        // lanes 0-15: row `wave`'s word w; lanes 16-31: the union's word w;
        // exclusive prefix sums of the popcounts over the 16 words
        const int w = lane & 15;
        uint32_t b = 0u;
        if (lane < 16) {
            b = c.tbits[wave][w];
        } else {
            for (int u = 0; u < M; u++) b |= c.tbits[u][w];
        }
        const int pc = __popc(b);
        int inc = pc;
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
            const int o = __shfl_up(inc, d, 16);
            if (w >= d) inc += o;
        }
        if (lane < 16) {
            c.tpre[wave][w] = inc - pc;
        } else if (wave == 0) {
            c.bits[w] = b;
            c.gpre[w] = inc - pc;
            if (w == 15) c.gpre[16] = inc;
        }
    }
    __syncthreads();
    if (i < P) {
        const int e = c.sel[i], t = i / K, w = e >> 5, sh = e & 31;
        const uint32_t below = (1u << sh) - 1u;
        int less = 0, before = 0;
        for (int u = 0; u < M; u++) {
            const uint32_t b = c.tbits[u][w];
            less += c.tpre[u][w] + __popc(b & below);
            before += u < t ? (int)((b >> sh) & 1u) : 0;
        }
        const int first_less = c.gpre[w] + __popc(c.bits[w] & below);
        c.pair[less + before] = i;
        if (before == 0) { c.exp_id[first_less] = e; c.exp_ptr[first_less] = less; }
    }
    if (i == 0) {
        const int n = c.gpre[16];
        c.n_exp = n;
        c.exp_ptr[n] = P;
    }
    __syncthreads();
}

// ---- top-K of all rows + routing inversion: one block, one wave per row ---------
// Published: sel/wts [M][K]; csr = {n_exp, exp_id[P], exp_ptr[P+1], pair[P]}
// and the per-slot descriptors at csr_desc_off(P); ctl[0] = the call's tag.
// With xh != nullptr, threads [kTopkThreads, blockDim.x) meanwhile write the
// activations x [M][H] (bf16) as scaled fp16 chunks for the INT8 dot:
// xh [M][H] fp16, xci [M][H/16] = (seed, 2^-k) of each 16-value chunk.
constexpr int kTopkThreads = 512;
template <int EPL>
__global__ void __launch_bounds__(1024)
k_topk_csr(const float *__restrict__ logits, int ld, int M, int K, int renorm, int *__restrict__ g_sel,
           float *__restrict__ g_wts, int *__restrict__ g_csr, const uint16_t *__restrict__ x, int H,
           uint4 *__restrict__ xh, float2 *__restrict__ xci, uint32_t *__restrict__ ctl) {
    __shared__ CsrLds c;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int P = M * K;
    if (threadIdx.x < kMaxRows * 16) (&c.tbits[0][0])[threadIdx.x] = 0u;
    if (wave < M) {
        int my_i;
        float my_w;
        wave_topk<EPL>(logits + (size_t)wave * ld, K, renorm, lane, c.tk[wave], my_i, my_w);
        if (lane < K) { c.sel[wave * K + lane] = my_i; c.wts[wave * K + lane] = my_w; }
    } else if (xh && (int)threadIdx.x >= kTopkThreads) {
        const int nch = M * (H / 16);
        for (int ch = threadIdx.x - kTopkThreads; ch < nch; ch += blockDim.x - kTopkThreads) {
            const uint4 a = reinterpret_cast<const uint4 *>(x)[2 * ch], b = reinterpret_cast<const uint4 *>(x)[2 * ch + 1];
            const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float v[16];
#pragma unroll
            for (int i = 0; i < 8; i++) { v[2 * i] = bf16_lo(d[i]); v[2 * i + 1] = bf16_hi(d[i]); }
            uint4 ha, hb;
            xci[ch] = chunk16_to_f16(v, ha, hb);
            xh[2 * ch] = ha;
            xh[2 * ch + 1] = hb;
        }
    }
    __syncthreads();
    csr_build_lds(c, M, K);
    for (int i = threadIdx.x; i < P; i += blockDim.x) {
        g_sel[i] = c.sel[i]; g_wts[i] = c.wts[i];
        g_csr[1 + i] = c.exp_id[i];
        g_csr[1 + P + (P + 1) + i] = c.pair[i];
    }
    for (int i = threadIdx.x; i <= P; i += blockDim.x) g_csr[1 + P + i] = c.exp_ptr[i];
    if (threadIdx.x == 0) {
        g_csr[0] = c.n_exp;
        ctl[0] = next_tag(ctl[0]);                // this call's partial-word tag (k_csr_down)
    }
    for (int u = threadIdx.x; u < P; u += blockDim.x) {
        int4 d = make_int4(-1, P, 0, 0);
        if (u < c.n_exp) {
            const int p0 = c.exp_ptr[u], np = c.exp_ptr[u + 1] - p0;
            d = make_int4(c.exp_id[u], p0 | (np << 16), c.pair[p0], np > 1 ? c.pair[p0 + 1] : 0);
        }
        reinterpret_cast<int4 *>(g_csr + csr_desc_off(P))[u] = d;
    }
}

// ---- the pairs of an expert, from sel -------------------------------------------
// Pair q = t K + k of the P = M K pairs has expert sel[q] (written by the router
// launch's selection tail). The workgroups of pair p run the expert's work only
// if p is its first pair (the owner); the K experts of a row are distinct, so an
// expert has at most M <= kMaxRows pairs. Ballots over the P ids give the owner
// test and the pair list (ascending pair id, i.e. (row, k) order) in scalar
// registers: no routing-inversion pass. Grid row y is pair y.
struct PairSet {
    int e, np;                 // e < 0: this workgroup's pair is not the owner
    unsigned long long a, c;   // the expert's pairs: bit q of a (q < 64), bit q - 64 of c
    int pl;                    // in lane j < np: the j-th pair id (ascending)
};
// the lowest pair of (a, c), removed from them (0 when none is left)
__device__ __forceinline__ int next_pair(unsigned long long &a, unsigned long long &c) {
    int q = 0;
    if (a) { q = (int)__builtin_ctzll(a); a &= a - 1ull; }
    else if (c) { q = 64 + (int)__builtin_ctzll(c); c &= c - 1ull; }
    return __builtin_amdgcn_readfirstlane(q);
}
__device__ __forceinline__ PairSet pairs_of(const int *__restrict__ sel, int P, int p) {
    const int lane = threadIdx.x & 63;
    PairSet r;
    r.e = __builtin_amdgcn_readfirstlane(sel[p]);
    const int s0 = lane < P ? sel[lane] : -1, s1 = lane + 64 < P ? sel[lane + 64] : -1;
    unsigned long long a = __ballot(s0 == r.e), c = __ballot(s1 == r.e);
    r.a = a;
    r.c = c;
    const int first = a ? (int)__builtin_ctzll(a) : 64 + (int)__builtin_ctzll(c);
    r.np = __builtin_amdgcn_readfirstlane(__popcll(a) + __popcll(c));
    if (__builtin_amdgcn_readfirstlane(first) != p) r.e = -1;
    // lane j: the j-th set bit of (a, c), by clearing the j lowest (an expert
    // with one pair, the common case at M = 8, has pair p alone: no walk)
    r.pl = p;
    if (r.np > 1) {
        const int na = __popcll(a);
        unsigned long long m = lane < na ? a : c;
        const int skip = lane < na ? lane : lane - na;
#pragma unroll
        for (int i = 0; i < kMaxRows - 1; i++)
            if (i < skip) m &= m - 1ull;
        r.pl = (lane < na ? 0 : 64) + (m ? (int)__builtin_ctzll(m) : 0);
    }
    return r;
}
// pair j of the set: j wave-uniform (readlane) or per thread (shuffle)
__device__ __forceinline__ int pair_at(const PairSet &ps, int j) { return __builtin_amdgcn_readlane(ps.pl, j); }
__device__ __forceinline__ int pair_of_lane(const PairSet &ps, int j) { return ps.np > 1 ? __shfl(ps.pl, j) : ps.pl; }

// ---- gate/up: one distinct expert per blockIdx.y ---------------------------------
// lanes per gate/up row (32 measured best for both formats at M = 8; 16 and 8
// were slower)
template <class F, int H>
constexpr int gateup_lpr() { return lpr_of(H / F::VPB / 16); }
constexpr int kGateupPG = 2;   // routed activation rows staged in LDS at a time
// threads per gate/up block (M = 8 over 48 layers, INT8 / NVFP4: 256 threads
// 58.0 / 47.0 us per layer; 64: 66.5 / 51.1; 128: 59.8 / 48.5; 512: 58.7 / 48.1;
// 1024: 62.0 / 52.5)
#ifndef QFM_GU_THREADS
#define QFM_GU_THREADS 256
#endif
constexpr int kGuThreads = QFM_GU_THREADS;
// One block per (distinct expert, RPB rows), one LPR-lane group per gate/up
// row. The row pair's weights are loaded first (the HBM stream starts at
// once); the activation rows of the expert's pairs are staged in LDS straight
// from memory, kGateupPG at a time (INT8: the scaled fp16 rows xh with their
// chunk (seed, 2^-k) xci, dot16_i8h; NVFP4: the bf16 rows x, f4_chunk_bx).
// (A persistent form over tile ranges with two tiles of weights in flight was
// slower: its registers allowed two waves per SIMD instead of four, and the
// dot and reduction latencies then went unhidden.)
template <class F, int H, int I, bool PAIRS>
__global__ void __launch_bounds__(kGuThreads)
k_csr_gateup(const uint8_t *__restrict__ Wg, const uint8_t *__restrict__ Wu,
             const float *__restrict__ Sg, const float *__restrict__ Su,          // INT8 row scales
             const uint8_t *__restrict__ Bg, const uint8_t *__restrict__ Bu,      // NVFP4 block scales
             const float *__restrict__ s2g, const float *__restrict__ s2u,        // NVFP4 per-expert scale
             const uint16_t *__restrict__ x, const uint4 *__restrict__ xh, const float2 *__restrict__ xci,
             int K, const int *__restrict__ rt, int P, float *__restrict__ hpair) {
    constexpr bool I8 = F::VPB == 1;
    constexpr int ROWB = H / F::VPB;             // bytes per gate/up row
    constexpr int LPR = gateup_lpr<F, H>();      // lanes per row
    constexpr int NST = ROWB / (LPR * 16);
    constexpr int RPB = kGuThreads / LPR;        // rows per block
    constexpr int NW = kGuThreads / 64;          // waves per block
    constexpr int XQ = H / 8;                    // 16-byte words per staged activation row
    constexpr int NCH = H / 16;                  // 16-value chunks per row
    constexpr int PG = kGateupPG;
    static_assert(XQ % 64 == 0 && (NCH * 2) % 64 == 0, "rows are staged in 64-lane wave loads");
    __shared__ uint4 s_x[PG * XQ];
    __shared__ float2 s_ci[I8 ? PG * NCH : 1];
    // PAIRS (rt = sel): grid row y is pair y, run by its expert's first pair
    // (pairs_of); otherwise (rt = the routing launch's csr buffer) grid row y is
    // the y-th distinct expert, found with one 16-byte descriptor load
    int e, np, p0 = 0;
    int4 dsc = make_int4(0, 0, 0, 0);
    unsigned long long pa = 0ull, pc = 0ull;     // PAIRS: pairs not staged yet, ascending
    if constexpr (PAIRS) {
        const PairSet ps = pairs_of(rt, P, blockIdx.y);
        args_now(ps.e, Wg, Wu);                  // (the weight bases requested with sel, before the branch)
        e = ps.e; np = ps.np; pa = ps.a; pc = ps.c;
    } else {
        dsc = reinterpret_cast<const int4 *>(rt + csr_desc_off(P))[blockIdx.y];   // one load before any weight
        // keep the descriptor one 16-byte load and the weight bases loaded before
        // the branch (the compiler otherwise sinks each field, and each kernel
        // argument, below the branch that first needs it: a round trip apiece)
        args_now(dsc.x, dsc.y, dsc.z, dsc.w, Wg, Wu);
        e = dsc.x; p0 = dsc.y & 0xFFFF; np = dsc.y >> 16;
    }
    if (e < 0) return;                           // not an expert's first pair / past the last expert
    const int *pair = rt + 1 + P + P + 1;        // csr: CSR position -> pair id
    const int l = threadIdx.x % LPR;
    const int row = blockIdx.x * RPB + threadIdx.x / LPR;
    const size_t roff = ((size_t)e * I + row) * ROWB;
    uint4 wg[NST], wu[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        wg[st] = ld_nt16(Wg + roff + (st * LPR + l) * 16);
        wu[st] = ld_nt16(Wu + roff + (st * LPR + l) * 16);
    }
    uint32_t bs[2 * NST];                         // NVFP4 block-scale pairs: gate chunks, then up chunks
    float rsg, rsu;
    if constexpr (!I8) {
        const size_t boff = ((size_t)e * I + row) * (H / 16);
#pragma unroll
        for (int st = 0; st < NST; st++) {
            bs[st] = *reinterpret_cast<const uint16_t *>(Bg + boff + (st * LPR + l) * 2);
            bs[NST + st] = *reinterpret_cast<const uint16_t *>(Bu + boff + (st * LPR + l) * 2);
        }
        rsg = s2g[e]; rsu = s2u[e];
    } else {
        rsg = Sg[(size_t)e * I + row]; rsu = Su[(size_t)e * I + row];
    }
    const uint4 *src = I8 ? xh : reinterpret_cast<const uint4 *>(x);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    static_assert(PG == 2, "two staged rows per group (pq0, pq1)");
    for (int j0 = 0; j0 < np; j0 += PG) {
        const int ng = min(PG, np - j0);
        // staged row j's pair id and hidden row (PAIRS: row = pair id; csr: row =
        // CSR position, pair id from the descriptor for the first two)
        int pq0 = 0, pq1 = 0;
        if constexpr (PAIRS) {
            pq0 = next_pair(pa, pc);
            pq1 = next_pair(pa, pc);
        }
        auto pair_id = [&](int j) -> int {
            if constexpr (PAIRS) return j == 0 ? pq0 : pq1;
            else return j0 + j == 0 ? dsc.z : j0 + j == 1 ? dsc.w : pair[p0 + j0 + j];
        };
        auto hid_row = [&](int j) -> int {
            if constexpr (PAIRS) return j == 0 ? pq0 : pq1;
            else return p0 + j0 + j;
        };
        if (j0 > 0) __syncthreads();             // the previous group's rows are consumed
        // straight into LDS (global_load_lds: lane i of a wave load writes base + 16 i / 4 i)
        for (int k = wave; k < ng * (XQ / 64); k += NW) {
            const int j = k / (XQ / 64), c = k - j * (XQ / 64);
            const int pr = pair_id(j);
            __builtin_amdgcn_global_load_lds(src + (size_t)(pr / K) * XQ + c * 64 + lane,
                                             (__attribute__((address_space(3))) void *)(s_x + j * XQ + c * 64), 16, 0, 0);
        }
        if constexpr (I8) {
            constexpr int CW = NCH * 2 / 64;
            const uint32_t *cs = reinterpret_cast<const uint32_t *>(xci);
            for (int k = wave; k < ng * CW; k += NW) {
                const int j = k / CW, c = k - j * CW;
                const int pr = pair_id(j);
                __builtin_amdgcn_global_load_lds(cs + (size_t)(pr / K) * NCH * 2 + c * 64 + lane,
                                                 (__attribute__((address_space(3))) void *)(reinterpret_cast<uint32_t *>(s_ci) + j * NCH * 2 + c * 64), 4, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);          // this wave's LDS loads (and its weights) have landed
        __syncthreads();

        for (int j = 0; j < ng; j++) {
            float ag = 0.0f, au = 0.0f;
#pragma unroll
            for (int st = 0; st < NST; st++) {
                const int ch = st * LPR + l;
                if constexpr (I8) {
                    const uint4 xa = s_x[j * XQ + 2 * ch], xb = s_x[j * XQ + 2 * ch + 1];
                    const float2 ci = s_ci[j * NCH + ch];
                    ag = fmaf(dot16_i8h(wg[st], xa, xb, ci.x), ci.y, ag);
                    au = fmaf(dot16_i8h(wu[st], xa, xb, ci.x), ci.y, au);
                } else {
                    uint32_t xw[16];                     // the 32 bf16 activations as packed pairs
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const uint4 a = s_x[j * XQ + 4 * ch + q];
                        xw[4 * q] = a.x; xw[4 * q + 1] = a.y; xw[4 * q + 2] = a.z; xw[4 * q + 3] = a.w;
                    }
                    ag += f4_chunk_bx(wg[st], bs[st], xw);        // (the hardware scale convert
                    au += f4_chunk_bx(wu[st], bs[NST + st], xw);  // measured slower here: 24.9 vs 22.5 us)
                }
            }
            ag = group_sum<LPR>(ag);
            au = group_sum<LPR>(au);
            if (l == 0) hpair[(size_t)hid_row(j) * I + row] = silu(ag * rsg) * (au * rsu);
        }
    }
}

// <down row, staged hidden row j> over this lane's NST chunks: INT8 (16 codes
// per chunk, dot16_i8h) or NVFP4 (32 codes per chunk, f4_chunk_h)
template <class F, int I, int LPR, int NST>
__device__ __forceinline__ float down_dot(const uint4 (&w)[NST], const f32x2_t (&bs)[NST], const uint4 *s_h16,
                                          const float2 *s_hci, int j, int l) {
    float d = 0.0f;
#pragma unroll
    for (int st = 0; st < NST; st++) {
        const int ch = st * LPR + l;
        if constexpr (F::VPB == 1) {
            const float2 ci = s_hci[j * (I / 16) + ch];
            d = fmaf(dot16_i8h(w[st], s_h16[j * (I / 8) + 2 * ch], s_h16[j * (I / 8) + 2 * ch + 1], ci.x), ci.y, d);
        } else {
            uint32_t xw[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint4 a = s_h16[j * (I / 8) + 4 * ch + q];
                xw[4 * q] = a.x; xw[4 * q + 1] = a.y; xw[4 * q + 2] = a.z; xw[4 * q + 3] = a.w;
            }
            d += f4_chunk_h(w[st], bs[st], xw, s_hci[j * (I / 16) + 2 * ch].y, s_hci[j * (I / 16) + 2 * ch + 1].y);
        }
    }
    return d;
}

// ---- partial words and the combine -------------------------------------------------
// A partial is stored as a 64-bit word (fp32 bits | tag << 32) at agent scope:
// written through to memory, readable from every XCD without a fence.
__device__ __forceinline__ void st_part(unsigned long long *p, float v, uint32_t tag) {
    st_agent_u64(p, (unsigned long long)__float_as_uint(v) | ((unsigned long long)tag << 32));
}
// The down launch's last M grid rows: workgroup (b, M - 1 - ...) owns output
// columns [c0, c0 + ROWS) of one row t. SL = 256 / ROWS adjacent lanes (one
// wave) share a column, lane j reading slots j, j + SL, ...: each wave first
// waits for one word, then each lane (bounded: 2^16 polls, a timeout counted
// in *tmo and the words used as found) until its words carry this call's tag,
// only pending words being read again; the column's values then go through LDS to its first lane, which sums
// them in slot order from 0 (k_pf_combine's order) and stores y (bf16, round
// to nearest even) or y32. The words come from workgroups of earlier grid
// rows, dispatched before this one, which never wait: the waits end.
template <int H, int ROWS>
__device__ __forceinline__ void csr_combine(const unsigned long long *__restrict__ pw, uint32_t tag, int t, int S,
                                            int c0, float *s_v, uint16_t *__restrict__ y, float *__restrict__ y32,
                                            uint32_t *__restrict__ tmo) {
    constexpr int SL = 256 / ROWS;                 // lanes per column
    constexpr int kMaxS = 17;                      // K <= 16 routed + the shared slot
    constexpr int NW = (kMaxS + SL - 1) / SL;      // words per lane
    constexpr int SP = kMaxS;                      // LDS floats per column
    static_assert(SL >= 1 && 64 % SL == 0, "a column's lanes must share a wave");
    const int c = threadIdx.x / SL, j = threadIdx.x - c * SL;
    const unsigned long long *w = pw + (size_t)t * S * H + c0 + c;
    {   // first one word per wave (its first column's slot 0): almost no traffic
        // while the producers still stream their weights
        const unsigned long long *w0 = pw + (size_t)t * S * H + c0 + (int)(threadIdx.x & ~63u) / SL;
        for (int it = 0; it < kTailSpinMax; it++) {
            const unsigned long long x = ld_agent_u64(w0);
            if (__builtin_amdgcn_readfirstlane((int)((uint32_t)(x >> 32) == tag))) break;
            __builtin_amdgcn_s_sleep(2);
        }
    }
    float v[NW];
    uint32_t pend = 0u;
#pragma unroll
    for (int q = 0; q < NW; q++) {
        const int sl = j + q * SL;
        v[q] = 0.0f;
        if (sl < S) {
            const unsigned long long x = ld_agent_u64(w + (size_t)sl * H);
            if ((uint32_t)(x >> 32) == tag) v[q] = __uint_as_float((uint32_t)x);
            else pend |= 1u << q;
        }
    }
    for (int it = 0; __builtin_amdgcn_ballot_w64(pend != 0u) != 0; it++) {
        if (it == kTailSpinMax) {
            if (pend) __hip_atomic_fetch_add(tmo, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int q = 0; q < NW; q++) {
            if (pend & (1u << q)) {
                const unsigned long long x = ld_agent_u64(w + (size_t)(j + q * SL) * H);
                if ((uint32_t)(x >> 32) == tag) {
                    v[q] = __uint_as_float((uint32_t)x);
                    pend &= ~(1u << q);
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < NW; q++)
        if (j + q * SL < S) s_v[c * SP + j + q * SL] = v[q];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");   // the column's lanes are in this wave
    if (j == 0) {
        float a = 0.0f;
        for (int sl = 0; sl < S; sl++) a += s_v[c * SP + sl];
        if (y32) y32[(size_t)t * H + c0 + c] = a;
        else y[(size_t)t * H + c0 + c] = f32_to_bf16(a);
    }
}

// ---- shared expert's down rows (INT8) for tokens [t0, t1): one k_csr_down block ----
// rows [c0, c0 + ROWS)
template <int H, int I, int ROWS>
__device__ __forceinline__ void csr_down_shared(const ShPtrs &sh, const float *__restrict__ hsh,
                                                const float *__restrict__ logits, int ld, int gated, int t0,
                                                int t1, int S, int K, int c0, uint4 *s_h16, float2 *s_hci,
                                                float *s_out, unsigned long long *__restrict__ pw, uint32_t tag) {
    constexpr int CPR = I / 16, LPR = lpr_of(CPR), NST = CPR / LPR, GROUPS = 256 / LPR, RPG = ROWS / GROUPS;
    static_assert(RPG >= 1 && RPG * GROUPS == ROWS, "shared rows must tile the block");
    const int l = threadIdx.x % LPR, grp = threadIdx.x / LPR;
    constexpr int TS = 2;                         // tokens per shared block
    const int nt = t1 - t0;
    H16Stage<I, TS> hst;                          // the tokens' hidden rows ahead of the weights
    hst.load(hsh + (size_t)t0 * I, nt);
    uint4 w[RPG][NST];
    f32x2_t bs[NST] = {};
    float rs[RPG];
#pragma unroll
    for (int q = 0; q < RPG; q++) {
        const int c = c0 + q * GROUPS + grp;
#pragma unroll
        for (int st = 0; st < NST; st++) w[q][st] = ld_nt16(sh.qd + (size_t)c * I + (st * LPR + l) * 16);
        rs[q] = sh.sd[c];
    }
    float gam[TS];
#pragma unroll
    for (int t = 0; t < TS; t++) gam[t] = gated ? logits[(size_t)(t0 + (t < nt ? t : 0)) * ld + (ld - 1)] : 0.0f;
    hst.store(nt, s_h16, s_hci);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TS; t++) {
        if (t >= nt) break;
        const float g = gated ? sigmoid(gam[t]) : 1.0f;
#pragma unroll
        for (int q = 0; q < RPG; q++) {
            float d = down_dot<FmtI8, I, LPR, NST>(w[q], bs, s_h16, s_hci, t, l);
            d = group_sum<LPR>(d);
            if (l == 0) s_out[t * ROWS + q * GROUPS + grp] = g * (d * rs[q]);
        }
    }
    __syncthreads();                              // contiguous runs of words, as in k_csr_down
    for (int i = threadIdx.x; i < nt * ROWS; i += 256) {
        const int t = i / ROWS, r = i - t * ROWS;
        st_part(pw + ((size_t)(t0 + t) * S + K) * H + c0 + r, s_out[i], tag);
    }
}

// ---- down: one distinct expert x ROWS rows per block, owned partials ---------------
#ifndef QFM_DOWN_ROWS_I8
#define QFM_DOWN_ROWS_I8 32
#endif
#ifndef QFM_DOWN_ROWS_F4
#define QFM_DOWN_ROWS_F4 32
#endif
template <class F, int I>
constexpr int down_rows() {
    constexpr int want = F::VPB == 1 ? QFM_DOWN_ROWS_I8 : QFM_DOWN_ROWS_F4;
    return want > 256 / lpr_of(I / F::VPB / 16) ? want : 256 / lpr_of(I / F::VPB / 16);
}
template <class F, int H, int I, bool PAIRS>
__global__ void __launch_bounds__(256)
k_csr_down(const uint8_t *__restrict__ Wd, const float *__restrict__ Sd, const uint8_t *__restrict__ Bd,
           const float *__restrict__ s2d, const float *__restrict__ hpair, const float *__restrict__ g_wts,
           const int *__restrict__ rt, int P, unsigned long long *__restrict__ pw, int K, ShPtrs sh,
           const float *__restrict__ hsh, const float *__restrict__ logits, int ld, int gated, int M,
           uint32_t *__restrict__ ctl, uint16_t *__restrict__ y, float *__restrict__ y32) {
    constexpr int ROWB = I / F::VPB;                   // bytes per down row
    constexpr int CPR = ROWB / 16;                     // 16-byte chunks per row
    constexpr int LPR = lpr_of(CPR);                   // lanes per row
    constexpr int NST = CPR / LPR;
    constexpr int GROUPS = 256 / LPR;                  // row groups per block
    constexpr int ROWS = down_rows<F, I>();
    __shared__ uint4 s_h16[kMaxRows * I / 8];
    __shared__ float2 s_hci[kMaxRows * I / 16];
    __shared__ float s_out[kMaxRows * ROWS];      // the block's partials, [pair j or token][row]
    const bool has_sh = sh.qd != nullptr;
    const int S = K + (has_sh ? 1 : 0);
    const int nsh = has_sh ? (M + 1) / 2 : 0;      // grid rows of shared blocks, two tokens each
    const uint32_t tag = ctl[0];                   // this call's partial-word tag
    if ((int)blockIdx.y >= (int)gridDim.y - M) {   // the combine rows, one per token row (dispatched last)
        static_assert(sizeof(s_h16) >= ROWS * 17 * sizeof(float), "combine values fit the staging buffer");
        csr_combine<H, ROWS>(pw, tag, (int)blockIdx.y - ((int)gridDim.y - M), S, blockIdx.x * ROWS,
                             reinterpret_cast<float *>(s_h16), y, y32, ctl + kTailRows);
        return;
    }
    if ((int)blockIdx.y < nsh) {                  // dispatched first
        const int t0 = blockIdx.y * 2;
        csr_down_shared<H, I, ROWS>(sh, hsh, logits, ld, gated, t0, min(M, t0 + 2), S, K, blockIdx.x * ROWS, s_h16,
                                    s_hci, s_out, pw, tag);
        return;
    }
    // as in k_csr_gateup: PAIRS, grid row y - nsh is a pair; csr, a distinct expert
    PairSet ps{};
    int e, np, p0 = 0;
    if constexpr (PAIRS) {
        ps = pairs_of(rt, P, (int)blockIdx.y - nsh);
        args_now(ps.e, Wd);
        e = ps.e; np = ps.np;
    } else {
        const int4 dsc = reinterpret_cast<const int4 *>(rt + csr_desc_off(P))[blockIdx.y - nsh];
        args_now(dsc.x, dsc.y, Wd);
        e = dsc.x; p0 = dsc.y & 0xFFFF; np = dsc.y >> 16;
    }
    if (e < 0) return;                           // not an expert's first pair / past the last expert
    const int *pair = rt + 1 + P + P + 1;        // csr: CSR position -> pair id
    const int l = threadIdx.x % LPR, grp = threadIdx.x / LPR;
    // the pairs' hidden rows first (in L2 or the memory-side cache: they arrive
    // before the weights, and loads retire in issue order, so their conversion
    // runs while the weights stream; M = 8 NVFP4 layer 47.1 -> 46.1 us)
    H16Stage<I, kMaxRows> hst;
    if constexpr (PAIRS) {
        hst.load_rows(hpair, ps, np);
        // (their addresses wait for the pair list, the weights' only for e:
        // without this barrier the scheduler issues the weights first and the
        // conversion then waits for them)
        __builtin_amdgcn_sched_barrier(0);
    } else {
        hst.load(hpair + (size_t)p0 * I, np);    // the expert's rows are contiguous in CSR order
    }
    // then the weights for this thread's rows (ROWS/GROUPS rows per group)
    constexpr int RPG = ROWS / GROUPS;
    uint4 w[RPG][NST];
    uint32_t braw[RPG * NST];                    // NVFP4 block-scale pairs
    f32x2_t bs[RPG][NST];
    float rs[RPG];
#pragma unroll
    for (int q = 0; q < RPG; q++) {
        const int c = blockIdx.x * ROWS + q * GROUPS + grp;
        const size_t roff = ((size_t)e * H + c) * ROWB;
#pragma unroll
        for (int st = 0; st < NST; st++) w[q][st] = ld_nt16(Wd + roff + (st * LPR + l) * 16);
        if constexpr (F::VPB == 2) {
            const size_t boff = ((size_t)e * H + c) * (I / 16);
#pragma unroll
            for (int st = 0; st < NST; st++) braw[q * NST + st] = *reinterpret_cast<const uint16_t *>(Bd + boff + (st * LPR + l) * 2);
            rs[q] = s2d[e];
        } else {
#pragma unroll
            for (int st = 0; st < NST; st++) braw[q * NST + st] = 0u;
            rs[q] = Sd[(size_t)e * H + c];
        }
    }
    hst.store(np, s_h16, s_hci);
    __syncthreads();
    if constexpr (F::VPB == 2) {
        f32x2_t dec[RPG * NST];
        e4m3_pairs(braw, dec);
#pragma unroll
        for (int q = 0; q < RPG; q++)
#pragma unroll
            for (int st = 0; st < NST; st++) bs[q][st] = dec[q * NST + st];
    }
    __shared__ int s_pr[kMaxRows];
    for (int j = 0; j < np; j++) {
        const int pr = PAIRS ? pair_at(ps, j) : pair[p0 + j];
        const float wp = g_wts[pr];
        if (threadIdx.x == 0) s_pr[j] = pr;
#pragma unroll
        for (int q = 0; q < RPG; q++) {
            float d = down_dot<F, I, LPR, NST>(w[q], bs[q], s_h16, s_hci, j, l);
            d = group_sum<LPR>(d);
            if (l == 0) s_out[j * ROWS + q * GROUPS + grp] = wp * (d * rs[q]);
        }
    }
    // each pair's ROWS partials leave as one contiguous run of words (the
    // write-through stores then fill whole memory segments)
    __syncthreads();
    for (int i = threadIdx.x; i < np * ROWS; i += 256) {
        const int j = i / ROWS, r = i - j * ROWS;
        const int pr = s_pr[j];
        st_part(pw + ((size_t)(pr / K) * S + pr % K) * H + blockIdx.x * ROWS + r, s_out[i], tag);
    }
}

// ---- launchers -------------------------------------------------------------------
// NVFP4 at M = 8 keeps the routing launch: measured per layer (48 layers,
// graph, A/B on one box, combine in the down launch) the pair-keyed form is
// 0.9 us slower there and 0.4 us faster at M = 7 (and faster at every smaller
// M); INT8 is faster pair-keyed at every M.
bool csr_routing_for(int fmt, int M) { return fmt == QFM_FMT_NVFP4 && M >= 8; }

int launch_csr_forward(const Qf4ExpCache *a, int fmt, const ShPtrs *sh, const uint16_t *x, const float *logits,
                       int ld, int gated, int M, float *hpair, const float *hsh, int *sel, float *wts, int *csr,
                       void *xh16, unsigned long long *pw, uint32_t *ctl, uint16_t *y, float *y32, hipStream_t s) {
    const int K = g_cfg.K, E = g_cfg.E, P = M * K;
    if (M < 1 || M > kMaxRows || P > kMaxPairs || E != 512) {
        set_error(-2, "csr path: needs 1 <= M <= %d, M*top_k <= %d, 512 experts", kMaxRows, kMaxPairs); return -2;
    }
    const bool use_csr = csr_routing_for(fmt, M);
    if (use_csr && !csr) { set_error(-1, "csr path: the routing launch needs the csr buffer"); return -1; }
    if (!pw || !ctl || K > 16) { set_error(-1, "csr path: needs the partial words and tags, top_k <= 16"); return -1; }
    ShPtrs sp{};
    if (sh) sp = *sh;
    const dim3 b256(256);
    const uint8_t *wg, *wu, *wd, *bg = nullptr, *bu = nullptr, *bd = nullptr;
    uint4 *xh = nullptr;                           // INT8: scaled fp16 activations, then their chunk (seed, 2^-k)
    float2 *xci = nullptr;
    if (fmt == QFM_FMT_INT8) {
        if (!a->i8_gate || !a->i8_up || !a->i8_down) { set_error(-1, "csr path: arena has no INT8 blobs"); return -1; }
        if (!xh16) { set_error(-1, "csr path: INT8 needs the fp16 activation buffer"); return -1; }
        xh = static_cast<uint4 *>(xh16);
        xci = reinterpret_cast<float2 *>(xh + (size_t)M * g_cfg.H / 8);
        wg = (const uint8_t *)a->i8_gate; wu = (const uint8_t *)a->i8_up; wd = (const uint8_t *)a->i8_down;
    } else {
        if (!a->w_gate || !a->s_gate || !a->s2g_dev) { set_error(-1, "csr path: arena has no NVFP4 blobs"); return -1; }
        wg = a->w_gate; wu = a->w_up; wd = a->w_down; bg = a->s_gate; bu = a->s_up; bd = a->s_down;
    }
#define QFM_CSR_KERNELS(F, HH, II, PAIRS, RT)                                                                       \
    hipLaunchKernelGGL((k_csr_gateup<F, HH, II, PAIRS>), dim3(II / (kGuThreads / gateup_lpr<F, HH>()), P),   \
                       dim3(kGuThreads), 0, s,                                                                   \
                       wg, wu, a->i8s_gate, a->i8s_up, bg, bu, a->s2g_dev, a->s2u_dev, x, xh, xci, K, RT, P,   \
                       hpair);                                                                                   \
    hipLaunchKernelGGL((k_csr_down<F, HH, II, PAIRS>), dim3(HH / down_rows<F, II>(), P + (sh ? (M + 1) / 2 : 0) + M), \
                       b256, 0, s, wd, a->i8s_down, bd, a->s2d_dev, hpair, wts, RT, P, pw, K, sp, hsh, logits, ld,      \
                       gated, M, ctl, y, y32)
#define QFM_CSR_LAUNCH(F, HH, II)                                                                                   \
    if (use_csr) {                                                                                                \
        hipLaunchKernelGGL((k_topk_csr<8>), dim3(1), dim3(xh ? 1024 : kTopkThreads), 0, s, logits, ld, M, K,      \
                           g_cfg.renorm, sel, wts, csr, x, HH, xh, xci, ctl);                                    \
        QFM_CSR_KERNELS(F, HH, II, false, csr);                                                                   \
    } else {                                                                                                      \
        QFM_CSR_KERNELS(F, HH, II, true, sel);                                                                    \
    }
    if (shape_2048()) {
        if (fmt == QFM_FMT_INT8) { QFM_CSR_LAUNCH(FmtI8, 2048, 512); } else { QFM_CSR_LAUNCH(FmtF4, 2048, 512); }
    } else if (shape_2560()) {
        if (fmt == QFM_FMT_INT8) { QFM_CSR_LAUNCH(FmtI8, 2560, 640); } else { QFM_CSR_LAUNCH(FmtF4, 2560, 640); }
    } else {
        set_error(-2, "csr path: unsupported shape"); return -2;
    }
#undef QFM_CSR_LAUNCH
#undef QFM_CSR_KERNELS
    return check_launch("csr_forward");
}

}  // namespace qfm
