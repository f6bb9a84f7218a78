// qfm_csr.hip -- multi-row decode (M <= 8 "Ocho" fork rows): weight-once-per-
// distinct-expert gate/up and down keyed by pair, INT8 and NVFP4 arenas.
//
// Reference behaviour: the M=8 CSR tier k_m8_build_csr / k_m8_gateup /
// k_m8_downacc (ocho/amd_server/qf_moe_m8_wave64.hip:72-211, :261-299) and the
// chunk path k_i8_csr_build / k_i8_gateup_csr / k_i8_downacc_csr /
// k_i8_combine (ocho/amd_server/qf8_moe_i8.hip:196-358): distinct experts in
// ascending id, the pairs of an expert in (token, k) order, every weight row
// read once per distinct expert and dotted against all rows routed to it,
// owned partials part[t][k][H] summed in k order (no atomics, deterministic).
//
// Launch sequence (all stream-ordered), after the router launch, whose
// selection tail has written sel/wts (and, INT8, the activations as scaled
// fp16 chunks):
//   k_csr_gateup   grid (I/rows, M*K), 256 threads: grid row y is pair y; it
//                  stores only if y is its expert's first pair, for all of the
//                  expert's pairs (ballots over sel, pairs_of / pairs_from).
//                  One lane group per gate/up row: the row pair is loaded
//                  once, then dotted with the LDS-staged activation row of each
//                  routed token. hidden is written per pair (row = pair id).
//                  NVFP4: workgroup (0, y) also writes pair y's descriptor for
//                  the down launch (pair_desc).
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
// An expert's pairs are visited in ascending pair id, i.e. (token, k) order,
// the order of the reference's CSR within one expert.
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
// the pair set of pair p with expert e, from s0 = sel[lane] and s1 = sel[lane +
// 64] (-1 past P) already loaded
__device__ __forceinline__ PairSet pairs_from(int s0, int s1, int e, int p) {
    const int lane = threadIdx.x & 63;
    PairSet r;
    r.e = e;
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
__device__ __forceinline__ PairSet pairs_of(const int *__restrict__ sel, int P, int p) {
    const int lane = threadIdx.x & 63;
    const int e = __builtin_amdgcn_readfirstlane(sel[p]);
    return pairs_from(lane < P ? sel[lane] : -1, lane + 64 < P ? sel[lane + 64] : -1, e, p);
}
// NVFP4: the down launch's view of grid row y, written by the gate/up launch's
// workgroup (0, y): {expert or -1 (not an owner), np, pair ids 0-3 and 4-7 as
// bytes (P <= 128)}: one 16-byte scalar load gives a down workgroup its expert
// and every pair (the ballots over sel cost a vector round trip more).
struct PairBytes {
    uint32_t lo, hi;
};
__device__ __forceinline__ int4 pair_desc(const PairSet &ps) {
    unsigned long long a = ps.a, c = ps.c;
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int j = 0; j < kMaxRows; j++) {
        if (j < ps.np) {
            const uint32_t q = (uint32_t)next_pair(a, c);
            if (j < 4) lo |= q << (8 * j);
            else hi |= q << (8 * (j - 4));
        }
    }
    return make_int4(ps.e, ps.e < 0 ? 0 : ps.np, (int)lo, (int)hi);
}
// pair j of the list (j < kMaxRows; per thread or wave-uniform)
__device__ __forceinline__ int pair_of_lane(const PairBytes &pb, int j) {
    return (int)(((j < 4 ? pb.lo : pb.hi) >> (8 * (j & 3))) & 0xFFu);
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
template <class F, int H, int I>
__global__ void __launch_bounds__(kGuThreads)
k_csr_gateup(const uint8_t *__restrict__ Wg, const uint8_t *__restrict__ Wu,
             const float *__restrict__ Sg, const float *__restrict__ Su,          // INT8 row scales
             const uint8_t *__restrict__ Bg, const uint8_t *__restrict__ Bu,      // NVFP4 block scales
             const float *__restrict__ s2g, const float *__restrict__ s2u,        // NVFP4 per-expert scale
             const uint16_t *__restrict__ x, const uint4 *__restrict__ xh, const float2 *__restrict__ xci,
             int K, const int *__restrict__ sel, int P, float *__restrict__ hpair, int4 *__restrict__ pdsc) {
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
    // grid row y is pair y; its expert's first pair (the owner) stores
    int e, np;
    unsigned long long pa = 0ull, pc = 0ull;     // pairs not staged yet, ascending
    // NVFP4 (SPEC): the pair's expert is known after one scalar load and the
    // owner test needs the ballots over sel (vector loads, ~0.35 us more per
    // block, wall-clock stamps): sel is requested, then the weights, and only
    // then are the ballots taken; a block that is not its expert's owner runs
    // without storing. INT8, bound by the weight stream, keeps the owner test
    // first (the non-owners' loads cost it more than the wait).
    constexpr bool SPEC = !I8;
    bool owner = true;
    int s0 = -1, s1 = -1;                        // SPEC: sel[lane], sel[lane + 64]
    if constexpr (SPEC) {
        const int lane = threadIdx.x & 63;
        e = __builtin_amdgcn_readfirstlane(sel[blockIdx.y]);
        s0 = lane < P ? sel[lane] : -1;
        s1 = lane + 64 < P ? sel[lane + 64] : -1;
        args_now(e, Wg, Wu);
        np = 0;
    } else {
        const PairSet ps = pairs_of(sel, P, blockIdx.y);
        args_now(ps.e, Wg, Wu);                  // (the weight bases requested with sel, before the branch)
        e = ps.e; np = ps.np; pa = ps.a; pc = ps.c;
    }
    if (e < 0) return;                           // not its expert's first pair (INT8)
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
    if constexpr (SPEC) {
        __builtin_amdgcn_sched_barrier(0);       // (the weights stay requested before the ballots wait on sel)
        const PairSet ps = pairs_from(s0, s1, e, blockIdx.y);
        owner = ps.e >= 0;
        np = ps.np; pa = ps.a; pc = ps.c;
        __builtin_assume(np >= 1);               // (pair y itself: no loop guard to sink the scale loads under)
        if (blockIdx.x == 0 && threadIdx.x == 0) pdsc[blockIdx.y] = pair_desc(ps);   // for the down launch
    }
    const uint4 *src = I8 ? xh : reinterpret_cast<const uint4 *>(x);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    static_assert(PG == 2, "two staged rows per group (pq0, pq1)");
    for (int j0 = 0; j0 < np; j0 += PG) {
        const int ng = min(PG, np - j0);
        // the group's pair ids (= their hidden rows)
        const int pq0 = next_pair(pa, pc), pq1 = next_pair(pa, pc);
        auto pair_id = [&](int j) -> int { return j == 0 ? pq0 : pq1; };
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
            if (owner && l == 0) hpair[(size_t)pair_id(j) * I + row] = silu(ag * rsg) * (au * rsu);
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
template <class F, int H, int I>
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
    // as in k_csr_gateup, grid row y - nsh is a pair, run by its expert's first
    // pair: INT8 from the ballots over sel (rt = sel), NVFP4 from the gate/up
    // launch's pair descriptor (rt = the descriptors; one scalar load; one
    // pointer for both keeps the kernel arguments in three 64-byte lines)
    constexpr bool DSC = F::VPB == 2;
    PairSet ps{};
    PairBytes pb{0u, 0u};
    int e, np;
    if constexpr (DSC) {
        const int4 dsc = reinterpret_cast<const int4 *>(rt)[blockIdx.y - nsh];   // one load before any weight
        args_now(dsc.x, dsc.y, dsc.z, dsc.w, Wd);
        e = dsc.x; np = dsc.y; pb.lo = (uint32_t)dsc.z; pb.hi = (uint32_t)dsc.w;
    } else {
        ps = pairs_of(rt, P, (int)blockIdx.y - nsh);
        args_now(ps.e, Wd);
        e = ps.e; np = ps.np;
    }
    if (e < 0) return;                           // not its expert's first pair
    const int l = threadIdx.x % LPR, grp = threadIdx.x / LPR;
    // the pairs' hidden rows first (in L2 or the memory-side cache: they arrive
    // before the weights, and loads retire in issue order, so their conversion
    // runs while the weights stream; M = 8 NVFP4 layer 47.1 -> 46.1 us)
    H16Stage<I, kMaxRows> hst;
    if constexpr (DSC) hst.load_rows(hpair, pb, np);
    else hst.load_rows(hpair, ps, np);
    // (without this barrier the scheduler issues the weights first, whose
    // addresses are ready earlier, and the conversion then waits for them)
    __builtin_amdgcn_sched_barrier(0);
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
        int pr;
        if constexpr (DSC) pr = pair_of_lane(pb, j);
        else pr = pair_at(ps, j);
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

// ---- launcher ---------------------------------------------------------------------
int launch_csr_forward(const Qf4ExpCache *a, int fmt, const ShPtrs *sh, const uint16_t *x, const float *logits,
                       int ld, int gated, int M, float *hpair, const float *hsh, const int *sel, const float *wts,
                       int4 *pdsc, void *xh16, unsigned long long *pw, uint32_t *ctl, uint16_t *y, float *y32,
                       hipStream_t s) {
    const int K = g_cfg.K, E = g_cfg.E, P = M * K;
    if (M < 1 || M > kMaxRows || P > kMaxPairs || E != 512) {
        set_error(-2, "csr path: needs 1 <= M <= %d, M*top_k <= %d, 512 experts", kMaxRows, kMaxPairs); return -2;
    }
    if (!pdsc || !pw || !ctl || K > 16) {
        set_error(-1, "csr path: needs the pair descriptors, partial words and tags, top_k <= 16"); return -1;
    }
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
#define QFM_CSR_LAUNCH(F, HH, II)                                                                                   \
    hipLaunchKernelGGL((k_csr_gateup<F, HH, II>), dim3(II / (kGuThreads / gateup_lpr<F, HH>()), P),          \
                       dim3(kGuThreads), 0, s,                                                                   \
                       wg, wu, a->i8s_gate, a->i8s_up, bg, bu, a->s2g_dev, a->s2u_dev, x, xh, xci, K, sel, P,  \
                       hpair, pdsc);                                                                             \
    hipLaunchKernelGGL((k_csr_down<F, HH, II>), dim3(HH / down_rows<F, II>(), P + (sh ? (M + 1) / 2 : 0) + M),      \
                       b256, 0, s, wd, a->i8s_down, bd, a->s2d_dev, hpair, wts,                                 \
                       fmt == QFM_FMT_INT8 ? sel : reinterpret_cast<const int *>(pdsc), P, pw, K, sp, hsh,          \
                       logits, ld, gated, M, ctl, y, y32)
    if (shape_2048()) {
        if (fmt == QFM_FMT_INT8) { QFM_CSR_LAUNCH(FmtI8, 2048, 512); } else { QFM_CSR_LAUNCH(FmtF4, 2048, 512); }
    } else if (shape_2560()) {
        if (fmt == QFM_FMT_INT8) { QFM_CSR_LAUNCH(FmtI8, 2560, 640); } else { QFM_CSR_LAUNCH(FmtF4, 2560, 640); }
    } else {
        set_error(-2, "csr path: unsupported shape"); return -2;
    }
#undef QFM_CSR_LAUNCH
    return check_launch("csr_forward");
}

}  // namespace qfm
