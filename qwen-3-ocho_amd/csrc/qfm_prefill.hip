// qfm_prefill.hip -- prefill (T tokens, T large): MFMA grouped GEMMs.
//
// Reference behaviour: the chunk path qf8_i8_experts_chunk
// (ocho/amd_server/qf8_moe_i8.hip:196-322, :372-395) and Spark's
// qf_prefill_experts_csr / qf_prefill_experts_mma
// (ocho/engine_spark/cuda/qf_prefill_moe.cu:129-265,
// ocho/engine_spark/cuda/qf_prefill_mma.cu:513-563): tokens grouped by expert,
// each expert's weights dotted against all of its tokens, owned partials per
// (token, k) summed by a combine kernel. Here the shared expert is one more
// group (every token, weight sigmoid(<g, x_t>)).
//
// Router (bit-exact selection at GEMM speed):
//   k_pf_router_mfma   logits~ = x . bf16(W)^T (+ bias) on bf16 MFMA, plus
//                      per-token ||x_t||_2; W rows' ||w_e||_2 come from
//                      k_pf_router_prep. |logit~ - logit| <= B_te =
//                      c * ||w_e|| ||x_t|| (Cauchy-Schwarz over the bf16
//                      rounding of W, the MFMA accumulation and the canonical
//                      fp32 order; constants below).
//   k_pf_select        one wave per token: tau = K-th largest (logit~ - B),
//                      candidates = {e : logit~ + B >= tau} (a superset of the
//                      exact top-K, ties included), their logits recomputed in
//                      the canonical order, then the exact top-K among them;
//                      also the exact shared-gate dot. Tokens whose candidate
//                      set overflows recompute every logit.
// Experts:
//   k_pf_count / k_pf_plan / k_pf_scatter   routing inversion: per-block LDS
//                      histograms, one planning block, LDS-counter scatter
//                      (row order inside a group is unspecified: every GEMM
//                      row is independent and partials are owned by (t, k),
//                      so y does not depend on it) and the GEMM work lists.
//   k_pf_gemm<GATEUP>  hidden[p][n] = silu(sg (x_p . Wg_n)) * (su (x_p . Wu_n))
//   k_pf_gemm<DOWN>    part[slot_p][c] = fp16(2^k * w_p * sd_c * (h_p . Wd_c)), k per 64 columns
//                      BM=128 rows x BK=64, waves of 64 x 64 on 16x16x32 MFMAs.
//                      INT8 gate/up (128 x 256 tiles, 8 waves): x rows as fp16
//                      scaled by 2^k per token, weights kept as int8 in LDS and
//                      widened at the fragment read to fp16 1024 + u
//                      (u = q + 128), f16 MFMA, 1152 * sum(x16) removed and 2^-k
//                      applied in the epilogue. INT8 down (128 x 128 tiles, 4
//                      waves, two blocks per CU): bf16 hidden rows, weights
//                      staged as bf16 u (exact), bf16 MFMA, 128 * sum(h) removed
//                      (the hidden sums come from the gate/up epilogue). NVFP4:
//                      e2m1 times its e4m3 block scale staged as bf16 (exact).
//   k_pf_combine_h     y[t] = sum over the K+1 slots of t, in slot order (fp32).
#include <type_traits>

#include "qfm_dev.h"
#include "qfm_internal.h"
#include "qfm_prefill_layout.h"

namespace qfm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int BM = 128, BN = 128;
constexpr int kCandMax = 64;

// bf16 bits of an exactly representable value (integers |v| <= 256): truncation is exact
__device__ __forceinline__ uint32_t pack_bf16_exact(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);   // high halves
}

// 16 int8 codes -> 16 bf16 in offset-binary form (q + 128, exact)
__device__ __forceinline__ void i8_to_bf16_ob(uint4 w, uint4 &o0, uint4 &o1) {
    const uint32_t d[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u, w.w ^ 0x80808080u};
    uint32_t o[8];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        o[2 * q] = pack_bf16_exact((float)(d[q] & 0xFFu), (float)((d[q] >> 8) & 0xFFu));
        o[2 * q + 1] = pack_bf16_exact((float)((d[q] >> 16) & 0xFFu), (float)(d[q] >> 24));
    }
    o0 = make_uint4(o[0], o[1], o[2], o[3]);
    o1 = make_uint4(o[4], o[5], o[6], o[7]);
}

// 16 int8 codes -> 16 fp16 1024 + u (u = q ^ 0x80 = q + 128; exact: unit
// spacing on [1024, 2048)), one v_perm_b32 per two codes
__device__ __forceinline__ void i8_to_f16_ob(uint4 w, uint4 &o0, uint4 &o1) {
    const uint32_t d[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u, w.w ^ 0x80808080u};
    uint32_t o[8];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        o[2 * q] = __builtin_amdgcn_perm(0x64646464u, d[q], 0x04010400u);
        o[2 * q + 1] = __builtin_amdgcn_perm(0x64646464u, d[q], 0x04030402u);
    }
    o0 = make_uint4(o[0], o[1], o[2], o[3]);
    o1 = make_uint4(o[4], o[5], o[6], o[7]);
}

// Two e2m1 codes of byte `sel` of w -> exact fp32 pair (unit scale), times the
// block scale s (products of a 2-bit and a 4-bit significand: exact in fp32 and
// in bf16), packed to bf16 by truncation (exact).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <int SEL>
__device__ __forceinline__ uint32_t f4_pair_bf16(uint32_t w, float s) {
    const f32x2_t v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, SEL);
    return pack_bf16_exact(v.x * s, v.y * s);
}
// 32 e2m1 codes (16 bytes, element 2i in the low nibble of byte i) with the
// two e4m3 block scales of their 16-element halves -> 32 bf16 (4 x 16 bytes)
__device__ __forceinline__ void f4_to_bf16(uint4 w, uint32_t sc2, uint4 (&o)[4]) {
    const float s0 = e4m3_scale(sc2 & 0xFFu), s1 = e4m3_scale((sc2 >> 8) & 0xFFu);
    o[0] = make_uint4(f4_pair_bf16<0>(w.x, s0), f4_pair_bf16<1>(w.x, s0), f4_pair_bf16<2>(w.x, s0), f4_pair_bf16<3>(w.x, s0));
    o[1] = make_uint4(f4_pair_bf16<0>(w.y, s0), f4_pair_bf16<1>(w.y, s0), f4_pair_bf16<2>(w.y, s0), f4_pair_bf16<3>(w.y, s0));
    o[2] = make_uint4(f4_pair_bf16<0>(w.z, s1), f4_pair_bf16<1>(w.z, s1), f4_pair_bf16<2>(w.z, s1), f4_pair_bf16<3>(w.z, s1));
    o[3] = make_uint4(f4_pair_bf16<0>(w.w, s1), f4_pair_bf16<1>(w.w, s1), f4_pair_bf16<2>(w.w, s1), f4_pair_bf16<3>(w.w, s1));
}

// ---- router prep: ||w_e||_2 (fp64 accumulate, rounded up) --------------------------
// Blocks [0, E): ||w_e||_2 (fp64 accumulate, rounded up) and bf16(W) for the
// router GEMM. Blocks [E, E + ceil(T/4)): one wave per token row, ||x_t||_2
// (fp64, rounded up) and sum(x_t) (fp32; the offset-binary correction of the
// gate/up GEMM), every load of the row in flight at once, lane partials
// combined by a butterfly (fixed order).
__global__ void __launch_bounds__(256) k_pf_router_prep(const float *__restrict__ W, int E, int H,
                                                         float *__restrict__ wnorm, uint16_t *__restrict__ wb,
                                                         const uint16_t *__restrict__ x, int T,
                                                         float *__restrict__ xnorm, float *__restrict__ xsum,
                                                         uint4 *__restrict__ x16, float *__restrict__ x16sum,
                                                         float *__restrict__ x16isc) {
    if ((int)blockIdx.x >= E) {
        constexpr int kMaxCh = 5;                    // 16-byte chunks per lane: H / 512 <= 5
        const int lane = threadIdx.x & 63;
        const int t = ((int)blockIdx.x - E) * 4 + (threadIdx.x >> 6);
        if (t >= T) return;
        const uint4 *xr = reinterpret_cast<const uint4 *>(x + (size_t)t * H);
        const int nch = H / 512;
        uint4 v[kMaxCh];
#pragma unroll
        for (int q = 0; q < kMaxCh; q++) v[q] = q < nch ? xr[q * 64 + lane] : make_uint4(0u, 0u, 0u, 0u);
        double sq = 0.0;
        float sx = 0.0f;
#pragma unroll
        for (int q = 0; q < kMaxCh; q++) {
            const uint32_t d[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float a = bf16_lo(d[u]), b = bf16_hi(d[u]);
                sq += (double)a * a + (double)b * b;
                sx += a + b;
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            sq += __shfl_xor(sq, m, WAVE);
            sx += __shfl_xor(sx, m, WAVE);
        }
        if (lane == 0) {
            xnorm[t] = (float)(sqrt(sq) * (1.0 + 1e-6));
            xsum[t] = sx;
        }
        if (x16) {
            // the row as fp16 scaled by 2^k (largest magnitude in [2^14, 2^15): no
            // overflow, bf16 values exact), with the sum of the scaled values and 2^-k
            float amax = 0.0f;
#pragma unroll
            for (int q = 0; q < kMaxCh; q++) {
                const uint32_t d[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
                for (int u = 0; u < 4; u++) amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(d[u])), fabsf(bf16_hi(d[u]))));
            }
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, WAVE));
            const int e = (int)(__float_as_uint(amax) >> 23);
            const int k = amax == 0.0f ? 0 : min(113, max(-113, 141 - e));
            const float sc = __uint_as_float((uint32_t)(127 + k) << 23);
            float hs = 0.0f;
            uint4 *xo = x16 + (size_t)t * (H / 8);
#pragma unroll
            for (int q = 0; q < kMaxCh; q++) {
                if (q >= nch) break;
                const uint32_t d[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
                uint32_t o[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const f16x2_t hp = {(_Float16)(bf16_lo(d[u]) * sc), (_Float16)(bf16_hi(d[u]) * sc)};
                    hs += (float)hp.x + (float)hp.y;
                    o[u] = __builtin_bit_cast(uint32_t, hp);
                }
                xo[q * 64 + lane] = make_uint4(o[0], o[1], o[2], o[3]);
            }
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) hs += __shfl_xor(hs, m, WAVE);
            if (lane == 0) {
                x16sum[t] = hs;
                x16isc[t] = __uint_as_float((uint32_t)(127 - k) << 23);
            }
        }
        return;
    }
    const int e = blockIdx.x;
    double s = 0.0;
    for (int k = threadIdx.x; k < H; k += 256) {
        const float w = W[(size_t)e * H + k];
        const double v = (double)w;
        s += v * v;
        wb[(size_t)e * H + k] = f32_to_bf16(w);     // the router GEMM's B operand (round to nearest even)
    }
    __shared__ double red[256];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int m = 128; m >= 1; m >>= 1) {
        if ((int)threadIdx.x < m) red[threadIdx.x] += red[threadIdx.x + m];
        __syncthreads();
    }
    if (threadIdx.x == 0) wnorm[e] = (float)(sqrt(red[0]) * (1.0 + 1e-6));
}

// ---- the MFMA tile engine ---------------------------------------------------------
// Block tile (16 MW WM) x (64 WN), WM x WN waves of (16 MW) x 64 (MW x 4
// v_mfma_f32_16x16x32_bf16 accumulators each), k-step BK2 = 64 (two 32-deep
// MFMA steps). Two LDS buffers (the k-step being multiplied and the next one)
// and NSTG (2 or 3) register stages of global loads, one barrier per k-step.
// A rows: bf16, row r at A + arow[r] * lda (arow < 0: absent row). B rows:
// int8 (staged as bf16 in offset-binary form u = q + 128, exact), bf16, or
// NVFP4 (packed e2m1 at bptr[n], e4m3 block scales per 16 at sptr[n]; staged
// as bf16 of e2m1 * scale, exact), row n at bptr[n] (bytes). K % BK2 == 0.
// acc[mb][nb][i] = C[16 MW wm + 16 mb + 4 (lane >> 4) + i][64 wn + 16 nb + (lane & 15)],
// wave = WN wm + wn. Staging: 16-byte chunks, consecutive threads on
// consecutive chunks of a row (A: 8 chunks per row, B: 4 int8 / 2 NVFP4 / 8 bf16).
//
// The register stages are named stage sets of native vector type (a
// dynamically indexed stage array went to scratch; uint4 stage members were
// promoted to LDS), and every k-step is one basic block: the global loads of
// step s + NSTG + 1 are clamped to the last k-step (a repeat of an address already
// loaded: L2 hits) and absent A rows read a row of zeros (their results are
// never stored), so no branch splits the step and the compiler schedules the
// fragment reads, MFMAs, the next step's conversion, LDS writes and global
// loads of a step together (explicit scheduling-group patterns measured
// slower than the compiler's own order).
constexpr int BK2 = 64;
// LDS rows of BK2 16-bit elements (128 bytes, eight 16-byte chunks), chunk q
// of row r stored at chunk position q ^ (r & 7). The MFMA fragment reads (16
// rows at one chunk per 16 lanes) and the staging writes are then free of
// bank conflicts; rows padded to 144 bytes cost four conflict cycles per
// fragment read (measured with SQ_LDS_BANK_CONFLICT on ds_read_b128).
constexpr int LDS2 = BK2;
__device__ __forceinline__ int lds_swz(int r, int q) { return r * LDS2 + ((q ^ (r & 7)) << 3); }
template <int BMt, int BNt, int BROW = LDS2>
struct TileLds {
    uint16_t a[2][BMt * LDS2];
    uint16_t b[2][BNt * BROW];                 // BROW 16-bit units per B row
};
// B row modes: int8 staged as bf16 (offset binary) or as fp16 (1024 + u), bf16,
// NVFP4 staged as bf16, or int8 kept as int8 in LDS (64-byte rows) and widened
// to fp16 at the fragment read (half the LDS bytes written and read for B).
enum { kB_I8 = 0, kB_BF16 = 2, kB_F4 = 3, kB_I8H = 4, kB_I8HL = 5 };
// int8 B rows in LDS: 8-byte chunk c of row r at chunk position c ^ (2 ((r >> 2) & 3)).
// A fragment read (16 rows at one chunk per 16 lanes, ds_read_b64) is then free
// of bank conflicts (6 conflict cycles per instruction unswizzled), and the two
// chunks a staging thread writes stay one aligned 16-byte pair.
__device__ __forceinline__ int lds_swz8(int r, int c) { return r * (LDS2 / 2) + ((c ^ (2 * ((r >> 2) & 3))) << 2); }
// 8 int8 codes -> 8 fp16 1024 + u (as i8_to_f16_ob)
__device__ __forceinline__ f16x8_t i8x8_to_f16_ob(uint32_t w0, uint32_t w1) {
    const uint32_t d0 = w0 ^ 0x80808080u, d1 = w1 ^ 0x80808080u;
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v o = {__builtin_amdgcn_perm(0x64646464u, d0, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, d0, 0x04030402u),
                      __builtin_amdgcn_perm(0x64646464u, d1, 0x04010400u), __builtin_amdgcn_perm(0x64646464u, d1, 0x04030402u)};
    return __builtin_bit_cast(f16x8_t, o);
}
// The A row that absent rows of a partial tile read: zeros (zero-initialized
// device memory, never written), at least as long as any K here. Multiplying
// zeros instead of a duplicated present row measured 2-3% faster on the
// gate/up GEMMs (same results: those rows are never stored).
constexpr int kZeroRowElems = 4096;
static __device__ __align__(256) uint16_t g_zero_row[kZeroRowElems];
template <int BMODE, int WM, int WN, int MW, int NSTG>
struct TileEngine {
    static_assert(NSTG == 2 || NSTG == 3, "two or three register stages");
    static constexpr bool BL8 = BMODE == kB_I8HL;                  // int8 B rows in LDS
    using Lds = TileLds<16 * MW * WM, 64 * WN, BL8 ? LDS2 / 2 : LDS2>;
    static constexpr int WMc = WM, WNc = WN, MWc = MW, WavesPerSimd = 2;
    static_assert(BMODE == kB_I8 || BMODE == kB_I8H || BMODE == kB_I8HL || BMODE == kB_F4 || BMODE == kB_BF16,
                  "int8 (bf16 or fp16 staging, or int8 in LDS), NVFP4 or bf16 B rows");
    static constexpr bool B8 = BMODE == kB_I8 || BMODE == kB_I8H || BL8;   // one byte per B value
    // MW m-blocks of 16 rows per wave: a wave computes (16 MW) x 64
    static constexpr int BMt = 16 * MW * WM, BNt = 64 * WN, NT = 64 * WM * WN;
    static constexpr int BCPR = B8 ? 4 : BMODE == kB_F4 ? 2 : 8;   // 16-byte B chunks per row per k-step
    static constexpr int NA = BMt * 8 / NT, NB = BNt * BCPR / NT;      // chunks per thread
    static_assert(NA * NT == BMt * 8 && NB * NT == BNt * BCPR, "staging must divide evenly");
    struct Stage {                                // native vector types: SROA keeps them in registers
        u32x4_t a[NA], b[NB];                     // (with uint4 the stages were promoted to LDS or scratch)
        uint32_t sc[NB];
    };
    __device__ static void run(const uint16_t *__restrict__ A, long lda, const int *arow,
                               const char *const *bptr, int K, Lds &L, f32x4_t (&acc)[MW][4],
                               const char *const *sptr = nullptr) {
        const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
        const int wm = wave / WN, wn = wave % WN;
        const uint16_t *ap[NA];
        int a_lds[NA];
#pragma unroll
        for (int j = 0; j < NA; j++) {
            const int c = t + j * NT, r = c >> 3, kc = c & 7;
            const int ar = arow[r];
            ap[j] = (ar >= 0 ? A + (long)ar * lda : g_zero_row) + kc * 8;
            a_lds[j] = lds_swz(r, kc);
        }
        // the row pointers come from an LDS table of generic pointers: address
        // them as global memory, or the loads become flat loads, which count
        // against lgkmcnt and make every LDS wait of the k-step wait for them
        typedef const __attribute__((address_space(1))) char *gptr_t;
        gptr_t bp[NB], sp[NB];
        int b_lds[NB];
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const int c = t + j * NT, r = c / BCPR, kc = c % BCPR;
            bp[j] = (gptr_t)bptr[r] + kc * 16;
            sp[j] = BMODE == kB_F4 ? (gptr_t)sptr[r] + kc * 2 : nullptr;
            // first 16-byte chunk of the thread's 1, 2 (int8) or 4 (NVFP4)
            // consecutive chunks; chunk h of them is at b_lds[j] ^ (8 h)
            b_lds[j] = BL8 ? lds_swz8(r, kc * 2) : lds_swz(r, B8 ? kc * 2 : BMODE == kB_F4 ? kc * 4 : kc);
        }
        auto gload = [&](int k0, Stage &g) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < NA; j++) g.a[j] = *reinterpret_cast<const u32x4_t *>(ap[j] + k0);
#pragma unroll
            for (int j = 0; j < NB; j++) {
                typedef const __attribute__((address_space(1))) u32x4_t *gv_t;
                typedef const __attribute__((address_space(1))) uint16_t *gs_t;
                if constexpr (B8) {
                    g.b[j] = *reinterpret_cast<gv_t>(bp[j] + k0);
                } else if constexpr (BMODE == kB_BF16) {
                    g.b[j] = *reinterpret_cast<gv_t>(bp[j] + (size_t)k0 * 2);
                } else {
                    g.b[j] = *reinterpret_cast<gv_t>(bp[j] + k0 / 2);
                    g.sc[j] = *reinterpret_cast<gs_t>(sp[j] + k0 / 16);
                }
            }
        };
        auto sstore = [&](int buf, const Stage &g) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < NA; j++) *reinterpret_cast<u32x4_t *>(&L.a[buf][a_lds[j]]) = g.a[j];
#pragma unroll
            for (int j = 0; j < NB; j++) {
                uint16_t *lb = L.b[buf];
                const int bo = b_lds[j];
                const uint4 bw = make_uint4(g.b[j].x, g.b[j].y, g.b[j].z, g.b[j].w);
                if constexpr (BMODE == kB_BF16 || BL8) {
                    *reinterpret_cast<uint4 *>(lb + bo) = bw;
                } else if constexpr (B8) {
                    uint4 o0, o1;
                    if constexpr (BMODE == kB_I8H) i8_to_f16_ob(bw, o0, o1);
                    else i8_to_bf16_ob(bw, o0, o1);
                    *reinterpret_cast<uint4 *>(lb + bo) = o0;
                    *reinterpret_cast<uint4 *>(lb + (bo ^ 8)) = o1;
                } else {
                    uint4 o[4];
                    f4_to_bf16(bw, g.sc[j], o);
#pragma unroll
                    for (int q = 0; q < 4; q++) *reinterpret_cast<uint4 *>(lb + (bo ^ (8 * q))) = o[q];
                }
            }
        };
#pragma unroll
        for (int mb = 0; mb < MW; mb++)
#pragma unroll
            for (int nb = 0; nb < 4; nb++) acc[mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        const int nk = K / BK2;
        // fragment rows start at multiples of 16, so row & 7 == lr & 7
        const int lr = lane & 15, fq0 = ((lane >> 4) ^ (lr & 7)) << 3;   // chunk position of kk = 0; kk = 1: ^ 32
        const int fb0 = ((lane >> 4) ^ (2 * ((lr >> 2) & 3))) << 2;      // int8 B rows: kk = 0; kk = 1: ^ 16
        // one k-step: MFMAs on LDS buffer s & 1, then stage `nx` (holding step
        // s + 1) goes to the other buffer and is refilled with step s + NSTG + 1
        auto step = [&](int s, Stage &nx) __attribute__((always_inline)) {
            const int buf = s & 1;
            bf16x8_t av[2][MW], bv[2][4];
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
#pragma unroll
                for (int mb = 0; mb < MW; mb++)
                    av[kk][mb] = *reinterpret_cast<const bf16x8_t *>(&L.a[buf][(wm * 16 * MW + mb * 16 + lr) * LDS2 + (fq0 ^ (kk * 32))]);
#pragma unroll
                for (int nb = 0; nb < 4; nb++) {
                    if constexpr (BL8) {
                        const uint2 w8 = *reinterpret_cast<const uint2 *>(&L.b[buf][(wn * 64 + nb * 16 + lr) * (LDS2 / 2) + (fb0 ^ (kk * 16))]);
                        bv[kk][nb] = __builtin_bit_cast(bf16x8_t, i8x8_to_f16_ob(w8.x, w8.y));
                    } else {
                        bv[kk][nb] = *reinterpret_cast<const bf16x8_t *>(&L.b[buf][(wn * 64 + nb * 16 + lr) * LDS2 + (fq0 ^ (kk * 32))]);
                    }
                }
            }
#pragma unroll
            for (int kk = 0; kk < 2; kk++)
#pragma unroll
                for (int mb = 0; mb < MW; mb++)
#pragma unroll
                    for (int nb = 0; nb < 4; nb++)
                        if constexpr (BMODE == kB_I8H || BL8)
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, av[kk][mb]),
                                                                                __builtin_bit_cast(f16x8_t, bv[kk][nb]),
                                                                                acc[mb][nb], 0, 0, 0);
                        else
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[kk][mb], bv[kk][nb], acc[mb][nb], 0, 0, 0);
            sstore(buf ^ 1, nx);
            gload(min(s + NSTG + 1, nk - 1) * BK2, nx);
            __syncthreads();
        };
        if constexpr (NSTG == 2) {
            Stage s0, s1;                              // stage (s mod 2) holds k-step s
            gload(0, s0);
            gload(min(1, nk - 1) * BK2, s1);
            sstore(0, s0);
            gload(min(2, nk - 1) * BK2, s0);
            __syncthreads();
            int s = 0;
            for (; s + 2 <= nk; s += 2) {
                step(s, s1);
                step(s + 1, s0);
            }
            if (s < nk) step(s, s1);
        } else {
            Stage s0, s1, s2;                          // stage (s mod 3) holds k-step s
            gload(0, s0);
            gload(min(1, nk - 1) * BK2, s1);
            gload(min(2, nk - 1) * BK2, s2);
            sstore(0, s0);
            gload(min(3, nk - 1) * BK2, s0);
            __syncthreads();
            int s = 0;
            for (; s + 3 <= nk; s += 3) {
                step(s, s1);
                step(s + 1, s2);
                step(s + 2, s0);
            }
            if (s < nk) step(s, s1);
            if (s + 1 < nk) step(s + 1, s2);
        }
    }
};

// router GEMM: 128 x 128 tiles, 2 x 2 waves; grouped expert GEMMs: 128 x 256, 2 x 4 waves
using RouterEngine = TileEngine<kB_BF16, 2, 2, 4, 2>;
// router GEMM slices along H, summed in slice order by k_pf_select (2 measured
// 5% slower than 1 at T = 8038: the 63 m-tiles x 4 n-tiles already fill the chip)
constexpr int kRouterKS = 1;
// INT8 tiles: 128 x 256 in 8 waves of 64 x 64 (two waves per SIMD). Four
// waves of 128 x 64 (MW = 8: one wave per SIMD, accumulators in AGPRs, 25%
// fewer LDS reads per MFMA) measured 1343 / 1149 us against 797 / 719 us.
// INT8 gate/up: int8 weights kept as int8 in LDS and widened to fp16 at the
// fragment read (one v_perm per two codes) against the fp16 x rows; widening
// while staging (fp16 B rows in LDS) measured 677 vs 639 us
using ExpertEngine = TileEngine<kB_I8HL, 2, 4, 4, 2>;
// INT8 down tiles: 128 x 128 in 4 waves, two blocks per CU (K = I is short, so
// one block's prologue and epilogue overlap the other block's k-steps). The
// weights are widened to bf16 while staging: int8 in LDS widened at the
// fragment read to bf16 (seven operations per four codes, done by both wave
// rows) measured 551 vs 542 us.
using DownEngineI8 = TileEngine<kB_I8, 2, 2, 4, 2>;
// NVFP4 launches: e2m1 tiles and the shared expert's INT8 tiles in one kernel
// (three register stages: loads four k-steps ahead; gate/up 831 -> 737 us.
// The INT8 engines and the router keep two: a third measured no faster for
// INT8 and cost the router GEMM its second wave per SIMD.)
using ExpertEngineF4 = TileEngine<kB_F4, 2, 4, 4, 3>;
using SharedEngineI8 = TileEngine<kB_I8, 2, 4, 4, 3>;     // shared tiles inside the NVFP4 launch
// weight rows per grouped-GEMM tile (gate/up: half gate, half up rows)
constexpr int GBN_I8 = ExpertEngine::BNt, GBN_F4 = ExpertEngineF4::BNt;

// Workgroups are dispatched to the 8 XCDs round-robin (block b on XCD b % 8).
// Map block b to tile (m, n) so that the nt n-tiles of one m-tile run back to
// back on the same XCD, whose L2 then serves the m-tile's A rows nt times.
// Bijective on [0, 8 * ceil(mt / 8) * nt).
__device__ __forceinline__ void xcd_tile(int b, int nt, int &m, int &n) {
    const int x = b & 7, slot = b >> 3;
    m = (slot / nt) * 8 + x;
    n = slot - (slot / nt) * nt;
}

// Gate/up GEMM order: XCD x takes the contiguous m-tile range [x c, (x + 1) c),
// c = ceil(mtot / 8), each m-tile's nt n-tiles back to back, so the m-tiles of
// one expert (which read the same weight tiles) share one XCD's L2: 621 vs
// 634 us against xcd_tile in interleaved runs (the down GEMM, whose weight
// tiles are a quarter the size, measured 542 vs 538 us and keeps xcd_tile).
// False for the blocks past the XCD's range (the grid is sized for a bound on
// the m-tiles).
__device__ __forceinline__ bool xcd_tile_contig(int b, int nt, int mtot, int &m, int &n) {
    const int x = b & 7, slot = b >> 3, c = (mtot + 7) >> 3;
    const int ml = slot / nt;
    n = slot - ml * nt;
    m = x * c + ml;
    return ml < c && m < mtot;
}

// ---- router GEMM: logits~ [T][E] --------------------------------------------------
__global__ void __launch_bounds__(256)
k_pf_router_mfma(const uint16_t *__restrict__ x, int T, int H, const uint16_t *__restrict__ Wb, int E,
                 float *__restrict__ lg_part) {
    __shared__ __align__(16) TileLds<RouterEngine::BMt, RouterEngine::BNt> lds;
    __shared__ int arow[BM];
    __shared__ const char *bptr[BN];
    int mt, et;
    const int ks = blockIdx.y, Hk = H / kRouterKS, k0 = ks * Hk;     // this block's slice of H
    xcd_tile(blockIdx.x, E / BN, mt, et);
    if (mt * BM >= T) return;
    const int t0 = mt * BM, e0 = et * BN;
    if (threadIdx.x < BM) arow[threadIdx.x] = (t0 + (int)threadIdx.x < T) ? t0 + (int)threadIdx.x : -1;
    if (threadIdx.x < BN) bptr[threadIdx.x] = reinterpret_cast<const char *>(Wb + (size_t)(e0 + threadIdx.x) * H + k0);
    __syncthreads();
    f32x4_t acc[4][4];
    RouterEngine::run(x + k0, H, arow, bptr, Hk, lds, acc);
    float *lg_approx = lg_part + (size_t)ks * T * E;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wm = wave >> 1, wn = wave & 1;
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
        for (int nb = 0; nb < 4; nb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = wm * 64 + mb * 16 + (lane >> 4) * 4 + i, c = wn * 64 + nb * 16 + (lane & 15);
                if (t0 + r < T) lg_approx[(size_t)(t0 + r) * E + e0 + c] = acc[mb][nb][i];
            }
}

// canonical-order dot of one router row with one token, computed by a full wave
template <int NJ>
__device__ __forceinline__ float canon_dot_wave(const float *__restrict__ w, const uint16_t *__restrict__ x, int lane) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const float4 wv = *reinterpret_cast<const float4 *>(w + j * 256 + lane * 4);
        const uint2 p = *reinterpret_cast<const uint2 *>(x + j * 256 + lane * 4);
        a = __fmaf_rn(wv.x, bf16_lo(p.x), a);
        a = __fmaf_rn(wv.y, bf16_hi(p.x), a);
        a = __fmaf_rn(wv.z, bf16_lo(p.y), a);
        a = __fmaf_rn(wv.w, bf16_hi(p.y), a);
    }
    return canon_butterfly(a);
}

// The same canonical dot for CB router rows at once (x held in registers):
// the CB rows' loads are all in flight before the first multiply and the CB
// fma chains and butterflies are independent. Each dot keeps the order above.
template <int NJ, int CB>
__device__ __forceinline__ void canon_dot_wave_batch(const float *__restrict__ W, int H, const int (&e)[CB],
                                                     const float (&xv)[NJ][4], int lane, float (&out)[CB]) {
    float4 wv[CB][NJ];
#pragma unroll
    for (int c = 0; c < CB; c++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
            wv[c][j] = *reinterpret_cast<const float4 *>(W + (size_t)e[c] * H + j * 256 + lane * 4);
#pragma unroll
    for (int c = 0; c < CB; c++) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            a = __fmaf_rn(wv[c][j].x, xv[j][0], a);
            a = __fmaf_rn(wv[c][j].y, xv[j][1], a);
            a = __fmaf_rn(wv[c][j].z, xv[j][2], a);
            a = __fmaf_rn(wv[c][j].w, xv[j][3], a);
        }
        out[c] = a;
    }
#pragma unroll
    for (int c = 0; c < CB; c++) out[c] = canon_butterfly(out[c]);
}

// Error-bound constant per unit of ||w_e|| ||x_t||: bf16 rounding of W
// (2^-9), MFMA fp32 accumulation over H products (<= 2 H ulps, any order),
// canonical order (H/64 + 6 roundings), with a factor-2 margin.
__device__ __forceinline__ float bound_coeff(int H) {
    return 2.0f * (0x1p-9f + (float)(2 * H) * 0x1p-24f + (float)(H / 64 + 8) * 0x1p-24f);
}

// one wave per token: candidates, exact logits, exact top-K, shared gate
template <int NJ, int EPL>
__global__ void __launch_bounds__(256)
k_pf_select(const uint16_t *__restrict__ x, int T, const float *__restrict__ W, const float *__restrict__ bias,
            const float *__restrict__ g, float *__restrict__ lg_approx, const float *__restrict__ xnorm,
            const float *__restrict__ wnorm, int K, int renorm, int *__restrict__ sel, float *__restrict__ wts,
            float *__restrict__ gam, int *__restrict__ n_fallback) {
    constexpr int H = NJ * 256, E = EPL * 64;
    __shared__ int s_cand[4][kCandMax];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + wave;
    if (t >= T) return;
    const uint16_t *xt = x + (size_t)t * H;
    const float cB = bound_coeff(H) * xnorm[t];
    float lo[EPL], hi[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = i * 64 + lane;
        float l = 0.0f;
#pragma unroll
        for (int q = 0; q < kRouterKS; q++) l += __builtin_nontemporal_load(&lg_approx[((size_t)q * T + t) * E + e]);   // slice order
        if (bias) l += bias[e];
        // the approximate logits, the x row and their write-back are touched once per
        // token: nontemporal, so the router rows of the candidates stay in L2
        __builtin_nontemporal_store(l, &lg_approx[(size_t)t * E + e]);          // the view's approximate logits
        const float b = cB * wnorm[e] + 1e-6f * (fabsf(l) + (bias ? fabsf(bias[e]) : 0.0f) + 1.0f);
        lo[i] = l - b;
        hi[i] = l + b;
    }
    // tau = K-th largest lower bound (K rounds of a wave-wide maximum)
    float tau;
    {
        // K-th largest of lo[] by repeated wave max (K <= 16, values need not be distinct)
        unsigned long long kk[EPL];
#pragma unroll
        for (int i = 0; i < EPL; i++) kk[i] = topk_key(lo[i], i * 64 + lane);
        unsigned long long b = 0;
        for (int k = 0; k < K; k++) {
            b = 0;
#pragma unroll
            for (int i = 0; i < EPL; i++) b = kk[i] > b ? kk[i] : b;
            b = __ockl_wfred_max_u64(b);
#pragma unroll
            for (int i = 0; i < EPL; i++) kk[i] = kk[i] == b ? 0ull : kk[i];
        }
        tau = topk_key_value(b);
    }
    // candidates: hi >= tau
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < EPL; i++) cnt += hi[i] >= tau ? 1 : 0;
    const unsigned long long ltm = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int off = 0, total = 0;
#pragma unroll
    for (int bt = 0; bt < 5; bt++) {
        const unsigned long long bb = __ballot((cnt >> bt) & 1);
        off += __popcll(bb & ltm) << bt;
        total += __popcll(bb) << bt;
    }
    // Without renormalization the weights divide by the softmax denominator over
    // all E logits, so every logit is recomputed exactly (the M <= 8 path's
    // denominator, bit for bit); a candidate overflow also takes every expert.
    const bool overflow = total > kCandMax;
    const bool full = overflow || !renorm;
    if (!full) {
#pragma unroll
        for (int i = 0; i < EPL; i++)
            if (hi[i] >= tau) s_cand[wave][off++] = i * 64 + lane;
    } else if (overflow && lane == 0) {
        atomicAdd(n_fallback, 1);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const int nc = full ? E : total;
    // exact logits of the candidates (all E on overflow) -> 64-bit keys; lane k < K
    // keeps the k-th best key so far (descending), maintained by insertion
    unsigned long long best = 0;
    float xv[NJ][4];                                // this token's x slice, canonical lane layout
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const u32x2_t p = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(xt + j * 256 + lane * 4));
        xv[j][0] = bf16_lo(p.x); xv[j][1] = bf16_hi(p.x); xv[j][2] = bf16_lo(p.y); xv[j][3] = bf16_hi(p.y);
    }
    constexpr int CB = 4;                           // candidates per batch of loads
    float exl[EPL];                                 // full: exact logit of expert i * 64 + lane
#pragma unroll
    for (int i = 0; i < EPL; i++) exl[i] = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += CB) {
        int eb[CB];
#pragma unroll
        for (int q = 0; q < CB; q++) {
            const int c = c0 + q < nc ? c0 + q : c0;  // past the end: repeat a candidate, result dropped
            eb[q] = full ? c : s_cand[wave][c];
        }
        float lb[CB];
        canon_dot_wave_batch<NJ, CB>(W, H, eb, xv, lane, lb);
#pragma unroll
        for (int q = 0; q < CB; q++) {
            if (c0 + q >= nc) break;
            float l = lb[q];
            if (bias) l = __fadd_rn(l, bias[eb[q]]);
            if (full) {                             // keep it in the lane that owns expert eb[q]
#pragma unroll
                for (int i = 0; i < EPL; i++)
                    if (eb[q] == i * 64 + lane) exl[i] = l;
            }
            const unsigned long long key = topk_key(l, eb[q]);
            // insert into the sorted lane list: lanes with a smaller key shift down
            const unsigned long long prev = __shfl_up(best, 1, WAVE);
            const bool ge_prev = lane == 0 || prev > key;
            if (lane < K && best < key) best = ge_prev ? key : prev;
        }
    }
    const float mx = topk_key_value(__shfl(best, 0, WAVE));
    const float ek = lane < K ? __expf(topk_key_value(best) - mx) : 0.0f;
    float denom = __ockl_wfred_add_f32(ek);
    if (!renorm) {                                  // every logit is exact here (full)
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; i++) s += __expf(exl[i] - mx);
        denom = __ockl_wfred_add_f32(s);
    }
    if (lane < K) {
        sel[(size_t)t * K + lane] = topk_key_index(best);
        wts[(size_t)t * K + lane] = ek / denom;
    }
    if (g) {
        const int e0[1] = {0};
        float gdv[1];
        canon_dot_wave_batch<NJ, 1>(g, H, e0, xv, lane, gdv);   // x from registers
        const float gd = gdv[0];
        if (lane == 0) gam[t] = sigmoid(gd);
    }
}

// ---- routing inversion --------------------------------------------------------------
constexpr int kPairsPerBlk = 4096;            // routed pairs per counting / scatter block

// Per-block expert histograms of the routed pairs, in LDS (no global atomics:
// a skewed router puts most pairs on a few experts).
__global__ void __launch_bounds__(256)
k_pf_count(const int *__restrict__ sel, int TK, int E, int *__restrict__ blk) {
    __shared__ int h[1024];
    for (int i = threadIdx.x; i < E; i += 256) h[i] = 0;
    __syncthreads();
    const int p0 = blockIdx.x * kPairsPerBlk, p1 = min(TK, p0 + kPairsPerBlk);
    for (int p = p0 + threadIdx.x; p < p1; p += 256) atomicAdd(&h[sel[p]], 1);
    __syncthreads();
    for (int i = threadIdx.x; i < E; i += 256) blk[(size_t)blockIdx.x * E + i] = h[i];
}

// One block of 1024 threads (G = E + has_sh <= 1024 groups): per-expert totals,
// blk turned in place into each block's exclusive prefix over the earlier
// blocks, group offsets off[0..G], and the GEMM work lists: item = (group,
// row0, rows, n-tile) for every 128-row m-tile of every group, n-tiles fastest,
// written by all threads (a hot expert owns most of the m-tiles).
__global__ void __launch_bounds__(1024)
k_pf_plan(int *__restrict__ blk, int nblk, int E, int has_sh, int T, int nt_gu, int nt_dn, int *__restrict__ off,
          int4 *__restrict__ items_gu, int4 *__restrict__ items_dn, int *__restrict__ n_items, int max_gu,
          int max_dn) {
    __shared__ int s_cnt[1024], s_mt[1024], s_off[1024], sa[1024], sb[1024];
    const int G = E + (has_sh ? 1 : 0);
    const int g = threadIdx.x;
    int c = 0;
    if (g < E) {
        int run = 0;
        for (int b0 = 0; b0 < nblk; b0 += 16) {      // 16 loads in flight, then the stores
            int v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = b0 + j < nblk ? blk[(size_t)(b0 + j) * E + g] : 0;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                if (b0 + j < nblk) blk[(size_t)(b0 + j) * E + g] = run;
                run += v[j];
            }
        }
        c = run;
    } else if (g == E && has_sh) {
        c = T;
    }
    const int mt = (c + BM - 1) / BM;
    sa[g] = c;
    sb[g] = mt;
    __syncthreads();
    for (int st = 1; st < 1024; st <<= 1) {      // inclusive scans of counts and m-tiles
        const int a = g >= st ? sa[g - st] : 0, b = g >= st ? sb[g - st] : 0;
        __syncthreads();
        sa[g] += a;
        sb[g] += b;
        __syncthreads();
    }
    s_cnt[g] = c;
    s_mt[g] = sb[g] - mt;                        // exclusive: first m-tile of group g
    s_off[g] = sa[g] - c;                        // exclusive: first pair of group g
    if (g <= G) off[g] = sa[g] - c;              // groups >= G are empty: off[G] = all pairs
    __syncthreads();
    const int mtot = s_mt[G];
    if (g == 0) { n_items[0] = mtot * nt_gu; n_items[1] = mtot * nt_dn; }
    // one thread per m-tile: its group (one search), then its n-tiles' items of
    // both lists, each stored at the index of the GEMM block that runs it (the
    // inverses of xcd_tile_contig and xcd_tile), as {group, first pair, rows,
    // n-tile}: a GEMM block then needs one load to know its tile
    const int cgu = (mtot + 7) >> 3;             // gate/up: m-tiles per XCD
    for (int m = g; m < mtot; m += 1024) {
        int lo = 0, hi = G - 1;                      // last group whose first m-tile is <= m
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_mt[mid] <= m) lo = mid; else hi = mid - 1;
        }
        const int row0 = (m - s_mt[lo]) * BM, rows = min(BM, s_cnt[lo] - row0), pb = s_off[lo] + row0;
        const int xg = m / cgu, mlg = m - xg * cgu;
        for (int n = 0; n < nt_gu; n++) {
            const int b = ((mlg * nt_gu + n) << 3) | xg;
            if (b < max_gu) items_gu[b] = make_int4(lo, pb, rows, n);
        }
        for (int n = 0; n < nt_dn; n++) {
            const int b = (((m >> 3) * nt_dn + n) << 3) | (m & 7);
            if (b < max_dn) items_dn[b] = make_int4(lo, pb, rows, n);
        }
    }
}

// pair -> group position. Routed pairs: block b starts expert e at off[e] +
// blk[b][e] and places its pairs with LDS counters; shared-expert pairs
// (blocks past the routed ones) in token order.
__global__ void __launch_bounds__(256)
k_pf_scatter(const int *__restrict__ sel, const float *__restrict__ wts, const float *__restrict__ gam, int T, int K,
             int E, int has_sh, const int *__restrict__ off, const int *__restrict__ blk, int *__restrict__ p_tok,
             int *__restrict__ p_slot, float *__restrict__ p_wt) {
    __shared__ int ctr[1024];
    const int S = K + has_sh, TK = T * K;
    const int nblk = (TK + kPairsPerBlk - 1) / kPairsPerBlk;
    if ((int)blockIdx.x < nblk) {
        for (int i = threadIdx.x; i < E; i += 256) ctr[i] = off[i] + blk[(size_t)blockIdx.x * E + i];
        __syncthreads();
        const int p0 = blockIdx.x * kPairsPerBlk, p1 = min(TK, p0 + kPairsPerBlk);
        for (int p = p0 + threadIdx.x; p < p1; p += 256) {
            const int e = sel[p], t = p / K, k = p - t * K;
            const int pos = atomicAdd(&ctr[e], 1);
            p_tok[pos] = t; p_slot[pos] = t * S + k; p_wt[pos] = wts[p];
        }
    } else if (has_sh) {
        const int t = ((int)blockIdx.x - nblk) * 256 + threadIdx.x;
        if (t < T) {
            const int pos = off[E] + t;
            p_tok[pos] = t; p_slot[pos] = t * S + K; p_wt[pos] = gam ? gam[t] : 1.0f;
        }
    }
}

// ---- grouped expert GEMMs -------------------------------------------------------------
struct GroupW {
    const int8_t *w;      // routed arena blob: INT8 [E][rows][K], or NVFP4 packed e2m1 [E][rows][K/2]
    const float *s;       // INT8 routed row scales [E][rows]
    const int8_t *w_sh;   // shared expert [rows][K] (INT8 in both formats)
    const float *s_sh;    // shared row scales [rows]
    const uint8_t *sc4;   // NVFP4 e4m3 block scales [E][rows][K/16]
    const float *s2;      // NVFP4 per-expert global scales [E]
};

// MODE kAllI8: every tile INT8. kRoutedF4: routed tiles (grp < E) of an
// NVFP4 arena (block scales staged into the bf16 B tile, the global scale s2
// applied in the epilogue) and the shared expert's tiles, INT8 in both formats.
// kDownI8: INT8 down on 128 x 128 tiles (DownEngineI8).
enum { kAllI8 = 0, kRoutedF4 = 1, kDownI8 = 2 };
template <int MODE>
using GemmEngine = std::conditional_t<MODE == kDownI8, DownEngineI8,
                                      std::conditional_t<MODE == kAllI8, ExpertEngine, ExpertEngineF4>>;
template <bool GATEUP, int MODE>
__global__ void __launch_bounds__(GemmEngine<MODE>::NT)
__attribute__((amdgpu_waves_per_eu(GemmEngine<MODE>::WavesPerSimd, GemmEngine<MODE>::WavesPerSimd)))
k_pf_gemm(const int4 *__restrict__ items, const int *__restrict__ n_items, int which, const int *__restrict__ p_tok, const int *__restrict__ p_slot, const float *__restrict__ p_wt,
          const uint16_t *__restrict__ A, int Kdim, int Nrows, GroupW g0, GroupW g1, int E,
          uint16_t *__restrict__ hid, uint16_t *__restrict__ part, int8_t *__restrict__ partk, int Hout, int ntiles,
          const float *__restrict__ xsum, float *__restrict__ hsum, int nt_gu, const float *__restrict__ xisc) {
    static_assert(MODE != kDownI8 || !GATEUP, "the narrow tiles are for the down GEMM");
    using Eng = GemmEngine<MODE>;
    constexpr int WN = Eng::WNc, TBN = Eng::BNt;
    static_assert(Eng::BMt == BM, "tiles of BM rows");
    constexpr bool H16 = MODE == kAllI8;            // fp16 A rows (scaled per token) and fp16-widened int8
    __shared__ __align__(16) typename Eng::Lds lds;
    __shared__ int arow[BM];
    __shared__ const char *bptr[TBN];
    constexpr bool F4 = MODE == kRoutedF4;
    __shared__ const char *sptr[F4 ? TBN : 1];
    __shared__ float rsum[BM], rscl[H16 ? BM : 1];
    __shared__ int rslot[GATEUP ? 1 : BM];          // down: the owned partial slot of each row
    __shared__ float rwt[GATEUP ? 1 : BM];          // down: the routing weight of each row
    // the tile count and this block's item (stored at the block's index by
    // k_pf_plan) as two independent loads ahead of the first branch
    const int nit = n_items[which];
    const int4 it = items[blockIdx.x];
    args_now(nit, it.x, it.y, it.z, it.w);
    int mi, ni;
    if constexpr (GATEUP) {
        if (!xcd_tile_contig(blockIdx.x, ntiles, nit / ntiles, mi, ni)) return;
    } else {
        xcd_tile(blockIdx.x, ntiles, mi, ni);
        if (mi * ntiles >= nit) return;
    }
    const int grp = it.x, pbase = it.y, rows = it.z, nt = it.w;
    const bool f4 = F4 && grp < E;
    const size_t rowb = f4 ? (size_t)Kdim / 2 : (size_t)Kdim;       // weight row bytes
    const int8_t *Wb, *Wb2 = nullptr;
    const float *Sb = nullptr, *Sb2 = nullptr;
    const uint8_t *Cb = nullptr, *Cb2 = nullptr;
    float s2a = 1.0f, s2b = 1.0f;
    if (grp < E) {
        Wb = g0.w + (size_t)grp * Nrows * rowb;
        if (f4) { Cb = g0.sc4 + (size_t)grp * Nrows * (Kdim / 16); s2a = g0.s2[grp]; }
        else Sb = g0.s + (size_t)grp * Nrows;
        if (GATEUP) {
            Wb2 = g1.w + (size_t)grp * Nrows * rowb;
            if (f4) { Cb2 = g1.sc4 + (size_t)grp * Nrows * (Kdim / 16); s2b = g1.s2[grp]; }
            else Sb2 = g1.s + (size_t)grp * Nrows;
        }
    } else {
        Wb = g0.w_sh; Sb = g0.s_sh;
        if (GATEUP) { Wb2 = g1.w_sh; Sb2 = g1.s_sh; }
    }
    // A row sums (the offset-binary correction): x rows' sums for gate/up; for
    // down, the sum of the nt_gu per-tile partial sums the gate/up epilogue
    // wrote for the pair's bf16 hidden row (fixed order: deterministic)
    if (threadIdx.x < BM) {
        const int r = threadIdx.x;
        float rs = 0.0f;
        if (GATEUP) {
            arow[r] = r < rows ? p_tok[pbase + r] : -1;
            if (r < rows) rs = xsum[arow[r]];
            if constexpr (H16) rscl[r] = r < rows ? xisc[arow[r]] : 0.0f;
        } else {
            arow[r] = r < rows ? pbase + r : -1;
            if (r < rows) {
                for (int q = 0; q < nt_gu; q++) rs += hsum[(size_t)(pbase + r) * nt_gu + q];
                rslot[r] = p_slot[pbase + r];
                rwt[r] = p_wt[pbase + r];
            }
        }
        rsum[r] = rs;
    }
    if (threadIdx.x < TBN) {
        const int n = threadIdx.x;
        if (GATEUP) {
            // wave column wn = n / 64 holds intermediate rows [(TBN / 2) nt + 32 wn, +32):
            // its n-blocks 0, 1 are their gate rows and n-blocks 2, 3 the same up rows
            const int wn = n >> 6, q = (n >> 4) & 3, o = nt * (TBN / 2) + wn * 32 + (q & 1) * 16 + (n & 15);
            bptr[n] = reinterpret_cast<const char *>((q < 2 ? Wb : Wb2) + (size_t)o * rowb);
            if (F4 && f4) sptr[n] = reinterpret_cast<const char *>((q < 2 ? Cb : Cb2) + (size_t)o * (Kdim / 16));
        } else {
            bptr[n] = reinterpret_cast<const char *>(Wb + (size_t)(nt * TBN + n) * rowb);
            if (F4 && f4) sptr[n] = reinterpret_cast<const char *>(Cb + (size_t)(nt * TBN + n) * (Kdim / 16));
        }
    }
    __syncthreads();
    // engine geometry: MWv m-blocks of 16 rows per wave, Eng::WMc waves along the rows
    constexpr int MWv = Eng::MWc;
    constexpr int RPW = 16 * MWv;                   // rows per wave
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, wm = wave / WN, wn = wave % WN;
    // the epilogue's column scales, loaded before the k-loop (their latency would
    // otherwise open the epilogue): gate/up columns o0 + 16 nb, down c0 + 16 nb
    const int o0 = nt * (TBN / 2) + wn * 32 + (lane & 15);
    const int c0 = nt * TBN + wn * 64 + (lane & 15);
    float sgv[2], suv[2], sbv[4];
    if constexpr (GATEUP) {
#pragma unroll
        for (int nb = 0; nb < 2; nb++) {
            sgv[nb] = f4 ? s2a : Sb[o0 + nb * 16];
            suv[nb] = f4 ? s2b : Sb2[o0 + nb * 16];
        }
    } else {
#pragma unroll
        for (int nb = 0; nb < 4; nb++) sbv[nb] = f4 ? s2a : Sb[c0 + nb * 16];
    }
    f32x4_t acc[MWv][4];
    if constexpr (F4) {
        if (grp < E) ExpertEngineF4::run(A, Kdim, arow, bptr, Kdim, lds, acc, sptr);
        else SharedEngineI8::run(A, Kdim, arow, bptr, Kdim, lds, acc);
    } else if constexpr (MODE == kDownI8) {
        DownEngineI8::run(A, Kdim, arow, bptr, Kdim, lds, acc);
    } else {
        ExpertEngine::run(A, Kdim, arow, bptr, Kdim, lds, acc);
    }
    // epilogues: the per-row values come from the LDS tables filled above (no
    // per-element global loads). The gate/up tile is staged in LDS (the
    // engine's buffers, free after its last barrier) so its rows leave as
    // 16-byte stores and the row sums come from the same pass, with no barrier
    // waiting on stores: epilogue 6.5 -> 4.8 us per tile, INT8 gate/up launch
    // 536 -> 514 us (wall-clock stamps per block)
    uint16_t *ep = reinterpret_cast<uint16_t *>(&lds);
    if constexpr (GATEUP) {
        // hidden tile [BM][HC] bf16, rows padded to HSR halfwords
        constexpr int HC = TBN / 2, HSR = HC + 8;
        static_assert(sizeof(lds) >= (size_t)BM * HSR * 2, "hidden tile fits the engine's LDS");
#pragma unroll
        for (int mb = 0; mb < MWv; mb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = wm * RPW + mb * 16 + (lane >> 4) * 4 + i;
                // offset-binary correction: bf16 rows 128 * sum(x), fp16 rows 1152 * sum(x16)
                const float cr = (f4 || r >= rows) ? 0.0f : (H16 ? 1152.0f : 128.0f) * rsum[r];
                const float ks = H16 ? rscl[r] : 1.0f;
#pragma unroll
                for (int nb = 0; nb < 2; nb++) {
                    const float gv = (acc[mb][nb][i] - cr) * ks * sgv[nb];
                    const float uv = (acc[mb][nb + 2][i] - cr) * ks * suv[nb];
                    ep[r * HSR + wn * 32 + nb * 16 + (lane & 15)] = r < rows ? f32_to_bf16(silu(gv) * uv) : (uint16_t)0;
                }
            }
        __syncthreads();
        // a row's HC / 8 16-byte chunks go to consecutive lanes (one contiguous
        // row segment per store), RPP rows per pass; the row's bf16 sum (the down
        // GEMM's offset correction): each lane's 8 values in order, then the
        // 16-lane reduction in its fixed order (deterministic)
        constexpr int CPR = HC / 8, RPP = Eng::NT / CPR;
        static_assert(CPR == 16 && BM % RPP == 0, "16 chunks per hidden row");
        const int cch = threadIdx.x % CPR, rr = threadIdx.x / CPR;
#pragma unroll
        for (int p = 0; p < BM / RPP; p++) {
            const int r = p * RPP + rr;
            float hs = 0.0f;
            if (r < rows) {
                const uint4 v = *reinterpret_cast<const uint4 *>(&ep[r * HSR + cch * 8]);
                *reinterpret_cast<uint4 *>(hid + (size_t)(pbase + r) * Nrows + nt * HC + cch * 8) = v;
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 4; j++) hs += bf16_lo(w[j]) + bf16_hi(w[j]);
            }
            hs = group_sum<CPR>(hs);
            if (cch == 0 && r < rows) hsum[(size_t)(pbase + r) * nt_gu + nt] = hs;
        }
    } else {
        // a wave's 64 columns of one row live in the 16 lanes of a row group (4
        // n-blocks each): that group of the partial row is stored as fp16 scaled
        // by 2^k, k putting its largest finite magnitude in [2^14, 2^15), and k
        // goes to partk (no fp16 overflow or underflow at any magnitude; inf and
        // NaN pass through)
        const int kg = (nt * TBN + wn * 64) >> 6, ngk = Hout >> 6;
        // pass 1: the values (in place) and each row group's largest magnitude;
        // the 16 row chains are independent, so their DPP steps interleave
        float mr[MWv][4];
#pragma unroll
        for (int mb = 0; mb < MWv; mb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = wm * RPW + mb * 16 + (lane >> 4) * 4 + i;
                const bool live = r < rows;
                const float cr = (f4 || !live) ? 0.0f : 128.0f * rsum[r], w = live ? rwt[r] : 0.0f;
#pragma unroll
                for (int nb = 0; nb < 4; nb++) acc[mb][nb][i] = w * ((acc[mb][nb][i] - cr) * sbv[nb]);
                mr[mb][i] = fmaxf(fmaxf(fabsf(acc[mb][0][i]), fabsf(acc[mb][1][i])),
                                  fmaxf(fabsf(acc[mb][2][i]), fabsf(acc[mb][3][i])));
            }
        bool bad = false;
#pragma unroll
        for (int mb = 0; mb < MWv; mb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                mr[mb][i] = row16_max(mr[mb][i]);
                bad = bad || !(mr[mb][i] <= 3.4028235e38f);
            }
        if (__builtin_amdgcn_ballot_w64(bad) != 0) {
            // rare (a non-finite value in the wave's tile): the finite maxima
#pragma unroll
            for (int mb = 0; mb < MWv; mb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float mf = 0.0f;
#pragma unroll
                    for (int nb = 0; nb < 4; nb++)
                        if ((__float_as_uint(acc[mb][nb][i]) & 0x7F800000u) != 0x7F800000u)
                            mf = fmaxf(mf, fabsf(acc[mb][nb][i]));
                    mr[mb][i] = row16_max(mf);
                }
        }
        // pass 2: scale by 2^k, round to fp16, store straight from the
        // accumulators (the tile staged in LDS for coalesced 16-byte row stores
        // measured 6-15 us slower per layer: the stores then wait for an LDS
        // round trip and a barrier, and the 2-byte stores already fill 32-byte
        // row segments)
#pragma unroll
        for (int mb = 0; mb < MWv; mb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = wm * RPW + mb * 16 + (lane >> 4) * 4 + i;
                const float m = mr[mb][i];
                const int k = m == 0.0f ? 0 : min(113, max(-113, 141 - (int)(__float_as_uint(m) >> 23)));
                if (r < rows) {
                    uint16_t *dst = part + (size_t)rslot[r] * Hout + c0;
#pragma unroll
                    for (int nb = 0; nb < 4; nb++)
                        dst[nb * 16] = __builtin_bit_cast(uint16_t, (_Float16)__builtin_ldexpf(acc[mb][nb][i], k));
                    if ((lane & 15) == 0) partk[(size_t)rslot[r] * ngk + kg] = (int8_t)k;
                }
            }
    }
}

// Four sums to y as bf16 (round to nearest even), or to y32 as fp32 when
// y32 != nullptr (y is then not written).
__device__ __forceinline__ void store4(uint16_t *y, float *y32, size_t i, float a0, float a1, float a2, float a3) {
    if (y32) {
        *reinterpret_cast<float4 *>(y32 + i) = make_float4(a0, a1, a2, a3);
    } else {
        *reinterpret_cast<uint2 *>(y + i) = make_uint2((uint32_t)f32_to_bf16(a0) | ((uint32_t)f32_to_bf16(a1) << 16),
                                                       (uint32_t)f32_to_bf16(a2) | ((uint32_t)f32_to_bf16(a3) << 16));
    }
}
// The prefill form: fp16 partials (the down GEMM's epilogue rounds each to
// nearest after scaling its 64-column group by 2^k, k in partk), summed in
// fp32 in slot order; four columns (8 bytes) per thread.
__global__ void __launch_bounds__(256)
k_pf_combine_h(const uint16_t *__restrict__ part, const int8_t *__restrict__ partk, int T, int S, int H,
               uint16_t *__restrict__ y, float *__restrict__ y32) {
    constexpr int kMaxS = 17;
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;       // index of 4 outputs
    if (i4 * 4 >= (size_t)T * H) return;
    const size_t t = i4 * 4 / H, c = i4 * 4 - t * H;
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 v[kMaxS];
#pragma unroll
    for (int k = 0; k < kMaxS; k++)
        if (k < S) v[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(part + (t * S + k) * H + c));
    int kk[kMaxS];
#pragma unroll
    for (int k = 0; k < kMaxS; k++)
        if (k < S) kk[k] = partk[(t * S + k) * (H >> 6) + (c >> 6)];
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < kMaxS; k++)
        if (k < S) {
            const uint32_t w[2] = {v[k].x, v[k].y};
            const float isc = __uint_as_float((uint32_t)(127 - kk[k]) << 23);
#pragma unroll
            for (int j = 0; j < 4; j++)
                a[j] += (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j >> 1] >> (16 * (j & 1)))) * isc;
        }
    store4(y, y32, t * H + c, a[0], a[1], a[2], a[3]);
}


// ---- launcher -------------------------------------------------------------------------
// The carve-up of one configuration (qfm_prefill_layout.h): gate/up tiles of
// GBN_F4 / GBN_I8 weight rows, down tiles of GBN_F4 (NVFP4) or
// DownEngineI8::BNt (INT8) output columns.
static PfLayout layout_of(int T, bool f4, bool has_sh) {
    const Cfg &c = g_cfg;
    return pf_layout(T, c.H, c.I, c.E, c.K, has_sh, f4 ? GBN_F4 : GBN_I8, f4 ? GBN_F4 : DownEngineI8::BNt, BM,
                     kRouterKS, kPairsPerBlk);
}

size_t prefill_ws_bytes(int T) {
    // the larger of the two arena formats, with the shared expert
    const size_t a = layout_of(T, false, true).total, b = layout_of(T, true, true).total;
    return a > b ? a : b;
}

void prefill_ws_view(void *ws, int T, float **lg, int **sel, float **wts, int **ctr) {
    const PfLayout Lw = layout_of(T, false, true);    // these regions do not depend on the format
    char *b = static_cast<char *>(ws);
    *lg = reinterpret_cast<float *>(b + Lw.off[kPfLg]);
    *sel = reinterpret_cast<int *>(b + Lw.off[kPfSel]);
    *wts = reinterpret_cast<float *>(b + Lw.off[kPfWts]);
    *ctr = reinterpret_cast<int *>(b + Lw.off[kPfCtr]);   // {candidate overflows, gate/up items, down items}
}

int launch_prefill(const qfm_layer *L, const uint16_t *x, int T, uint16_t *y, float *y32, void *ws, int gated,
                   hipStream_t s) {
    const Cfg &c = g_cfg;
    if (c.E != 512 || !(shape_2048() || shape_2560())) { set_error(-2, "prefill: unsupported shape"); return -2; }
    static_assert(kZeroRowElems >= 2560, "the zero A row must cover every K of the supported shapes");
    const int E = c.E, K = c.K, H = c.H, I = c.I;
    const Qf4ExpCache *a = L->arena;
    const bool f4 = L->fmt == QFM_FMT_NVFP4;
    if (!a) { set_error(-1, "prefill: no arena"); return -1; }
    if (!f4 && (!a->i8_gate || !a->i8_up || !a->i8_down || !a->i8s_gate || !a->i8s_up || !a->i8s_down)) {
        set_error(-1, "prefill: arena has no INT8 blobs"); return -1;
    }
    if (f4 && (!a->w_gate || !a->w_up || !a->w_down || !a->s_gate || !a->s_up || !a->s_down || !a->s2g_dev ||
               !a->s2u_dev || !a->s2d_dev)) {
        set_error(-1, "prefill: arena has no NVFP4 blobs"); return -1;
    }
    const bool has_sh = L->sh_gate.w != nullptr;
    const int S = K + (has_sh ? 1 : 0);      // partial slots per token: K routed (+ shared)
    const PfLayout Lw = layout_of(T, f4, has_sh);
    char *b = static_cast<char *>(ws);
    auto at = [&](PfRegion r) { return static_cast<void *>(b + Lw.off[r]); };
    float *lg = static_cast<float *>(at(kPfLg));
    float *xnorm = static_cast<float *>(at(kPfXnorm));
    float *wnorm = static_cast<float *>(at(kPfWnorm));
    uint16_t *wb16 = static_cast<uint16_t *>(at(kPfWb16));
    int *sel = static_cast<int *>(at(kPfSel));
    float *wts = static_cast<float *>(at(kPfWts));
    float *gam = static_cast<float *>(at(kPfGam));
    int *ctr = static_cast<int *>(at(kPfCtr));
    int *off = static_cast<int *>(at(kPfOff));
    const int nblk = Lw.nblk;
    int *blk = static_cast<int *>(at(kPfBlk));
    const size_t max_mt = Lw.max_mt;                 // bound on m-tiles, a multiple of 8
    const int nt_gu = Lw.nt_gu, nt_dn = Lw.nt_dn;
    int4 *items_gu = static_cast<int4 *>(at(kPfItemsGu));
    int4 *items_dn = static_cast<int4 *>(at(kPfItemsDn));
    int *p_tok = static_cast<int *>(at(kPfTok));
    int *p_slot = static_cast<int *>(at(kPfSlot));
    float *p_wt = static_cast<float *>(at(kPfPwt));
    uint16_t *hid = static_cast<uint16_t *>(at(kPfHid));
    uint16_t *part = static_cast<uint16_t *>(at(kPfPart));
    int8_t *partk = static_cast<int8_t *>(at(kPfPartK));
    float *xsum = static_cast<float *>(at(kPfXsum));
    float *hsum = static_cast<float *>(at(kPfHsum));
    uint4 *x16 = static_cast<uint4 *>(at(kPfX16));
    float *x16sum = static_cast<float *>(at(kPfX16sum));
    float *x16isc = static_cast<float *>(at(kPfX16isc));

    const float *g = (has_sh && gated) ? L->sh_gate_inp : nullptr;
    // zero the small counters with a fill kernel (no memset node in captured graphs)
    launch_fill_f32(reinterpret_cast<float *>(ctr), 8, 0.0f, s);
    hipLaunchKernelGGL(k_pf_router_prep, dim3((unsigned)(E + (T + 3) / 4)), dim3(256), 0, s, L->router, E, H, wnorm,
                       wb16, x, T, xnorm, xsum, f4 ? nullptr : x16, x16sum, x16isc);
    const int mt_router = ((T + BM - 1) / BM + 7) / 8 * 8;
    hipLaunchKernelGGL(k_pf_router_mfma, dim3(mt_router * (E / BN), kRouterKS), dim3(256), 0, s, x, T, H, wb16, E, lg);
    if (H == 2048)
        hipLaunchKernelGGL((k_pf_select<8, 8>), dim3((T + 3) / 4), dim3(256), 0, s, x, T, L->router, L->router_bias,
                           g, lg, xnorm, wnorm, K, c.renorm, sel, wts, gam, ctr);
    else
        hipLaunchKernelGGL((k_pf_select<10, 8>), dim3((T + 3) / 4), dim3(256), 0, s, x, T, L->router, L->router_bias,
                           g, lg, xnorm, wnorm, K, c.renorm, sel, wts, gam, ctr);
    hipLaunchKernelGGL(k_pf_count, dim3(nblk), dim3(256), 0, s, sel, T * K, E, blk);
    hipLaunchKernelGGL(k_pf_plan, dim3(1), dim3(1024), 0, s, blk, nblk, E, has_sh ? 1 : 0, T, nt_gu, nt_dn, off,
                       items_gu, items_dn, ctr + 1, (int)(max_mt * nt_gu), (int)(max_mt * nt_dn));
    hipLaunchKernelGGL(k_pf_scatter, dim3((unsigned)(nblk + (has_sh ? (T + 255) / 256 : 0))), dim3(256), 0, s, sel,
                       wts, g ? gam : nullptr, T, K, E, has_sh ? 1 : 0, off, blk, p_tok, p_slot, p_wt);
    GroupW gg, gu, gd;
    if (f4) {
        gg = GroupW{reinterpret_cast<const int8_t *>(a->w_gate), nullptr, L->sh_gate.w, L->sh_gate.s, a->s_gate, a->s2g_dev};
        gu = GroupW{reinterpret_cast<const int8_t *>(a->w_up), nullptr, L->sh_up.w, L->sh_up.s, a->s_up, a->s2u_dev};
        gd = GroupW{reinterpret_cast<const int8_t *>(a->w_down), nullptr, L->sh_down.w, L->sh_down.s, a->s_down, a->s2d_dev};
    } else {
        gg = GroupW{a->i8_gate, a->i8s_gate, L->sh_gate.w, L->sh_gate.s, nullptr, nullptr};
        gu = GroupW{a->i8_up, a->i8s_up, L->sh_up.w, L->sh_up.s, nullptr, nullptr};
        gd = GroupW{a->i8_down, a->i8s_down, L->sh_down.w, L->sh_down.s, nullptr, nullptr};
    }
    const dim3 g_gu((unsigned)(max_mt * nt_gu)), g_dn((unsigned)(max_mt * nt_dn)),
        nth(f4 ? ExpertEngineF4::NT : ExpertEngine::NT), nth_dn(f4 ? ExpertEngineF4::NT : DownEngineI8::NT);
    if (f4) {
        hipLaunchKernelGGL((k_pf_gemm<true, kRoutedF4>), g_gu, nth, 0, s, items_gu, ctr + 1, 0, p_tok, p_slot,
                           p_wt, x, H, I, gg, gu, E, hid, part, partk, H, nt_gu, xsum, hsum, nt_gu, nullptr);
        hipLaunchKernelGGL((k_pf_gemm<false, kRoutedF4>), g_dn, nth, 0, s, items_dn, ctr + 1, 1, p_tok, p_slot,
                           p_wt, hid, I, H, gd, gd, E, hid, part, partk, H, nt_dn, xsum, hsum, nt_gu, nullptr);
    } else {
        hipLaunchKernelGGL((k_pf_gemm<true, kAllI8>), g_gu, nth, 0, s, items_gu, ctr + 1, 0, p_tok, p_slot, p_wt,
                           reinterpret_cast<const uint16_t *>(x16), H, I, gg, gu, E, hid, part, partk, H, nt_gu, x16sum, hsum,
                           nt_gu, x16isc);
        hipLaunchKernelGGL((k_pf_gemm<false, kDownI8>), g_dn, nth_dn, 0, s, items_dn, ctr + 1, 1, p_tok, p_slot, p_wt,
                           hid, I, H, gd, gd, E, hid, part, partk, H, nt_dn, xsum, hsum, nt_gu, nullptr);
    }
    hipLaunchKernelGGL(k_pf_combine_h, dim3((unsigned)(((size_t)T * H / 4 + 255) / 256)), dim3(256), 0, s, part, partk,
                       T, S, H, y, y32);
    return check_launch("prefill");
}

}  // namespace qfm
