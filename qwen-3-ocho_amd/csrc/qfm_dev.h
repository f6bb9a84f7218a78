// qfm_dev.h -- device helpers shared by the MoE kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qfm {

constexpr int WAVE = 64;

// Lanes per weight row for a row of cpr 16-byte chunks: the largest of
// 32/16/8/4 that divides it (every lane then owns cpr/lpr chunks).
constexpr int lpr_of(int cpr) { return cpr % 32 == 0 ? 32 : cpr % 16 == 0 ? 16 : cpr % 8 == 0 ? 8 : 4; }

// ---- bf16 ----------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
// round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// ---- int8 x fp32 dot of one 16-byte chunk ---------------------------------
// Codes are consumed in offset-binary form: u = q ^ 0x80 = q + 128 is an
// unsigned byte, widened exactly by v_cvt_f32_ubyteN (one op per code); the
// caller seeds the accumulator with -128 * sum(x) over the same elements.
// (A sign-extending extract followed by an int->float conversion is not
// used: hipcc 7.2 folds that pair into v_cvt_f32_u32_sdwa with a sext
// source, an unsigned conversion that turns negative codes into ~4e9.)
__device__ __forceinline__ float dot16_u8(const uint4 w, const float *x, float acc) {
    const uint32_t d[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u, w.w ^ 0x80808080u};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        acc = fmaf((float)(d[q] & 0xFFu), x[q * 4 + 0], acc);
        acc = fmaf((float)((d[q] >> 8) & 0xFFu), x[q * 4 + 1], acc);
        acc = fmaf((float)((d[q] >> 16) & 0xFFu), x[q * 4 + 2], acc);
        acc = fmaf((float)(d[q] >> 24), x[q * 4 + 3], acc);
    }
    return acc;
}

// ---- int8 x fp16 dot of one 16-byte chunk (v_dot2_f32_f16) ------------------
// The offset-binary code u = q ^ 0x80 = q + 128 placed in the low byte of the
// fp16 pattern 0x6400 (1024.0) reads 1024 + u = q + 1152 exactly (fp16 has
// unit spacing on [1024, 2048)), so one v_perm_b32 widens two codes into an
// fp16 pair and one v_dot2_f32_f16 multiplies it with two activations, with
// exact products (11 x 11 significant bits) and fp32 accumulation. The
// activations are fp16 pairs in memory order (xa: values 0..7, xb: 8..15);
// the caller seeds acc with -1152 * (sum of the 16 activations).
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f16x2_t as_h2(uint32_t v) { return __builtin_bit_cast(f16x2_t, v); }
__device__ __forceinline__ float dot16_i8h(const uint4 w, const uint4 xa, const uint4 xb, float acc) {
    const uint32_t d[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u, w.w ^ 0x80808080u};
    const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
    for (int q = 0; q < 4; q++) {
        // perm selector bytes 0..3 pick bytes of the second operand, 4 the first's (0x64)
        acc = __builtin_amdgcn_fdot2(as_h2(__builtin_amdgcn_perm(0x64646464u, d[q], 0x04010400u)), as_h2(xv[2 * q]),
                                     acc, false);
        acc = __builtin_amdgcn_fdot2(as_h2(__builtin_amdgcn_perm(0x64646464u, d[q], 0x04030402u)),
                                     as_h2(xv[2 * q + 1]), acc, false);
    }
    return acc;
}
constexpr float kI8hOffset = 1152.0f;

// 16 fp32 activations -> 16 fp16 scaled by 2^k, k chosen so the largest
// magnitude lands in [2^14, 2^15) (no overflow; values with at most 11
// significant bits, bf16 ones among them, convert exactly unless they are
// 2^-28 below the chunk's largest). Returns (seed, 2^-k): seed = -1152 * the
// sum of the scaled values, the dot16_i8h seed; 2^-k undoes the scaling.
__device__ __forceinline__ float2 chunk16_to_f16(const float *v, uint4 &ha, uint4 &hb) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
    const int e = (int)(__float_as_uint(amax) >> 23);
    const int k = amax == 0.0f ? 0 : min(113, max(-113, 141 - e));
    const float sc = __uint_as_float((uint32_t)(127 + k) << 23), isc = __uint_as_float((uint32_t)(127 - k) << 23);
    uint32_t h[8];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float a = v[2 * i] * sc, b = v[2 * i + 1] * sc;
        const f16x2_t hp = {(_Float16)a, (_Float16)b};   // round to nearest even
        h[i] = __builtin_bit_cast(uint32_t, hp);
        sum += a + b;
    }
    ha = make_uint4(h[0], h[1], h[2], h[3]);
    hb = make_uint4(h[4], h[5], h[6], h[7]);
    return make_float2(-kI8hOffset * sum, isc);
}

// ---- hidden rows staged in LDS as scaled fp16 chunks ---------------------------
// Rows h[0..n) (n <= RMAX) of I fp32 values (contiguous), one 16-value chunk
// per thread and pass of an NT-thread block: s_h16 two 16-byte words per
// chunk, s_hci its (seed, 2^-k) (chunk16_to_f16). In two halves, so the loads
// can be issued ahead of others whose data arrives later (loads retire in
// issue order): load() into registers, then store() converts and writes LDS.
template <int I, int RMAX, int NT = 256>
struct H16Stage {
    static constexpr int CPT = (RMAX * (I / 16) + NT - 1) / NT;   // chunks per thread
    float v[CPT][16];
    __device__ __forceinline__ void load(const float *__restrict__ h, int n) {
#pragma unroll
        for (int q = 0; q < CPT; q++) {
            const int c = (int)threadIdx.x + q * NT;
            if (c < n * (I / 16)) {
                const float4 *hp = reinterpret_cast<const float4 *>(h) + 4 * c;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float4 f = hp[j];
                    v[q][4 * j] = f.x; v[q][4 * j + 1] = f.y; v[q][4 * j + 2] = f.z; v[q][4 * j + 3] = f.w;
                }
            }
        }
    }
    // rows h + pair_of_lane(ids, j) * I for j < n (ids: a pair set, whose j-th
    // id a lane gets with a shuffle, or a pair descriptor's packed id bytes)
    template <class IDS>
    __device__ __forceinline__ void load_rows(const float *__restrict__ h, const IDS &ids, int n) {
#pragma unroll
        for (int q = 0; q < CPT; q++) {
            const int c = (int)threadIdx.x + q * NT;
            const int j = c / (I / 16), o = c - j * (I / 16);
            const int r = pair_of_lane(ids, j < RMAX ? j : 0);     // (every lane calls it: a shuffle needs all)
            if (c < n * (I / 16)) {
                const float4 *hp = reinterpret_cast<const float4 *>(h + (size_t)r * I) + 4 * o;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float4 f = hp[k];
                    v[q][4 * k] = f.x; v[q][4 * k + 1] = f.y; v[q][4 * k + 2] = f.z; v[q][4 * k + 3] = f.w;
                }
            }
        }
    }
    __device__ __forceinline__ void store(int n, uint4 *s_h16, float2 *s_hci) {
#pragma unroll
        for (int q = 0; q < CPT; q++) {
            const int c = (int)threadIdx.x + q * NT;
            if (c < n * (I / 16)) {
                uint4 ha, hb;
                s_hci[c] = chunk16_to_f16(v[q], ha, hb);
                s_h16[2 * c] = ha;
                s_h16[2 * c + 1] = hb;
            }
        }
    }
};
// One wave converts a bf16 row of H values to fp16 scaled by 2^k (largest
// magnitude in [2^14, 2^15): exact for bf16 values, no overflow); writes the
// row (H / 8 16-byte words, same value order) and info = (sum of the scaled
// values, 2^-k). (group_max / group_sum are defined further down.)
template <int G> __device__ float group_sum(float v);
template <int G> __device__ float group_max(float v);
template <int H>
__device__ __forceinline__ void wave_row_to_f16(const uint16_t *__restrict__ x, uint4 *__restrict__ xo,
                                                float2 *__restrict__ info, int lane) {
    constexpr int NC = H / 512;                     // 16-byte words per lane
    uint4 v[NC];
#pragma unroll
    for (int q = 0; q < NC; q++) v[q] = reinterpret_cast<const uint4 *>(x)[q * 64 + lane];
    float amax = 0.0f;
#pragma unroll
    for (int q = 0; q < NC; q++) {
        const uint32_t d[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
        for (int u = 0; u < 4; u++) amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(d[u])), fabsf(bf16_hi(d[u]))));
    }
    amax = group_max<64>(amax);
    const int e = (int)(__float_as_uint(amax) >> 23);
    const int k = amax == 0.0f ? 0 : min(113, max(-113, 141 - e));
    const float sc = __uint_as_float((uint32_t)(127 + k) << 23);
    float hs = 0.0f;
#pragma unroll
    for (int q = 0; q < NC; q++) {
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
    hs = group_sum<64>(hs);
    if (lane == 0) *info = make_float2(hs, __uint_as_float((uint32_t)(127 - k) << 23));
}

// Kernel arguments are read through the scalar cache on first use, and the
// compiler places each argument's load below the first branch that needs it:
// a kernel whose arguments span several 64-byte lines can then take one
// dependent scalar-cache miss per line before its first memory load.
// args_now(...) makes every value given live in SGPRs at that point, so all
// the lines are requested together (one miss).
template <typename T>
__device__ __forceinline__ void arg_now(const T &v) { asm volatile("" ::"s"(v)); }
template <typename... T>
__device__ __forceinline__ void args_now(const T &...v) { (arg_now(v), ...); }

// 64-bit loads and stores at agent scope (coherent across the XCDs' L2s
// without a fence: written through, read from the memory side)
__device__ __forceinline__ unsigned long long ld_agent_u64(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u64(unsigned long long *p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt16(const void *p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- cross-lane reductions -------------------------------------------------
// Sum over aligned groups of G lanes (G a power of two <= 64); every lane of
// the group ends with the group total. Within 16-lane rows the steps are DPP
// adds (xor 1, xor 2, half-row mirror, row mirror: no LDS round trip); the
// 32-lane step is one ds_swizzle (lane ^ 16), the 64-lane one a bpermute.
// (hipcc 7.2 drops the second result of v_permlane16_swap / 32_swap, so the
// gfx950 row swaps are not used.)
template <int G>
__device__ float group_sum(float v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group of 2^k lanes");
    if constexpr (G >= 2)   // quad_perm [1,0,3,2]
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    if constexpr (G >= 4)   // quad_perm [2,3,0,1]
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    if constexpr (G >= 8)   // row_half_mirror
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    if constexpr (G >= 16)  // row_mirror
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    if constexpr (G >= 32)  // ds_swizzle bit-mask mode, lane ^ 16 within 32 lanes: and 0x1F, or 0, xor 0x10
        v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    if constexpr (G >= 64) v += __shfl_xor(v, 32, WAVE);
    return v;
}

// The canonical router reduction of 64 lane partials: p[l] + p[l ^ m] for
// m = 1, 2, 4, 8, 16, 32, each step one fp32 rounding (the oracle's
// canon_dot). After the xor-1 and xor-2 steps every quad holds one value, so
// the half-row mirror partner (l ^ 7) carries the value of l ^ 4; after the
// xor-4 step every 8-lane group does, so the row mirror (l ^ 15) carries that
// of l ^ 8: four DPP adds reproduce the first four steps exactly, a ds_swizzle
// (l ^ 16) and one bpermute (l ^ 32) the last two. Every lane ends with the sum.
__device__ __forceinline__ float canon_butterfly(float a) {
    a = __fadd_rn(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), 0xB1, 0xF, 0xF, false)));
    a = __fadd_rn(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), 0x4E, 0xF, 0xF, false)));
    a = __fadd_rn(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), 0x141, 0xF, 0xF, false)));
    a = __fadd_rn(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), 0x140, 0xF, 0xF, false)));
    a = __fadd_rn(a, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, a), 0x401F)));
    return __fadd_rn(a, __shfl_xor(a, 32, WAVE));
}

// max over the 16 lanes of a DPP row, all in VALU DPP moves (no LDS round
// trip): quad permutes xor 1 and xor 2, then the half-row and row mirrors
// (canon_butterfly's first four steps)
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
    return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
}

// v from lane l ^ M (M = 1, 2: DPP quad permutes; 4, 8, 16: ds_swizzle in
// bitmask mode; 32: bpermute)
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane xor of a power of two");
    if constexpr (M == 1) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    else if constexpr (M == 2) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    else if constexpr (M < 32) return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (M << 10) | 0x1F));
    else return __shfl_xor(v, 32, WAVE);
}

// The canonical reduction (canon_butterfly's addition tree: level m adds the
// partial sums of lanes l and l ^ m) of R rows at once, R = 2, 4 or 8,
// computed reduce-scatter style: at the levels m < R, lane l keeps the rows
// whose bit matches bit m of l and trades the others with lane l ^ m (which
// holds the same rows), so every addition still combines the partial sums of
// lanes l and l ^ m of one row; the levels m >= R are a plain butterfly.
// R - 1 + 6 - log2(R) cross-lane steps instead of 6 R. Lane l returns the
// sum of row l & (R - 1).
template <int R, int M = 1>
__device__ __forceinline__ float canon_scatter_level(const float (&v)[R], int lane) {
    if constexpr (R == 1) {
        float s = v[0];
        if constexpr (M <= 1) s = __fadd_rn(s, lane_xor<1>(s));
        if constexpr (M <= 2) s = __fadd_rn(s, lane_xor<2>(s));
        if constexpr (M <= 4) s = __fadd_rn(s, lane_xor<4>(s));
        if constexpr (M <= 8) s = __fadd_rn(s, lane_xor<8>(s));
        if constexpr (M <= 16) s = __fadd_rn(s, lane_xor<16>(s));
        return __fadd_rn(s, lane_xor<32>(s));
    } else {
        const bool hi = (lane & M) != 0;
        float n[R / 2];
#pragma unroll
        for (int j = 0; j < R / 2; j++) {
            const float keep = hi ? v[2 * j + 1] : v[2 * j];
            const float send = hi ? v[2 * j] : v[2 * j + 1];
            n[j] = __fadd_rn(keep, lane_xor<M>(send));
        }
        return canon_scatter_level<R / 2, 2 * M>(n, lane);
    }
}
template <int R>
__device__ __forceinline__ float canon_reduce_rows(const float (&a)[R], int lane) {
    static_assert(R == 2 || R == 4 || R == 8, "2, 4 or 8 rows");
    return canon_scatter_level<R, 1>(a, lane);
}

// Max over aligned groups of G lanes (same steps as group_sum).
template <int G>
__device__ float group_max(float v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group of 2^k lanes");
    if constexpr (G >= 2)
        v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    if constexpr (G >= 4)
        v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    if constexpr (G >= 8)
        v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
    if constexpr (G >= 16)
        v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
    if constexpr (G >= 32)
        v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F)));
    if constexpr (G >= 64) v = fmaxf(v, __shfl_xor(v, 32, WAVE));
    return v;
}

// ---- wave-wide reductions from the ROCm device library (ockl) -------------
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_max_u64(unsigned long long);
extern "C" __device__ __attribute__((const)) float __ockl_wfred_add_f32(float);

// Order-preserving 64-bit selection key of a logit: descending value, ties to
// the lower index. -0.0 is folded onto +0.0 (they compare equal as floats).
__device__ __forceinline__ unsigned long long topk_key(float v, int e) {
    const uint32_t b = __float_as_uint(v + 0.0f);
    const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)e);
}
__device__ __forceinline__ int topk_key_index(unsigned long long key) {
    return (int)(0xFFFFFFFFu - (uint32_t)key);
}
__device__ __forceinline__ float topk_key_value(unsigned long long key) {
    const uint32_t k = (uint32_t)(key >> 32);
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// ---- wave top-K --------------------------------------------------------------
// One wave selects the top-K (K <= 16) of E = 64*EPL logits lr[0..E) (EPL <= 16):
// descending value, ties to the lower index (64-bit keys, all distinct).
// Wave-uniform control flow; lds: kTopkLds u64 of wave-private LDS, 16-byte aligned.
//
// Method (latency-bound: one wave, so few dependent steps and independent
// accumulators). 31-bit keys k31 = (value prefix << IB) | (E - 1 - e), IB =
// index bits (9 for E = 512, 22-bit prefix of the sortable value bits), are distinct; T31 = the K-th largest of the 64 lane maxima of k31 (rank by
// broadcast compares, sign of the 31-bit difference), P = its value prefix.
// Every element of the true top-K has a prefix >= P (K distinct lane maxima
// have prefix >= P and the K-th largest element is >= the least of them), so
// C = {prefix >= P} contains the top-K; typically |C| ~ K. If |C| > 64 (ties
// in the prefix) the exact 64-bit form of the same bound is used instead:
// T = K-th largest 64-bit lane maximum, C = {key >= T}, |C| <= K*EPL. C is
// compacted to LDS with ballots and mbcnt and each candidate's exact rank
// within C is its rank among all E.
constexpr int kTopkLds = 16 + 256 + 64 + 64;   // results, candidates, junk slots, lane maxima
// (LOAD false: v[] already holds the logits, v[i] = logit i * 64 + lane; lr unused)
template <int EPL, bool LOAD = true>
__device__ __forceinline__ int topk_candidates(const float *lr, int K, int lane, unsigned long long *lds,
                                               float (&v)[EPL]) {
    static_assert(EPL >= 1 && EPL <= 16, "E = 64 * EPL, EPL <= 16");
    constexpr int E = 64 * EPL;
    constexpr int IB = E <= 64 ? 6 : E <= 128 ? 7 : E <= 256 ? 8 : E <= 512 ? 9 : 10;   // index bits
    constexpr int PB = 31 - IB;                                                        // value-prefix bits
    unsigned long long key[EPL];
    uint32_t k31[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        if constexpr (LOAD) v[i] = lr[i * 64 + lane];
        key[i] = topk_key(v[i], i * 64 + lane);
        k31[i] = ((uint32_t)(key[i] >> (64 - PB)) << IB) | (uint32_t)(E - 1 - (i * 64 + lane));
    }
    unsigned long long *cand = lds + 16, *lm = lds + 16 + 256 + 64;
    uint32_t *lm32 = reinterpret_cast<uint32_t *>(lm);
    uint32_t mx = k31[0];
#pragma unroll
    for (int i = 1; i < EPL; i++) mx = max(mx, k31[i]);
    lm32[lane] = mx;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    uint32_t r4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int h = 0; h < 2; h++) {
        uint4 p[8];
#pragma unroll
        for (int q = 0; q < 8; q++) p[q] = reinterpret_cast<const uint4 *>(lm32)[h * 8 + q];
#pragma unroll
        for (int q = 0; q < 8; q++) {      // keys < 2^31: the difference's sign bit is (other > mine)
            r4[0] += (mx - p[q].x) >> 31; r4[1] += (mx - p[q].y) >> 31;
            r4[2] += (mx - p[q].z) >> 31; r4[3] += (mx - p[q].w) >> 31;
        }
    }
    const uint32_t rank = r4[0] + r4[1] + r4[2] + r4[3];
    const uint32_t T31 = (uint32_t)__builtin_amdgcn_readlane((int)mx, __builtin_ctzll(__ballot(rank == (uint32_t)(K - 1))));
    const uint32_t P = T31 & ~((1u << IB) - 1u);
    unsigned long long b[EPL];
    int base[EPL], tot = 0;
#pragma unroll
    for (int i = 0; i < EPL; i++) b[i] = __ballot(k31[i] >= P);
#pragma unroll
    for (int i = 0; i < EPL; i++) { base[i] = tot; tot += __popcll(b[i]); }
    if (tot > 64) {
        // exact bound: 64-bit lane maxima (wave-uniform branch)
        unsigned long long m64 = key[0];
#pragma unroll
        for (int i = 1; i < EPL; i++) m64 = key[i] > m64 ? key[i] : m64;
        lm[lane] = m64;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        int ra[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 64; j += 8) {
            ulonglong2 p[4];
#pragma unroll
            for (int q = 0; q < 4; q++) p[q] = *reinterpret_cast<const ulonglong2 *>(lm + j + 2 * q);
#pragma unroll
            for (int q = 0; q < 4; q++) ra[q] += (p[q].x > m64 ? 1 : 0) + (p[q].y > m64 ? 1 : 0);
        }
        const int r64 = ra[0] + ra[1] + ra[2] + ra[3];
        const int tl = __builtin_ctzll(__ballot(r64 == K - 1));
        const uint32_t t_hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(m64 >> 32), tl);
        const uint32_t t_lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)m64, tl);
        const unsigned long long T = ((unsigned long long)t_hi << 32) | t_lo;
        tot = 0;
#pragma unroll
        for (int i = 0; i < EPL; i++) b[i] = __ballot(key[i] >= T);
#pragma unroll
        for (int i = 0; i < EPL; i++) { base[i] = tot; tot += __popcll(b[i]); }
    }
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const bool in = (b[i] >> lane) & 1ull;
        const int pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(b[i] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b[i], base[i]));
        cand[in ? pos : 256 + lane] = key[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    return tot;
}
// rank of candidate key c among the first n candidates (16 per pass, 4 accumulators)
__device__ __forceinline__ int topk_cand_rank(const unsigned long long *cand, int n, unsigned long long c) {
    int ra[4] = {0, 0, 0, 0};
    for (int i0 = 0; i0 < n; i0 += 16) {
        ulonglong2 p[8];
#pragma unroll
        for (int q = 0; q < 8; q++) p[q] = *reinterpret_cast<const ulonglong2 *>(cand + i0 + 2 * q);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            ra[q & 3] += (i0 + 2 * q < n && p[q].x > c) ? 1 : 0;
            ra[(q + 2) & 3] += (i0 + 2 * q + 1 < n && p[q].y > c) ? 1 : 0;
        }
    }
    return ra[0] + ra[1] + ra[2] + ra[3];
}
// Lane k < K receives the k-th expert id and its weight exp(l_k - l_max) /
// denom, denom = sum over the K selected (renorm) or over all E (plain softmax).
template <int EPL, bool LOAD>
__device__ __forceinline__ void wave_topk_v(float (&v)[EPL], const float *lr, int K, int renorm, int lane,
                                            unsigned long long *lds, int &my_i, float &my_w) {
    const int n = topk_candidates<EPL, LOAD>(lr, K, lane, lds, v);
    const unsigned long long *cand = lds + 16;
    for (int j = lane; j < n; j += 64) {
        const unsigned long long cj = cand[j];
        const int r = topk_cand_rank(cand, n, cj);
        if (r < K) lds[r] = cj;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const unsigned long long mine = lane < K ? lds[lane] : 0ull;
    const unsigned long long first = lds[0];
    const float mxv = topk_key_value(first);
    const float ek = lane < K ? __expf(topk_key_value(mine) - mxv) : 0.0f;
    float denom;
    if (renorm) {
        denom = __ockl_wfred_add_f32(ek);
    } else {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; i++) t += __expf(v[i] - mxv);
        denom = __ockl_wfred_add_f32(t);
    }
    my_i = lane < K ? topk_key_index(mine) : -1;
    my_w = ek / denom;
}
template <int EPL>
__device__ __forceinline__ void wave_topk(const float *lr, int K, int renorm, int lane,
                                          unsigned long long *lds, int &my_i, float &my_w) {
    float v[EPL];
    wave_topk_v<EPL, true>(v, lr, K, renorm, lane, lds, my_i, my_w);
}
// The same from logits held in registers (v[i] = logit i * 64 + lane)
template <int EPL>
__device__ __forceinline__ void wave_topk_regs(float (&v)[EPL], int K, int renorm, int lane,
                                               unsigned long long *lds, int &my_i, float &my_w) {
    wave_topk_v<EPL, false>(v, nullptr, K, renorm, lane, lds, my_i, my_w);
}
// The expert id of rank `job` (< K) only (wave-uniform result): same candidate
// set and ranks as wave_topk, no permutation through LDS and no softmax.
template <int EPL>
__device__ __forceinline__ int wave_topk_one(const float *lr, int K, int job, int lane, unsigned long long *lds) {
    float v[EPL];
    const int n = topk_candidates<EPL>(lr, K, lane, lds, v);
    const unsigned long long *cand = lds + 16;
    int found = -1;
    for (int j = lane; j < n; j += 64) {
        const unsigned long long cj = cand[j];
        if (topk_cand_rank(cand, n, cj) == job) found = topk_key_index(cj);
    }
    return __builtin_amdgcn_readlane(found, __builtin_ctzll(__ballot(found >= 0)));
}

// x slice of one 32-lane group: lane l holds x[st*512 + 16l + i], i < 16.
template <int H>
__device__ __forceinline__ void load_x_slice_bf16(const uint16_t *x, int l, float (&xs)[H / 512][16]) {
#pragma unroll
    for (int st = 0; st < H / 512; st++) {
        const int k0 = st * 512 + l * 16;
        const uint4 a = *reinterpret_cast<const uint4 *>(x + k0);
        const uint4 b = *reinterpret_cast<const uint4 *>(x + k0 + 8);
        const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int q = 0; q < 8; q++) { xs[st][2 * q] = bf16_lo(d[q]); xs[st][2 * q + 1] = bf16_hi(d[q]); }
    }
}
template <int H>
__device__ __forceinline__ void load_x_slice_f32(const float *x, int l, float (&xs)[H / 512][16]) {
#pragma unroll
    for (int st = 0; st < H / 512; st++) {
        const int k0 = st * 512 + l * 16;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = *reinterpret_cast<const float4 *>(x + k0 + 4 * q);
            xs[st][4 * q] = f.x; xs[st][4 * q + 1] = f.y; xs[st][4 * q + 2] = f.z; xs[st][4 * q + 3] = f.w;
        }
    }
}

// ---- silu / sigmoid ----------------------------------------------------------
// (v_rcp_f32, 1 ulp, in place of the IEEE division sequence)
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }
__device__ __forceinline__ float sigmoid(float g) { return __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// ---- NVFP4 number formats -----------------------------------------------------
// E2M1 code -> float: +-{0, .5, 1, 1.5, 2, 3, 4, 6}; built from the bit
// fields (exponent e = (n >> 1) & 3, mantissa m = n & 1, sign bit 3).
__device__ __forceinline__ float e2m1(uint32_t nib) {
    const uint32_t e = (nib >> 1) & 3u, m = nib & 1u;
    const uint32_t mag = e ? (((e + 126u) << 23) | (m << 22)) : (m ? 0x3F000000u : 0u);
    return __uint_as_float(mag | ((nib & 8u) << 28));
}
// E4M3 block scale -> float: e == 0 -> m * 2^-9; else (1 + m/8) * 2^(e-7);
// 0x7F -> +inf (the checkpoint never stores it).
__device__ __forceinline__ float e4m3(uint32_t b) {
    const uint32_t e = (b >> 3) & 15u, m = b & 7u;
    const float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0x1p-9f;
    return ((b & 0x7Fu) == 0x7Fu) ? __uint_as_float(0x7F800000u) : v;
}

// NVFP4 chunk: 32 e2m1 values (adjacent pairs: byte i = value 2i low nibble,
// 2i+1 high nibble) with two e4m3 block scales (values 0..15 and 16..31).
// Codes are converted by the gfx950 v_cvt_scalef32_pk_f32_fp4 instruction
// with a unit scale (exact e2m1 values); each 16-value group is scaled once.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float f4_group16(uint32_t lo, uint32_t hi, const float *x) {
    float a = 0.0f;
    const uint32_t w[2] = {lo, hi};
#pragma unroll
    for (int d = 0; d < 2; d++) {
        f32x2_t v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 0);
        f32x2_t v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 1);
        f32x2_t v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 2);
        f32x2_t v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 3);
        a = fmaf(v0.x, x[d * 8 + 0], a); a = fmaf(v0.y, x[d * 8 + 1], a);
        a = fmaf(v1.x, x[d * 8 + 2], a); a = fmaf(v1.y, x[d * 8 + 3], a);
        a = fmaf(v2.x, x[d * 8 + 4], a); a = fmaf(v2.y, x[d * 8 + 5], a);
        a = fmaf(v3.x, x[d * 8 + 6], a); a = fmaf(v3.y, x[d * 8 + 7], a);
    }
    return a;
}
// ue4m3 block scale byte exactly as the reference decodes it
// (ocho/amd_server/qf_nvfp4_wave64.hip:68-73): e = b >> 3 (five bits: bytes
// >= 0x80 are large unsigned scales), m = b & 7; e == 0 -> m * 2^-9, else
// (1 + m/8) * 2^(e-7); 0x7F -> +inf. Not the OCP E4M3 hardware convert, which
// reads bit 7 as a sign and 0x7F as NaN.
__device__ __forceinline__ float e4m3_scale(uint32_t b) {
    b &= 0xFFu;
    const uint32_t e = b >> 3, m = b & 7u;
    const uint32_t bits = b == 0x7Fu ? 0x7F800000u : ((e + 120u) << 23) | (m << 20);
    return e ? __uint_as_float(bits) : (float)m * 0x1p-9f;
}
// Both e4m3 block scales of a 16-bit pair (byte 0 low). The gfx950 OCP E4M3
// convert (v_cvt_pk_f32_fp8, one op for the pair) gives the same fp32 bits as
// e4m3_scale for bytes 0x00..0x7E (checked on the box over all 256 bytes);
// bytes >= 0x7F differ (0x7F: +inf here, NaN there; bit 7 set: large
// unsigned scales here, negative values there) and take e4m3_scale.
// e4m3_pairs decodes NS pairs with the convert when no lane of the wave holds
// such a byte (a wave-uniform choice), otherwise with e4m3_scale.
__device__ __forceinline__ bool e4m3_pair_hw_ok(uint32_t s2b) {
    return ((s2b | (s2b + 0x0101u)) & 0x8080u) == 0;   // both bytes < 0x7F (a carry out of byte 0 means byte 0 >= 0xFF)
}
template <int NS>
__device__ __forceinline__ void e4m3_pairs(const uint32_t (&s2b)[NS], f32x2_t (&out)[NS]) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < NS; i++) ok = ok && e4m3_pair_hw_ok(s2b[i]);
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) {
#pragma unroll
        for (int i = 0; i < NS; i++) out[i] = __builtin_amdgcn_cvt_pk_f32_fp8(s2b[i], false);
    } else {
#pragma unroll
        for (int i = 0; i < NS; i++) out[i] = f32x2_t{e4m3_scale(s2b[i] & 0xFFu), e4m3_scale((s2b[i] >> 8) & 0xFFu)};
    }
}
__device__ __forceinline__ float f4_chunk(uint4 w, uint32_t s2b, const float *x) {
    const float g0 = f4_group16(w.x, w.y, x);
    const float g1 = f4_group16(w.z, w.w, x + 16);
    return fmaf(e4m3_scale(s2b & 0xFFu), g0, e4m3_scale((s2b >> 8) & 0xFFu) * g1);
}

// NVFP4 chunk against bf16 activations: 32 e2m1 codes (w) with two e4m3 block
// scales (s2b) dotted with 32 bf16 values held as 16 packed pairs (xw[i] =
// x[2i] | x[2i+1] << 16, the memory order). gfx950 converts each code pair to
// a bf16 pair (v_cvt_scalef32_pk_bf16_fp4, unit scale: exact) and
// v_dot2_f32_bf16 multiplies a pair with fp32 accumulation (bf16 products
// are exact in fp32), so one conversion and one dot per two weights.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float f4_group16_bx(uint32_t lo, uint32_t hi, const uint32_t *xw) {
    float a = 0.0f;
    const uint32_t w[2] = {lo, hi};
#pragma unroll
    for (int d = 0; d < 2; d++) {
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 0),
                                            __builtin_bit_cast(bf16x2_t, xw[d * 4 + 0]), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 1),
                                            __builtin_bit_cast(bf16x2_t, xw[d * 4 + 1]), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 2),
                                            __builtin_bit_cast(bf16x2_t, xw[d * 4 + 2]), a, false);
        a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], 1.0f, 3),
                                            __builtin_bit_cast(bf16x2_t, xw[d * 4 + 3]), a, false);
    }
    return a;
}
__device__ __forceinline__ float f4_chunk_bx(uint4 w, uint32_t s2b, const uint32_t *xw) {
    const float g0 = f4_group16_bx(w.x, w.y, xw);
    const float g1 = f4_group16_bx(w.z, w.w, xw + 8);
    return fmaf(e4m3_scale(s2b & 0xFFu), g0, e4m3_scale((s2b >> 8) & 0xFFu) * g1);
}
// with the two block scales already decoded (sc.x: values 0..15, sc.y: 16..31)
__device__ __forceinline__ float f4_chunk_bx(uint4 w, f32x2_t sc, const uint32_t *xw) {
    const float g0 = f4_group16_bx(w.x, w.y, xw);
    const float g1 = f4_group16_bx(w.z, w.w, xw + 8);
    return fmaf(sc.x, g0, sc.y * g1);
}

// NVFP4 chunk against scaled fp16 activations: 32 e2m1 codes (w), two e4m3
// block scales (s2b), the 32 activations as 16 fp16 pairs (xw) in two
// 16-value chunks with inverse scales isc0, isc1 (chunk16_to_f16). Codes are
// converted to fp16 pairs (v_cvt_scalef32_pk_f16_fp4, unit scale: exact) and
// multiplied by v_dot2_f32_f16; each 16-value group is scaled once.
__device__ __forceinline__ float f4_group16_h(uint32_t lo, uint32_t hi, const uint32_t *xw) {
    float a = 0.0f;
    const uint32_t w[2] = {lo, hi};
#pragma unroll
    for (int d = 0; d < 2; d++) {
        a = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w[d], 1.0f, 0), as_h2(xw[d * 4 + 0]), a, false);
        a = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w[d], 1.0f, 1), as_h2(xw[d * 4 + 1]), a, false);
        a = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w[d], 1.0f, 2), as_h2(xw[d * 4 + 2]), a, false);
        a = __builtin_amdgcn_fdot2(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w[d], 1.0f, 3), as_h2(xw[d * 4 + 3]), a, false);
    }
    return a;
}
__device__ __forceinline__ float f4_chunk_h(uint4 w, f32x2_t sc, const uint32_t *xw, float isc0, float isc1) {
    const float g0 = f4_group16_h(w.x, w.y, xw);
    const float g1 = f4_group16_h(w.z, w.w, xw + 8);
    return fmaf(sc.x * isc0, g0, (sc.y * isc1) * g1);
}

// ---- Philox-4x32-10 (Salmon et al. 2011) ------------------------------------
struct u4 { uint32_t v[4]; };
__device__ __forceinline__ u4 philox(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                     uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; r++) {
        const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        if (r != 9) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
    }
    u4 o; o.v[0] = c0; o.v[1] = c1; o.v[2] = c2; o.v[3] = c3;
    return o;
}

}  // namespace qfm
