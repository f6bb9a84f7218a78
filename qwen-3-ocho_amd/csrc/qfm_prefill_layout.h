// qfm_prefill_layout.h -- the prefill workspace carve-up, in one place.
//
// Plain C++ (no HIP): the launcher, the workspace sizing and the workspace
// view all take their offsets from pf_layout(), and the CPU tests replay it
// (tests/test_prefill_layout.py) for every token count, format, shape and
// tile width to check that the regions are disjoint, inside the workspace,
// and large enough for everything the planning and GEMM kernels index.
#pragma once
#include <stddef.h>

namespace qfm {

// Regions of the prefill workspace, in address order.
enum PfRegion {
    kPfLg,        // fp32 [slices][T][E] approximate router logits (slice 0 ends as the view's logits)
    kPfXnorm,     // fp32 [T] ||x_t||
    kPfWnorm,     // fp32 [E] ||w_e||
    kPfWb16,      // bf16 [E][H] router weights
    kPfSel,       // int [T][K]
    kPfWts,       // fp32 [T][K]
    kPfGam,       // fp32 [T] shared-expert gate
    kPfCtr,       // int [8] {candidate overflows, gate/up items, down items, ...}
    kPfOff,       // int [E + 2] group offsets
    kPfBlk,       // int [nblk][E] per counting block histograms
    kPfItemsGu,   // int4 [max_mt * nt_gu] gate/up work items, each at the index of the block that runs it
    kPfItemsDn,   // int4 [max_mt * nt_dn] down work items, likewise
    kPfTok,       // int [P] pair -> token
    kPfSlot,      // int [P] pair -> partial slot
    kPfPwt,       // fp32 [P] pair weight
    kPfHid,       // bf16 [P][I] hidden rows
    kPfPart,      // fp16 [P][H] owned partials, each 64-column group scaled by 2^k
    kPfPartK,     // int8 [P][H / 64] the k of each partial group
    kPfXsum,      // fp32 [T] sum(x_t)
    kPfHsum,      // fp32 [P][nt_gu] hidden row sums per gate/up n-tile
    kPfX16,       // fp16 [T][H] x rows scaled by 2^k (INT8 gate/up)
    kPfX16sum,    // fp32 [T]
    kPfX16isc,    // fp32 [T]
    kPfCount
};

struct PfLayout {
    size_t off[kPfCount], bytes[kPfCount];
    size_t total;              // bytes from the first region to the end of the last
    size_t P;                  // pairs: T * (K + shared)
    size_t max_mt;             // bound on the 128-row m-tiles over all groups (a multiple of 8)
    int nt_gu, nt_dn;          // n-tiles of the gate/up and down GEMMs
    int nblk;                  // counting / scatter blocks
};

// T tokens; (H, I, E, K) the configuration; has_sh: shared expert present;
// gu_rows: weight rows per gate/up tile (gate and up interleaved: I / (gu_rows
// / 2) n-tiles); dn_cols: output columns per down tile; bm: rows per m-tile;
// slices: router GEMM k-slices; pairs_per_blk: pairs per counting block.
inline PfLayout pf_layout(int T, int H, int I, int E, int K, bool has_sh, int gu_rows, int dn_cols, int bm,
                          int slices, int pairs_per_blk) {
    PfLayout L{};
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t t = (size_t)T;
    L.P = t * (size_t)(K + (has_sh ? 1 : 0));
    L.nt_gu = I / (gu_rows / 2);
    L.nt_dn = H / dn_cols;
    L.nblk = (int)((t * K + pairs_per_blk - 1) / pairs_per_blk);
    // every group of c rows takes ceil(c / bm) <= c / bm + 1 m-tiles: at most
    // P / bm + (E + 1) over the E routed groups and the shared one
    L.max_mt = (L.P / bm + E + 2 + 7) / 8 * 8;
    const size_t want[kPfCount] = {
        (size_t)slices * t * E * 4, t * 4, (size_t)E * 4, (size_t)E * H * 2, t * K * 4, t * K * 4, t * 4, 8 * 4,
        (size_t)(E + 2) * 4, (size_t)L.nblk * E * 4, L.max_mt * L.nt_gu * 16, L.max_mt * L.nt_dn * 16,
        L.P * 4, L.P * 4, L.P * 4, L.P * I * 2, L.P * H * 2, L.P * (size_t)(H / 64), t * 4, L.P * L.nt_gu * 4,
        t * H * 2, t * 4, t * 4};
    size_t o = 0;
    for (int r = 0; r < kPfCount; r++) {
        L.off[r] = o;
        L.bytes[r] = want[r];
        o += al(want[r]);
    }
    L.total = o;
    return L;
}

}  // namespace qfm
