// Host-only view of the prefill workspace carve-up for tests/test_prefill_layout.py:
// exposes pf_layout (qwen-3-ocho_amd/csrc/qfm_prefill_layout.h) through a C ABI.
#include "../qwen-3-ocho_amd/csrc/qfm_prefill_layout.h"

extern "C" int pf_layout_c(int T, int H, int I, int E, int K, int has_sh, int gu_rows, int dn_cols, int bm, int slices,
                           int pairs_per_blk, unsigned long long *off, unsigned long long *bytes,
                           unsigned long long *meta) {
    const qfm::PfLayout L = qfm::pf_layout(T, H, I, E, K, has_sh != 0, gu_rows, dn_cols, bm, slices, pairs_per_blk);
    for (int r = 0; r < qfm::kPfCount; r++) {
        off[r] = L.off[r];
        bytes[r] = L.bytes[r];
    }
    meta[0] = L.total; meta[1] = L.P; meta[2] = L.max_mt;
    meta[3] = (unsigned long long)L.nt_gu; meta[4] = (unsigned long long)L.nt_dn; meta[5] = (unsigned long long)L.nblk;
    return qfm::kPfCount;
}
