// ref_exports.hip -- TEST INFRASTRUCTURE ONLY. Part of the oracle/_ref build
// of the reference's own HIP kernels (compiled in place from the reference
// checkout by oracle/Makefile's `ref` target, never copied): the reference
// declares its router launchers `static inline` in qf_router_wave64.h
// (:80-106), so they have no exported symbol; these wrappers export them under
// ref_* names for the cross-check tests. No arithmetic here.
#include "qf_router_wave64.h"

extern "C" {
void ref_rtr_gemv(const uint16_t *router, const float *x, float *logits, hipStream_t s) {
    qf_rtr_gemv_launch(router, x, logits, s);
}
void ref_rtr_topk10(const float *logits, int *sel_ids, float *wts, hipStream_t s) {
    qf_rtr_topk10_launch(logits, sel_ids, wts, s);
}
void ref_rtr_topk10_rows(const float *logits, int *sel_ids, float *wts, int T, hipStream_t s) {
    qf_rtr_topk10_rows_launch(logits, sel_ids, wts, T, s);
}
void ref_rtr_dispatch(const int *sel_ids, int *slot_for_expert, int *expert_in_slot, uint64_t *age, uint64_t *clock,
                      int *route_slot, volatile QfRouteMailbox *mb, uint32_t seq, int nslots, hipStream_t s) {
    qf_rtr_dispatch_launch(sel_ids, slot_for_expert, expert_in_slot, age, clock, route_slot, mb, seq, nslots, s);
}
void ref_rtr_hist(const int *sel_ids, unsigned int *hist, hipStream_t s) { qf_rtr_hist_launch(sel_ids, hist, s); }
}
