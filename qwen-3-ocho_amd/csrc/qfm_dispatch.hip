// qfm_dispatch.hip -- device side of the non-resident expert arena: the LRU
// slot dispatch that maps a token's top-K experts to cache slots and posts
// the misses to the pinned host mailbox, and the selection histogram.
//
// Dispatch semantics (ocho/amd_server/qf_router_wave64.hip:183-256), for
// k = 0 .. K-1 in order: a resident expert (slot_for_expert[e] >= 0) is a hit
// and its slot's age becomes ++clock; otherwise the victim is the slot with
// the smallest (age, slot index) pair, its previous expert (if any) is
// unmapped, e is mapped to it, its age becomes ++clock and (e, slot) is
// appended to the mailbox (at most QF_ROUTE_MB_CAP entries). route_slot[k]
// receives the slot either way. Then miss_n, and seq last, are published to
// the host.
//
// One wave does the whole token: the slot map, the reverse map and the ages
// are read into LDS once, the K sequential steps run on LDS (victim search:
// each lane scans every 64th slot, then a wave-wide minimum of the packed
// key age * 1024 + slot), and every table is written back once at the end.
// Mailbox stores go to fine-grained (coherent) pinned host memory; seq is a
// system-scope release store after them.
#include "qfm_internal.h"
#include "../../include/qf_store.h"

namespace qfm {

constexpr int kDispMaxSlots = 512;
constexpr int kDispMaxExperts = 512;

__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(v, off, 64);
        v = o < v ? o : v;
    }
    return v;
}

__global__ void __launch_bounds__(64)
k_rtr_dispatch(const int *__restrict__ sel, int K, int *__restrict__ slot_for_expert, int *__restrict__ expert_in_slot,
               uint64_t *__restrict__ age, uint64_t *__restrict__ clock, int *__restrict__ route_slot,
               QfRouteMailbox *mb, uint32_t seq, int nslots, int n_experts) {
    __shared__ int s_sfe[kDispMaxExperts];
    __shared__ int s_eis[kDispMaxSlots];
    __shared__ unsigned long long s_age[kDispMaxSlots];
    __shared__ int s_route[QF_ROUTE_MB_CAP], s_miss_e[QF_ROUTE_MB_CAP], s_miss_s[QF_ROUTE_MB_CAP];
    const int lane = threadIdx.x;
    for (int i = lane; i < n_experts; i += 64) s_sfe[i] = slot_for_expert[i];
    for (int i = lane; i < nslots; i += 64) {
        s_eis[i] = expert_in_slot[i];
        s_age[i] = age[i];
    }
    unsigned long long clk = *clock;
    int nmiss = 0;
    __syncthreads();
    for (int k = 0; k < K; k++) {
        const int e = sel[k];
        const bool valid = e >= 0 && e < n_experts;
        int slot = valid ? s_sfe[e] : -1;
        if (valid && slot < 0) {
            unsigned long long best = ~0ull;
            for (int i = lane; i < nslots; i += 64) {
                const unsigned long long key = s_age[i] * 1024ull + (unsigned long long)i;
                best = key < best ? key : best;
            }
            best = wave_min_u64(best);
            slot = (int)(best & 1023ull);
            if (lane == 0) {
                const int ev = s_eis[slot];
                if (ev >= 0) s_sfe[ev] = -1;
                s_sfe[e] = slot;
                s_eis[slot] = e;
                if (nmiss < QF_ROUTE_MB_CAP) {
                    s_miss_e[nmiss] = e;
                    s_miss_s[nmiss] = slot;
                }
            }
            nmiss = min(nmiss + 1, QF_ROUTE_MB_CAP);
        }
        if (lane == 0) {
            if (slot >= 0) s_age[slot] = ++clk;
            s_route[k] = slot;
        }
        __syncthreads();
    }
    for (int i = lane; i < n_experts; i += 64) slot_for_expert[i] = s_sfe[i];
    for (int i = lane; i < nslots; i += 64) {
        expert_in_slot[i] = s_eis[i];
        age[i] = s_age[i];
    }
    if (lane < K) route_slot[lane] = s_route[lane];
    if (lane < nmiss) {
        mb->miss_expert[lane] = s_miss_e[lane];
        mb->miss_slot[lane] = s_miss_s[lane];
    }
    if (lane == 0) {
        *clock = clk;
        mb->miss_n = (uint32_t)nmiss;
    }
    __syncthreads();
    if (lane == 0)
        __hip_atomic_store(const_cast<uint32_t *>(&mb->seq), seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void __launch_bounds__(64) k_rtr_hist(const int *__restrict__ sel, int K, unsigned *__restrict__ hist,
                                                 int n_experts) {
    const int k = threadIdx.x;
    if (k < K) {
        const int e = sel[k];
        if (e >= 0 && e < n_experts) atomicAdd(&hist[e], 1u);
    }
}

}  // namespace qfm

using namespace qfm;

extern "C" {

int qf_rtr_dispatch_launch_ex(const int *sel_ids, int *slot_for_expert, int *expert_in_slot, uint64_t *age,
                              uint64_t *clock, int *route_slot, volatile QfRouteMailbox *mb, uint32_t seq, int nslots,
                              hipStream_t s) {
    const int E = g_cfg.E, K = g_cfg.K;
    if (!sel_ids || !slot_for_expert || !expert_in_slot || !age || !clock || !route_slot || !mb) {
        set_error(-1, "qf_rtr_dispatch_launch: null argument");
        return -1;
    }
    if (nslots < K || nslots > kDispMaxSlots || nslots > E || E > kDispMaxExperts || K > QF_ROUTE_MB_CAP) {
        set_error(-2, "qf_rtr_dispatch_launch: nslots = %d outside [top_k %d, %d]", nslots, K,
                  E < kDispMaxSlots ? E : kDispMaxSlots);
        return -2;
    }
    hipLaunchKernelGGL(k_rtr_dispatch, dim3(1), dim3(64), 0, s, sel_ids, K, slot_for_expert, expert_in_slot, age,
                       clock, route_slot, const_cast<QfRouteMailbox *>(mb), seq, nslots, E);
    return check_launch("qf_rtr_dispatch") ? -3 : 0;
}

void qf_rtr_dispatch_launch(const int *sel_ids, int *slot_for_expert, int *expert_in_slot, uint64_t *age,
                            uint64_t *clock, int *route_slot, volatile QfRouteMailbox *mb, uint32_t seq, int nslots,
                            hipStream_t s) {
    (void)qf_rtr_dispatch_launch_ex(sel_ids, slot_for_expert, expert_in_slot, age, clock, route_slot, mb, seq, nslots,
                                    s);
}

int qf_rtr_hist_launch_ex(const int *sel_ids, unsigned int *hist, hipStream_t s) {
    if (!sel_ids || !hist) {
        set_error(-1, "qf_rtr_hist_launch: null argument");
        return -1;
    }
    if (g_cfg.K > 64) {
        set_error(-2, "qf_rtr_hist_launch: top_k %d above 64", g_cfg.K);
        return -2;
    }
    hipLaunchKernelGGL(k_rtr_hist, dim3(1), dim3(64), 0, s, sel_ids, g_cfg.K, hist, g_cfg.E);
    return check_launch("qf_rtr_hist") ? -3 : 0;
}

void qf_rtr_hist_launch(const int *sel_ids, unsigned int *hist, hipStream_t s) {
    (void)qf_rtr_hist_launch_ex(sel_ids, hist, s);
}

}  // extern "C"
