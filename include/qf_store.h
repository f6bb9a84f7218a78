/*
 * qf_store.h -- expert arena ingest and residency for the MI355X MoE path.
 *
 * The on-disk side of the drop-in: the reference engine's mmap'd weight store
 * (ocho/amd_server/qwenflash.h:12-39, reader.cpp), its fixed-slot expert
 * cache (ocho/amd_server/qf_nvfp4_wave64.h:125-247, qf_expert_slots.cpp) and
 * the device-resident LRU dispatch that drives it (qf_router_wave64.h:62-106).
 * Struct layouts are byte-compatible with the reference's so an engine built
 * against them passes the same objects; reference-named entry points keep the
 * reference's names, argument order, return values and meaning.
 *
 * Store formats accepted by qf_store_open(path):
 *   - the reference's index: path is a directory holding shards.txt (one shard
 *     file path per line) and manifest.bin (an array of 512-byte QfEntry
 *     records; data_off is the tensor's byte offset in its shard file);
 *   - safetensors, read directly: path is one .safetensors file or a directory
 *     of them (every regular file whose name ends in ".safetensors", in byte
 *     order of the file names). The index is built from each file's JSON
 *     header: dtype code, ne[] (fastest first), absolute data offset, nbytes;
 *     for "X.weight" entries scale2_off/scale2_file point at "X.weight_scale_2"
 *     and input_off/input_file at "X.input_scale" when those exist.
 * Both forms are validated at open: every entry must lie inside its mapped
 * shard, names must be unique and NUL-terminated, and a safetensors entry's
 * byte count must equal its shape times its element size.
 */
#ifndef QF_STORE_H
#define QF_STORE_H
#include "qf_moe.h"

#ifdef __cplusplus
extern "C" {
#endif
#pragma GCC visibility push(default)

#define QF_MAX_NAME 256
#define QF_REC_SIZE 512
#define QF_MANIFEST_MAGIC 0x51464D31u  /* "QFM1" */
#define QF_ROUTE_MB_CAP 16

/* dtype codes (qwenflash.h:16): 1..5 are the reference's; 6.. are this
 * library's additions for the other safetensors dtypes. */
enum {
    QF_DT_BF16 = 1, QF_DT_F32 = 2, QF_DT_U8 = 3, QF_DT_F8_E4M3 = 4, QF_DT_I64 = 5,
    QF_DT_F16 = 6, QF_DT_I8 = 7, QF_DT_I32 = 8, QF_DT_F64 = 9, QF_DT_F8_E5M2 = 10,
    QF_DT_I16 = 11, QF_DT_U16 = 12, QF_DT_U32 = 13, QF_DT_U64 = 14, QF_DT_BOOL = 15
};

/* One tensor of the store (qwenflash.h:12-24). */
typedef struct {
    uint32_t file_idx;
    uint32_t dtype;
    uint64_t ne[4];          /* dims, fastest first; unused dims are 1 */
    uint64_t data_off;       /* byte offset into the shard file */
    uint64_t nbytes;
    uint64_t scale2_off;     /* weight_scale_2 offset, 0 if absent */
    uint64_t input_off;      /* input_scale offset, 0 if absent */
    uint32_t scale2_file;
    uint32_t input_file;
    uint32_t flags;
} QfRec;

/* One 512-byte manifest record (qwenflash.h:26-30). */
typedef struct {
    char    name[QF_MAX_NAME];
    QfRec   rec;
    uint8_t _pad[168];
} QfEntry;

/* The opened store (qwenflash.h:32-39): entries sorted by name (strcmp). */
typedef struct {
    int      n_shards;
    char   (*shard_paths)[1024];
    int     *shard_fds;
    void   **shard_maps;
    size_t  *shard_sizes;
    QfEntry *entries;
    int      n_entries;
} QfStore;

/* Miss mailbox of the non-resident arena (qwenflash.h:73-83): written on the
 * device by qf_rtr_dispatch into pinned mapped host memory, seq last. */
struct QfRouteMailbox {
    volatile uint32_t seq;
    volatile uint32_t miss_n;
    volatile int32_t  miss_expert[QF_ROUTE_MB_CAP];
    volatile int32_t  miss_slot[QF_ROUTE_MB_CAP];
};

/* Per-GPU transfer context (qf_nvfp4_wave64.h:178-183): two pinned staging
 * buffers (one expert slot each, sized for the largest supported shape), one
 * event per buffer, one transfer stream. */
typedef struct {
    void        *buf[2];
    hipEvent_t   ev[2];
    int          cur;
    hipStream_t  xfer;
} Qf4ExpXfer;

/* ---- store (reader.cpp) -------------------------------------------------- */
/* 0 on success; -1 nothing to open at path (no shards.txt, no .safetensors),
 * -2 manifest.bin unreadable or not a whole number of records, -3 a shard
 * could not be opened, -4 a shard could not be mapped, -5 an invalid index or
 * safetensors header (message in qfm_last_error). On failure st is left
 * closed. Replaces qf_store_open (ocho/amd_server/reader.cpp:15-61). */
int            qf_store_open(QfStore *st, const char *path);
/* Binary search by exact name; NULL when absent. Replaces qf_find (reader.cpp:63-72). */
const QfEntry *qf_find(const QfStore *st, const char *name);
/* Unmaps and frees; st is zeroed. Replaces qf_store_close (reader.cpp:74-88). */
void           qf_store_close(QfStore *st);
/* Host address of an entry's bytes (shard base + data_off). */
const void    *qfm_store_data(const QfStore *st, const QfEntry *e);

/* ---- expert cache (qf_expert_slots.cpp) ---------------------------------- */
/* Modes of qfm_expcache_init (the reference picks them from the environment:
 * QF8_MOE_FP8, QF_M1_INT8, QF_M1_INT8_ONLY; qf_expert_slots.cpp:105-144). */
#define QFM_EXPCACHE_NVFP4     1   /* NVFP4 slot arrays (checkpoint form) */
#define QFM_EXPCACHE_INT8      2   /* + INT8 slot arrays built from NVFP4 on load */
#define QFM_EXPCACHE_INT8_ONLY 4   /* with INT8: the NVFP4 arrays are a 2-slot staging ring */
#define QFM_EXPCACHE_FP8       8   /* FP8 lane-chunk arrays instead of NVFP4 */

int  qf4_expxfer_init(Qf4ExpXfer *xf);                       /* qf_expert_slots.cpp:35-57 */
void qf4_expxfer_free(Qf4ExpXfer *xf);                       /* :59-66 */
/* Allocates `slots` device slots (slots <= 0: QF_EXPERT_CACHE_SLOTS, else 192;
 * clamped to n_experts; at least top_k), the host maps (all empty), the per-expert scale_2
 * tables (host and device, read from the store's weight_scale_2 tensors), the
 * device routing state and the pinned miss mailbox. Modes from the
 * environment as in the reference. Replaces qf4_expcache_init (:91-204). */
int  qf4_expcache_init(Qf4ExpCache *c, const QfStore *st, int layer, int slots);
/* The same with the modes given explicitly (QFM_EXPCACHE_*; the environment is
 * not read). FP8 excludes NVFP4 and INT8; INT8_ONLY needs INT8 and NVFP4. */
int  qfm_expcache_init(Qf4ExpCache *c, const QfStore *st, int layer, int slots, int modes);
/* Device bytes qfm_expcache_init(.., slots, modes) allocates at the current
 * shape (slot arrays, scales, device routing state); 0 for invalid modes or
 * slots. The init prices this before allocating (qfm_set_hbm_budget). */
size_t qfm_expcache_bytes(int slots, int modes);
/* Releases every device, host and pinned allocation of the cache (also those
 * of a synthetic arena from qfm_arena_init). Replaces qf4_expcache_free (:206-228). */
void qf4_expcache_free(Qf4ExpCache *c);
/* Full residency: uploads every expert into slot == expert, sets the host and
 * device maps to the identity and fully_resident = 1 (INT8_ONLY: each expert
 * goes through the staging ring and is converted into its INT8 slot). The
 * copies are ordered before later work on `compute`. Returns 1 when fully
 * resident, 0 when slots < n_experts, -1 on error. Replaces
 * qf4_expcache_prefill (:345-365). */
int  qf4_expcache_prefill(Qf4ExpCache *c, const QfStore *st, Qf4ExpXfer *xf, hipStream_t compute);
/* Host-side LRU: the slot holding `expert`, loading it on a miss (first empty
 * slot, else the least recently used). Returns the slot or -1. Replaces
 * qf4_expcache_prepare (:367-391). */
int  qf4_expcache_prepare(Qf4ExpCache *c, const QfStore *st, Qf4ExpXfer *xf, int expert,
                          hipStream_t compute);
/* Host side of the device dispatch: waits (bounded) until the mailbox carries
 * seq == c->expected_seq, uploads each recorded miss into its device-chosen
 * slot, orders `compute` after the copies, clears miss_n. 0 or -1. Replaces
 * qf4_expcache_service (:422-459). */
int  qf4_expcache_service(Qf4ExpCache *c, const QfStore *st, Qf4ExpXfer *xf, hipStream_t compute);
/* Cumulative lookups, misses and bytes uploaded. Replaces qf4_expcache_stats (:412-420). */
void qf4_expcache_stats(unsigned long long *calls, unsigned long long *miss, unsigned long long *bytes);

/* NVFP4 expert (checkpoint form, rows x in) -> FP8 lane-chunk form: every row
 * cut into 64 contiguous chunks of in/64 values; chunk l's values v =
 * e2m1 * (ue4m3 * s2) are stored as E4M3 codes of v / sc[row][l] with
 * sc = chunk absmax / 448 (1 for an all-zero chunk). Host function, run once
 * per (expert, projection) at load. in a multiple of 64 and of 16. Replaces
 * qf8_fp8_pack_expert (ocho/amd_server/qf8_moe_fp8.h:57-59, qf8_moe_fp8.hip:217-246). */
int  qf8_fp8_pack_expert(const uint8_t *nvfp4_w, const uint8_t *nvfp4_s, float s2, int rows, int in,
                         uint8_t *w8_out, float *scale_out);

/* ---- device dispatch (qf_router_wave64.hip:173-256) ----------------------- */
/* One token's K = top_k selections sel_ids[0..K) -> route_slot[0..K): hits
 * refresh their slot's age (++clock); a miss takes the slot with the smallest
 * (age, slot) pair, unmaps its previous expert, maps the new one and posts
 * (expert, slot) to the mailbox; miss_n, then seq, are published last
 * (system-scope release). The maps/ages/clock are the cache's *_dev arrays;
 * mb its mb_dev; nslots in [top_k, min(n_experts, 512)]. The _ex form returns
 * 0, or -1 / -2 on a rejected argument (nothing launched), -3 on a launch
 * error. Replaces qf_rtr_dispatch / qf_rtr_dispatch_launch (qf_router_wave64.h:62-69, :99-106). */
void qf_rtr_dispatch_launch(const int *sel_ids, int *slot_for_expert, int *expert_in_slot, uint64_t *age,
                            uint64_t *clock, int *route_slot, volatile QfRouteMailbox *mb, uint32_t seq, int nslots,
                            hipStream_t s);
int  qf_rtr_dispatch_launch_ex(const int *sel_ids, int *slot_for_expert, int *expert_in_slot, uint64_t *age,
                               uint64_t *clock, int *route_slot, volatile QfRouteMailbox *mb, uint32_t seq,
                               int nslots, hipStream_t s);
/* hist[e] += 1 for each of the K selections (atomic, order-free). Replaces
 * qf_rtr_hist / qf_rtr_hist_launch (qf_router_wave64.h:54, :85-90). */
void qf_rtr_hist_launch(const int *sel_ids, unsigned int *hist, hipStream_t s);
int  qf_rtr_hist_launch_ex(const int *sel_ids, unsigned int *hist, hipStream_t s);

/* ---- dense tensors ------------------------------------------------------- */
/* bf16 [rows][K] -> int8 [rows][K] + fp32 [rows] per-row scale: s = absmax/127
 * (1 for an all-zero row), q = rint(w * (1/s)) clamped to +-127. Allocates
 * m->w / m->s. The _host form reads a host matrix through a bounded staging
 * buffer. K >= 16, K % 16 == 0. Replace qf8_i8_quant_bf16 and
 * qf8_i8_quant_bf16_host (ocho/amd_server/qf8_dense_i8.h:24-28). */
int  qf8_i8_quant_bf16(const uint16_t *W, int rows, int K, Qf8I8Mat *m, hipStream_t s);
int  qf8_i8_quant_bf16_host(const uint16_t *Whost, int rows, int K, Qf8I8Mat *m, hipStream_t s);

/* ---- whole MoE layer from a store ---------------------------------------- */
/* Builds out->layer from the store's tensors of `layer`: router
 * mlp.gate.weight (BF16 or F32 [E][H] -> fp32), shared expert
 * mlp.shared_expert.{gate,up,down}_proj.weight (BF16, or F32 rounded to BF16
 * -> per-row INT8 via qf8_i8_quant_bf16), shared gate vector
 * mlp.shared_expert_gate.weight (-> fp32 [H]) and the routed experts into a
 * fully resident arena (fmt QFM_FMT_NVFP4: NVFP4 slots; QFM_FMT_INT8: INT8
 * slots through the staging ring). Names and byte-count checks follow
 * qf_hip4_stage.hip:530-580, :628-641 and qf_expert_slots.cpp:230-251.
 * Release with qfm_synth_layer_destroy. 0 or a negative code. */
int  qfm_layer_load(qfm_synth_layer *out, const QfStore *st, int layer, int fmt, Qf4ExpXfer *xf,
                    hipStream_t s);
/* Host-only preflight: checks that every tensor qfm_layer_load would read for
 * `layer` exists with the expected byte count (no device work). Returns 0, or
 * -1 with the first missing or mis-sized tensor in qfm_last_error. */
int  qfm_store_check_layer(const QfStore *st, int layer);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif
