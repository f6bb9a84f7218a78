/*
 * qfm_oracle.h -- CPU restatement of the quantized MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * implementation: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load it.  Nothing in the product path (the HIP library
 * libqfm.so and its host code) links, loads or calls it.
 *
 * Reference files restated (paths relative to the reference checkout):
 *   router softmax / top-k / renorm  ocho/amd_server/qf_router_wave64.hip:69-155,
 *                                    ocho/engine_spark/cuda/qf.cu:1184-1271
 *   INT8 expert (exact + X8 modes)   ocho/amd_server/qf8_moe_i8.hip:58-144
 *   NVFP4 -> INT8 arena build        ocho/amd_server/qf8_moe_i8.hip:146-195
 *   dense bf16 -> INT8 per row       ocho/amd_server/qf8_dense_i8.hip:41-60
 *   FP8 lane-chunk format            ocho/amd_server/qf8_moe_fp8.hip:19-37, :217-246
 *   INT8 x X8 GEMV, hyper-connection ocho/amd_server/qf8_dense_i8.hip:78-175, qf8_hc.hip:99-103
 *   NVFP4 decode / expert            ocho/amd_server/qf_nvfp4_wave64.hip:10-21, 62-101,
 *                                    :175-216, :406-454
 *   routing inversion (CSR)          ocho/amd_server/qf8_moe_i8.hip:323-358,
 *                                    ocho/amd_server/qf_moe_m8_wave64.hip:261-299
 *   shared expert (+sigmoid gate)    ocho/amd_server/qf8_dense_i8.hip:173-181, :346-358
 *   Philox-4x32-10                   stoch/include/philox.cuh:17-35 (KAT at :11)
 *
 * Every function is plain C, compiled with -ffp-contract=off so that the
 * floating-point operation order written here is the one executed.
 *
 * Parity pinning (what checks each function; see tests/test_oracle_*.py):
 *   orc_philox4x32_10      Random123 / reference KAT (ctr = key = 0), two more KATs
 *   orc_e2m1 / orc_e4m3    exhaustive 16 / 256 code tables vs the closed forms and the
 *                          reference's LUT form (qf.cu:163-172)
 *   orc_e4m3_encode        round trip over all finite codes + brute-force nearest
 *   orc_bf16_rne           numpy bit-level RNE restatement over 2^20 random floats
 *   orc_router_logits      fp64 numpy matmul within the fp32 error bound; exact on
 *                          power-of-two inputs; canonical order reproduced in numpy
 *   orc_topk               brute force (numpy lexsort) + constructed tie catalogue
 *   orc_i8_expert          numpy fp64 matmul of the dequantized weights; closed forms
 *                          on one-hot weights; zero input
 *   orc_nvfp4_expert       numpy fp64 matmul after an independent numpy dequant
 *   orc_csr_build          invariants (permutation, ascending ids, token order)
 *   orc_x8_quant           numpy restatement + invariants (|q| <= 127, q*s ~ v)
 *   orc_m8_reduce4         exact integer sums; an order-sensitive case whose
 *                          result differs for every other association
 *   orc_nvfp4_to_i8        closed forms: the row maximum maps to +-127, an
 *                          all-zero row keeps scale 1, constant rows, codes
 *                          reconstruct within scale/2, 5-bit exponent field
 *   orc_i8_quant_bf16      closed forms: row maximum -> +-127, all-zero row keeps
 *                          scale 1, exact half-way ties round to even (rint,
 *                          not round), clamp; numpy restatement on random rows
 *   orc_f8_decode          all 256 codes vs torch float8_e4m3fn (0x7F / 0xFF: closed form 480)
 *   orc_f8_encode          round trip over every code it emits; nearest-even vs torch on the
 *                          normal range; closed forms for the truncated subnormals, the flush
 *                          below 2^-9 and the saturation from 2^8 up
 *   orc_fp8_pack_expert    chunk maximum -> 0x7E, zero chunk keeps scale 1, numpy
 *                          restatement of the value formula on random experts
 *   orc_i8_gemv            numpy fp64 matmul of codes x dequantized X8 rows; closed forms of
 *                          the two activations; one-hot rows
 *   orc_hc_norm            numpy restatement; unit-RMS rows give normed = R * (1 + w)
 *   orc_hc_combine         numpy restatement; equal streams reduce to sigmoid * normed
 *   orc_stream_inject      numpy float32 fma restatement (np.float32 products rounded once)
 *   orc_shexp_bf16         numpy fp64 matmuls of the bf16 weights; closed forms: one-hot gate /
 *                          up / down rows pick single activations, zero x leaves y unchanged,
 *                          a zero gate_inp row gives the factor sigmoid(0) = 1/2
 *   orc_moe_layer          recomposition from the pieces with numpy fp64 experts
 */
#ifndef QFM_ORACLE_H
#define QFM_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- synthetic data generator (identical definition on the device side) ---- */
enum {
    ORC_T_QG = 1, ORC_T_QU = 2, ORC_T_QD = 3,      /* int8 codes            */
    ORC_T_SG = 4, ORC_T_SU = 5, ORC_T_SD = 6,      /* per-row fp32 scales   */
    ORC_T_ROUTER = 7, ORC_T_X = 8, ORC_T_SHGATE = 9, ORC_T_BIAS = 10,
    ORC_T_FG = 11, ORC_T_FU = 12, ORC_T_FD = 13,   /* packed e2m1 bytes     */
    ORC_T_FSG = 14, ORC_T_FSU = 15, ORC_T_FSD = 16 /* e4m3 block scales     */
};
void     orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
uint32_t orc_word(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t j);
int8_t   orc_gen_i8(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n);
float    orc_gen_rowscale(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n);
float    orc_gen_gauss(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n);
uint8_t  orc_gen_fp4byte(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n);
uint8_t  orc_gen_e4m3scale(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n);
/* bulk forms (OpenMP over n) */
void orc_fill_i8(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, int8_t *out);
void orc_fill_rowscale(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, float *out);
void orc_fill_gauss(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, float scale, float *out);
void orc_fill_gauss_bf16(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, uint16_t *out);
void orc_fill_fp4byte(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, uint8_t *out);
void orc_fill_e4m3scale(uint32_t seed, uint32_t layer, uint32_t tensor, uint64_t n0, uint64_t cnt, uint8_t *out);

/* ---- number formats ---- */
float    orc_e2m1(uint32_t nib);
float    orc_e4m3(uint32_t b);
uint8_t  orc_e4m3_encode(float v);          /* nearest, ties to even; finite positive normals */
uint16_t orc_bf16_rne(float f);
float    orc_bf16_to_f32(uint16_t h);

/* ---- router ---- */
/* logits[m][e] in the canonical fp32 order; x is bf16 [M][H]; bias optional [E] */
void orc_router_logits(const float *W, const uint16_t *x, const float *bias,
                       int M, int E, int H, float *logits);
/* top-K by descending logit, ties to the lower index; weights renormalized
   over the K selected (renorm = 1) or plain softmax probabilities (renorm = 0).
   w64 receives the fp64 weights, w32 the fp32 form. */
void orc_topk(const float *logits, int M, int E, int K, int renorm,
              int *sel, double *w64, float *w32);

/* ---- experts (fp64 accumulate) ---- */
/* h[r] = silu(sg_r <Qg_r,x>) * (su_r <Qu_r,x>), y[c] = sd_c <Qd_c,h> */
void orc_i8_expert(const double *x, const int8_t *Qg, const float *sg,
                   const int8_t *Qu, const float *su, const int8_t *Qd, const float *sd,
                   int H, int I, double *h, double *y);
void orc_nvfp4_expert(const double *x, const uint8_t *Fg, const uint8_t *Sg, float s2g,
                      const uint8_t *Fu, const uint8_t *Su, float s2u,
                      const uint8_t *Fd, const uint8_t *Sd, float s2d,
                      int H, int I, double *h, double *y);
/* dequantize one NVFP4 matrix [rows][K] into fp64 */
void orc_nvfp4_dequant(const uint8_t *F, const uint8_t *S, float s2, int rows, int K, double *out);

/* ---- NVFP4 -> INT8 arena conversion (bit-exact restatement) ---- */
void orc_nvfp4_to_i8(const uint8_t *W, const uint8_t *S, float s2, int rows, int K, int8_t *Wo, float *So);
/* dense bf16 [rows][K] -> per-row INT8 codes + fp32 scales (qf8_i8_quant_bf16's rule) */
void orc_i8_quant_bf16(const uint16_t *W, int rows, int K, int8_t *Wo, float *So);
/* FP8 lane-chunk format: E4M3 decode / encode of the reference's packer and the pack itself */
float   orc_f8_decode(uint8_t b);
uint8_t orc_f8_encode(float v);
void    orc_fp8_pack_expert(const uint8_t *W, const uint8_t *S, float s2, int rows, int in, uint8_t *w8, float *sc);
/* dense INT8 x X8 GEMV, hyper-connection norm / combine, stream inject */
void orc_i8_gemv(const int8_t *W, const float *s, int rows, int K, const int8_t *xq, const float *xs, int act, double *y);
void orc_hc_norm(const float *R, const uint16_t *w, int H, double *normed);
void orc_hc_combine(const float *hcy, const float *normed, int H, double *mixed);
void orc_stream_inject(float *R, const float *y, const float *inj, int H);
/* bf16 shared expert, M rows of fp32 x [M][H]: eg/eu [M][I], g1 [M], ed [M][H] (fp64) and
   y [M][H] (fp64, in/out: y += sigmoid(g1) * ed) */
void orc_shexp_bf16(const uint16_t *gate, const uint16_t *up, const uint16_t *down, const uint16_t *gate_inp,
                    const float *x, int M, int H, int I, double *eg, double *eu, double *g1, double *ed, double *y);

/* ---- X8 activation quantizer (reference's lossy activation mode) ---- */
void orc_x8_quant(const float *v, int n, int8_t *q, float *s);

/* ---- four-card combine of fp32 partials ---- */
void orc_m8_reduce4(float *y, const float *y0, const float *y1, const float *y2, const float *y3, long n);

/* ---- routing inversion ---- */
int orc_csr_build(const int *sel, const float *wt, int T, int K, int E,
                  int *exp_ids, int *exp_ptr, int *pair_tok, int *pair_k, float *pair_wt,
                  int *n_pairs);

/* ---- whole MoE layer from the generator (fp64) ----
   fmt: 0 = INT8 routed experts, 1 = NVFP4 routed experts (shared stays INT8).
   gated: 1 = y += sigmoid(<g,x>) * shared(x), 0 = y += shared(x).
   Returns 0 on success. */
typedef struct {
    int H, I, E, K;
    int fmt, gated, renorm, use_bias;
    uint32_t seed, layer, x_layer;   /* x_layer: generator layer id of the input rows */
    int x_row0;                      /* first generated input row */
} orc_layer_cfg;
int orc_moe_layer(const orc_layer_cfg *cfg, int M, uint16_t *x_out, float *logits,
                  int *sel, double *w64, double *y64, uint16_t *ybf16);

/* ---- CPU baseline (timed, fp32 accumulate, OpenMP) ----
   A full resident INT8 layer on the host: router [E][H] fp32, per-expert
   code/scale arrays laid out [E+1] (index E = shared expert). */
typedef struct {
    const float *router;   /* [E][H] */
    const int8_t *qg, *qu, *qd;   /* [E+1][I][H], [E+1][I][H], [E+1][H][I] */
    const float *sg, *su, *sd;    /* [E+1][I], [E+1][I], [E+1][H] */
    const float *shgate;          /* [H] */
} orc_host_layer;
void orc_cpu_moe_layer_fast(const orc_host_layer *L, int H, int I, int E, int K,
                            const uint16_t *x, int M, float *y, int nthreads);
#ifdef __cplusplus
}
#endif
#endif
