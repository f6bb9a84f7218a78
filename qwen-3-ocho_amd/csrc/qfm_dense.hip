// qfm_dense.hip -- load-time conversion of dense bf16 matrices to the INT8
// per-row form (Qf8I8Mat) that the shared expert kernels read.
//
// Rule (ocho/amd_server/qf8_dense_i8.hip:41-60): per row, s = absmax / 127
// (1 for an all-zero row), q = rint(w * (1 / s)) clamped to +-127, both
// divisions IEEE-rounded. One wave per row, four rows per block: the row is
// read twice (maximum, then codes) in 16-byte words, the maximum reduced
// across the wave with DPP, the codes written as 8-byte words.
#include "qfm_internal.h"
#include "qfm_dev.h"
#include "../../include/qf_store.h"

#include <cstring>

namespace qfm {

__global__ void __launch_bounds__(256)
k_quant_rows_bf16(const uint16_t *__restrict__ W, int rows, int K, int8_t *__restrict__ q, float *__restrict__ s) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;                                  // wave-uniform
    const uint4 *src = reinterpret_cast<const uint4 *>(W + (size_t)row * K);
    const int nw = K / 8;                                     // 16-byte words (8 values) per row
    float amax = 0.0f;
    for (int i = lane; i < nw; i += 64) {
        const uint4 v = src[i];
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++) amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(d[j])), fabsf(bf16_hi(d[j]))));
    }
    amax = group_max<64>(amax);
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    uint2 *dst = reinterpret_cast<uint2 *>(q + (size_t)row * K);
    for (int i = lane; i < nw; i += 64) {
        const uint4 v = src[i];
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
        uint32_t pk[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c0 = min(127, max(-127, (int)rintf(bf16_lo(d[j]) * inv)));
            const int c1 = min(127, max(-127, (int)rintf(bf16_hi(d[j]) * inv)));
            pk[j >> 1] |= (((uint32_t)c0 & 0xFFu) | (((uint32_t)c1 & 0xFFu) << 8)) << (16 * (j & 1));
        }
        dst[i] = make_uint2(pk[0], pk[1]);
    }
    if (lane == 0) s[row] = scale;
}

static int quant_args_ok(const void *W, int rows, int K, const Qf8I8Mat *m, const char *who) {
    if (!W || !m || rows < 1 || K < 16 || (K % 16)) {
        set_error(-1, "%s: bad arguments (rows %d, K %d; K must be a positive multiple of 16)", who, rows, K);
        return 0;
    }
    return 1;
}

static int alloc_mat(Qf8I8Mat *m, int rows, int K, const char *who) {
    std::memset(m, 0, sizeof *m);
    if (hipMalloc(reinterpret_cast<void **>(&m->w), (size_t)rows * K) != hipSuccess ||
        hipMalloc(reinterpret_cast<void **>(&m->s), (size_t)rows * sizeof(float)) != hipSuccess) {
        if (m->w) (void)hipFree(m->w);
        if (m->s) (void)hipFree(m->s);
        std::memset(m, 0, sizeof *m);
        set_error(-4, "%s: hipMalloc failed", who);
        return -1;
    }
    m->rows = rows;
    m->K = K;
    return 0;
}

int launch_quant_rows_bf16(const uint16_t *W, int rows, int K, int8_t *q, float *s, hipStream_t st) {
    hipLaunchKernelGGL(k_quant_rows_bf16, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, W, rows, K, q, s);
    return check_launch("k_quant_rows_bf16");
}

}  // namespace qfm

using namespace qfm;

extern "C" int qf8_i8_quant_bf16(const uint16_t *W, int rows, int K, Qf8I8Mat *m, hipStream_t s) {
    if (!quant_args_ok(W, rows, K, m, "qf8_i8_quant_bf16")) return -1;
    if (alloc_mat(m, rows, K, "qf8_i8_quant_bf16")) return -1;
    if (launch_quant_rows_bf16(W, rows, K, m->w, m->s, s)) {
        (void)hipFree(m->w);
        (void)hipFree(m->s);
        std::memset(m, 0, sizeof *m);
        return -1;
    }
    return 0;
}

extern "C" int qf8_i8_quant_bf16_host(const uint16_t *Whost, int rows, int K, Qf8I8Mat *m, hipStream_t s) {
    if (!quant_args_ok(Whost, rows, K, m, "qf8_i8_quant_bf16_host")) return -1;
    if (alloc_mat(m, rows, K, "qf8_i8_quant_bf16_host")) return -1;
    // bounded staging: at most 8 MiB of bf16 rows per round
    const int rb = (int)std::max<size_t>(4, std::min<size_t>((size_t)rows, (size_t(8) << 20) / ((size_t)K * 2)));
    uint16_t *stage = nullptr;
    if (hipMalloc(reinterpret_cast<void **>(&stage), (size_t)rb * K * 2) != hipSuccess) {
        set_error(-4, "qf8_i8_quant_bf16_host: staging hipMalloc failed");
        return -1;
    }
    int rc = 0;
    for (int r0 = 0; r0 < rows && !rc; r0 += rb) {
        const int nr = std::min(rb, rows - r0);
        if (hipMemcpyAsync(stage, Whost + (size_t)r0 * K, (size_t)nr * K * 2, hipMemcpyHostToDevice, s) != hipSuccess) {
            set_error(-3, "qf8_i8_quant_bf16_host: upload failed");
            rc = -1;
            break;
        }
        if (launch_quant_rows_bf16(stage, nr, K, m->w + (size_t)r0 * K, m->s + r0, s) ||
            hipStreamSynchronize(s) != hipSuccess) {
            set_error(-3, "qf8_i8_quant_bf16_host: conversion failed");
            rc = -1;
        }
    }
    (void)hipStreamSynchronize(s);
    (void)hipFree(stage);
    if (rc) {
        (void)hipFree(m->w);
        (void)hipFree(m->s);
        std::memset(m, 0, sizeof *m);
    }
    return rc;
}
