// Kernel argument structures shared by the host planner (capi.cpp) and the HIP kernels.
// Plain structs passed by value as kernel arguments.
#ifndef KUDNN_PLAN_TYPES_H
#define KUDNN_PLAN_TYPES_H

#include <stdint.h>

#include "../../include/kudnn_hip.h"

// Epilogue of one GEMM launch: y[m,n] = bin(act(round_c(alpha*acc + beta*c[m,n] + bias[m,n])), src[m,n]).
// All strides are in elements; *_bs are the batch strides for the three (right-aligned) batch dims.
struct EpiParams {
    float alpha;
    float beta;
    float act_alpha;
    float act_beta;   // second activation parameter (CLIP / CLIP_V2 upper bound, LINEAR / HARDSIGMOID / HARDSWISH offset,
                      // POW exponent)
    float gamma;
    int act;      // KUDNN_ACT_*, KUDNN_ACT_UNIMPLEMENTED = none
    int bin;      // KUDNN_BINARY_*
    int c_dt;     // dtype of C: rounding point of the GEMM stage and of the activation
    int bias_dt;
    int src_dt;
    int y_dt;
    int store_c;  // also store the GEMM-stage value to c (LinearResFWD writes C and linearRes)
    int fast4;    // 4-wide vector epilogue allowed (host-checked contiguity and alignment)
    int fast8;    // 8-wide vector epilogue allowed
    int acc_i32;  // the accumulators are int32 bit patterns (s8 MFMA): the exact integer epilogue
    void *c;              // C (read when beta != 0, written when store_c)
    const void *bias;     // nullptr = no bias
    const void *src;      // binary operand
    void *y;              // final output
    int64_t c_sm, c_sn, bias_sm, bias_sn, src_sm, src_sn, y_sm, y_sn;
    int64_t bdim[3];      // batch dims (right-aligned), product = number of batches in grid.y
    int64_t c_bs[3], bias_bs[3], src_bs[3], y_bs[3];
    // Integer GEMMs with a u8 operand run on the s8 MFMA with that operand shifted by -128; the terms the shift
    // removes come back here: y += corr_m[b * corr_m_bs + m] + corr_n[b * corr_n_bs + n] + corr_c (int32, wrapping;
    // b the linear batch index, a null vector adds nothing).
    const int32_t *corr_m;
    const int32_t *corr_n;
    int64_t corr_m_bs, corr_n_bs;
    int32_t corr_c;
};

// Operands of the MFMA / skinny kernels: A is [M][K] with row stride lda, B is [N][K] with row stride ldb,
// both contiguous along K, element type = the kernel's compute type (or, with b_kmajor, B is [K][N]).
struct GemmOperands {
    const void *a;
    const void *b;
    int64_t M, N, K;
    int64_t lda, ldb;
    int64_t a_bs[3], b_bs[3];  // batch strides (elements), same batch dims as EpiParams::bdim
    int b_kmajor;  // 1: B is stored [K][N] (N contiguous, row pitch ldb along k): the 16-bit ping-pong kernel and the
                   // 4-wave fp32 kernels read it
};

#endif  // KUDNN_PLAN_TYPES_H
