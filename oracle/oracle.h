/*
 * oracle.h -- declarations of the CPU oracle (oracle.c). TEST INFRASTRUCTURE ONLY: included by the oracle itself and
 * by the C++ API test; the product never includes it.
 */
#ifndef KUDNN_ORACLE_H
#define KUDNN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t ndims;
    int32_t dtype;
    int64_t dims[5];
    int64_t strides[5]; /* logical order, 0 for size-1 dims */
} otensor;

/* Bits of ogemm.reordered: the tensor has more than two dims and a layout other than the standard ABC.. order, so the
 * reference's BatchedExtendedGemm hands ChooseImpl an f32 copy of it (src/dnn/src/kudnn_gemm.cpp:722-765). */
#define O_REORDERED_A 1
#define O_REORDERED_B 2
#define O_REORDERED_C 4
#define O_REORDERED_BIAS 8

typedef struct {
    otensor a, b, c, bias; /* bias.ndims == 0: no bias */
    const void *pa, *pb, *pbias;
    void *pc;
    float alpha, beta;
    int32_t reordered; /* O_REORDERED_* bits */
} ogemm;

int oracle_gemm(const ogemm *g);
int oracle_linear_act(const ogemm *g, int kind, float act_alpha);
int oracle_linear_res(const ogemm *g, const otensor *res, const void *pres, const otensor *lr, void *plr, int kind,
                      float gamma);
int oracle_linear_postops(const ogemm *g, int act_kind, float act_alpha, float act_beta, int bin_kind,
                          const otensor *src, const void *psrc, float gamma);
int oracle_fill(void *p, int dtype, int64_t n, uint64_t seed, int dist, double lo, double hi);
int64_t oracle_f32_to_int_sat(float v, int dt);

#ifdef __cplusplus
}
#endif

#endif /* KUDNN_ORACLE_H */
