/*
 * oracle.c -- CPU restatement of KuDNN's Linear/GEMM + post-op path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only
 * as the checker (or, for the CPU baseline, as the timed port of the reference's portable loops). The
 * product (libkudnn_hip.so, libkudnn.so) never links or calls it.
 *
 * It composes the reference's stages literally, on host arrays, with the reference's storage dtype
 * between stages:
 *   oracle_gemm        GEMMWrapper per dtype combination (src/dnn/src/kudnn_gemm.cpp:151-241) inside the
 *                      broadcast batch loop of BatchedExtendedGemm (:767-807), bias as in AddBias (:65-149)
 *   oracle_activation  the vml FWD kernels: RELU (kernels/vml/relu/relu.c:14-49, 225-260),
 *                      SWISH (swish/vml_sve_la_swishf.c:31-47, vml_sve_la_sigmoid.h:25-47),
 *                      GELU_TANH (gelu_tanh/vml_sve_la_gelu_tanh.h:22-39), GELU_ERF (gelu_erf/vml_sve_la_gelu_erf.h:20-28),
 *                      and the other 18 kinds of the forward table (kudnn_eltwise.cpp:333-400), each citing its
 *                      kernel source in oracle_act_f32; f32 math, bf16 results stored by the kind's rule
 *                      (truncation vml_sve_base.h:111-118, overflow-to-Inf first :97-109, or RNE for ELU_DST)
 *   oracle_res_add     AddOps (src/dnn/src/kudnn_linear_res.cpp:57-122): flat element-wise over
 *                      linearRes's size, f32 math, RNE back to bf16
 *   oracle_binary      the element-wise stage of the post-op chain (ADD/EXT as AddOps; MUL element-wise)
 *
 * Deliberate restatement choices:
 *   - GEMM sums are accumulated in double and rounded once to f32 (KML's f32 summation order is closed
 *     and not restatable); fp32 parity is then judged against this correctly-rounded value.
 *   - cblas_bgemm (bf16 C without bias) has KML-internal rounding; it is restated as RNE of the f32 value.
 *   - bias is indexed through its own strides (the reference indexes a full [M,N] bias with C's leading
 *     dimension, which is the same thing whenever bias and C share a layout).
 *   - RES_EXT computes fmaf(res, gamma, c), the contraction GCC applies to `c + res * gamma` on aarch64.
 *
 * Pinning (tests/test_oracle.py): bf16 bit patterns, closed forms and special values of the activations,
 * integer-valued GEMMs that are exact in f32 whatever the order, numpy float64 matmuls, and the
 * reference gtest's own naive oracle (linear_activation_gtest.cpp:24-88) restated in numpy.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "oracle.h"

#define O_F32 1
#define O_F16 2
#define O_BF16 3
#define O_S32 4
#define O_S8 5
#define O_U8 6

#define O_ACT_NONE 0
#define O_ACT_ABS 1
#define O_ACT_EXP 2
#define O_ACT_LINEAR 3
#define O_ACT_LOG 4
#define O_ACT_RELU 5
#define O_ACT_ROUND 6
#define O_ACT_SQRT 7
#define O_ACT_SQUARE 8
#define O_ACT_TANH 9
#define O_ACT_SIGMOID 10
#define O_ACT_POW 11
#define O_ACT_CLIP 12
#define O_ACT_CLIP_V2 13
#define O_ACT_HARDSIGMOID 14
#define O_ACT_HARDSWISH 15
#define O_ACT_ELU 19
#define O_ACT_GELU_TANH 20
#define O_ACT_ELU_DST 22
#define O_ACT_SWISH 25
#define O_ACT_SRELU 26
#define O_ACT_GELU_ERF 27
#define O_ACT_MISH 28

#define O_RES_EXT 0
#define O_RES_MUL 1
#define O_RES_IDENTIAL 2

#define O_BIN_NONE 0
#define O_BIN_ADD 1
#define O_BIN_EXT 2
#define O_BIN_MUL 3


/* ------------------------------------------------------------------------------------------------ */
/* element conversions                                                                              */

static uint32_t f2u(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float u2f(uint32_t u)
{
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Service::ConvertFp32ToBf16 / vcvth_bf16_f32: BFCVT, round to nearest even (service.cpp:48-67). */
uint16_t oracle_f32_to_bf16_rne(float f)
{
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return (uint16_t)((u >> 16) | 0x0040u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* SvCvtBF16F32FullX: keep the top half of each f32 (vml_sve_base.h:111-118). */
uint16_t oracle_f32_to_bf16_trunc(float f) { return (uint16_t)(f2u(f) >> 16); }

/* SvF32CvtBf16InfSpecial then truncation (vml_sve_base.h:97-109), used by RELU's bf16 kernel. */
uint16_t oracle_f32_to_bf16_trunc_inf(float f)
{
    uint32_t u = f2u(f);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f7f8000u && a < 0x7f800000u) {
        u = (u & 0x80000000u) | 0x7f800000u;
    }
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE binary16 <-> binary32, round to nearest even (implicit __fp16 conversions). */
float oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) {
            return u2f(sign);
        }
        /* subnormal: value = man * 2^-24 */
        float v = (float)man * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    if (exp == 31) {
        return u2f(sign | 0x7f800000u | (man << 13));
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16_rne(float f)
{
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) {
        return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    }
    if (a >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a < 0x38800000u) { /* below the smallest normal 2^-14: subnormal or zero */
        float v = u2f(a) * 16777216.0f; /* in units of 2^-24 */
        float r = nearbyintf(v);        /* default rounding mode: nearest even */
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t e = (a >> 23) - 112u;
    uint32_t m = a & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h += 1u;
    }
    return (uint16_t)(sign | h);
}

static float ld(const void *p, int dt, int64_t i)
{
    switch (dt) {
        case O_F32: return ((const float *)p)[i];
        case O_BF16: return oracle_bf16_to_f32(((const uint16_t *)p)[i]);
        case O_F16: return oracle_f16_to_f32(((const uint16_t *)p)[i]);
        case O_S8: return (float)((const int8_t *)p)[i];
        case O_U8: return (float)((const uint8_t *)p)[i];
        case O_S32: return (float)((const int32_t *)p)[i];
        default: return 0.0f;
    }
}

/* Integer elements exactly (8-bit and 32-bit types). */
static int64_t ld_int(const void *p, int dt, int64_t i)
{
    switch (dt) {
        case O_S8: return ((const int8_t *)p)[i];
        case O_U8: return ((const uint8_t *)p)[i];
        case O_S32: return ((const int32_t *)p)[i];
        default: return 0;
    }
}

/* ConvertFp32ToS32 / ToS8 / ToU8 (src/dnn/src/service.cpp:77-115): below the type's minimum -> minimum, above its
 * maximum -> maximum, else static_cast of nearbyintf (round half to even in the default rounding mode). The reference
 * leaves two inputs to the hardware's conversion, undefined in C++: NaN, and for s32 +2^31 (equal to
 * (float)INT32_MAX, so not above it). They are restated as aarch64's saturating fcvtzs / fcvtzu give them, the target
 * the reference is built for: NaN -> 0, +2^31 -> INT32_MAX. */
int64_t oracle_f32_to_int_sat(float v, int dt)
{
    const double lo = dt == O_S32 ? -2147483648.0 : (dt == O_S8 ? -128.0 : 0.0);
    const double hi = dt == O_S32 ? 2147483647.0 : (dt == O_S8 ? 127.0 : 255.0);
    if (isnan(v)) {
        return 0;
    }
    if ((double)v < lo) {
        return (int64_t)lo;
    }
    if ((double)v > hi) {
        return (int64_t)hi;
    }
    return (int64_t)nearbyintf(v);
}

/* Stores with RNE (the conversion the reference applies when it writes a typed buffer); integer types through
 * oracle_f32_to_int_sat. */
static void st(void *p, int dt, int64_t i, float v)
{
    switch (dt) {
        case O_F32: ((float *)p)[i] = v; break;
        case O_BF16: ((uint16_t *)p)[i] = oracle_f32_to_bf16_rne(v); break;
        case O_F16: ((uint16_t *)p)[i] = oracle_f32_to_f16_rne(v); break;
        case O_S32: ((int32_t *)p)[i] = (int32_t)oracle_f32_to_int_sat(v, dt); break;
        case O_S8: ((int8_t *)p)[i] = (int8_t)oracle_f32_to_int_sat(v, dt); break;
        case O_U8: ((uint8_t *)p)[i] = (uint8_t)oracle_f32_to_int_sat(v, dt); break;
        default: break;
    }
}

static int64_t total(const otensor *t)
{
    int64_t n = 1;
    if (t->ndims == 0) {
        return 0;
    }
    for (int i = 0; i < t->ndims; ++i) {
        n *= t->dims[i];
    }
    return n;
}

/* ------------------------------------------------------------------------------------------------ */
/* activations (vml FWD kernels, f32 math)                                                          */

/* RELU: lanes with x <= 0 are multiplied by alpha, others pass through (relu.c:14-25). */
static float act_relu(float x, float alpha) { return (x <= 0.0f) ? x * alpha : x; }

/* SWISH: x * 1/(1 + e^t) with t = -alpha*x; t > 87 gives 0, t < -87 gives 1 (vml_sve_la_sigmoid.h:37-47). */
static float act_swish(float x, float alpha)
{
    float t = -alpha * x;
    float s;
    if (t > 87.0f) {
        s = 0.0f;
    } else if (t < -87.0f) {
        s = 1.0f;
    } else {
        s = 1.0f / (1.0f + expf(t));
    }
    return x * s;
}

/* GELU_TANH: 0.5*x*(1 + tanh(sqrt(2/pi)*x*(1 + 0.044715*x^2))) (vml_sve_la_gelu_tanh.h:22-39). */
static float act_gelu_tanh(float x)
{
    const float c0 = 0.7978845608028654f; /* sqrt(2/pi), 0x1.988454p-1 */
    const float c1 = 0.044715f;           /* 0x1.6e4e26p-5 */
    float y = (1.0f + c1 * x * x) * x * c0;
    return (1.0f + tanhf(y)) * 0.5f * x;
}

/* GELU_ERF: s + s*erf(x/sqrt(2)) with s = x/2 (vml_sve_la_gelu_erf.h:20-28). */
static float act_gelu_erf(float x)
{
    float s = x * 0.5f;
    return s + s * erff(x * 0.70710678118654752f);
}

/* SRELU: ln(1 + e^(alpha*x)) / alpha; alpha*x at or above expf's upper bound (0x1.62e43p6) returns x, and alpha*x
 * is clamped below at expf's lower bound (-0x1.5d58ap6) (soft_relu/vml_sve_la_softrelu.h:31-86). */
static float act_srelu(float x, float alpha)
{
    const float ax = alpha * x;
    if (ax >= 0x1.62e43p6f) {
        return x;
    }
    return log1pf(expf(ax > -0x1.5d58ap6f ? ax : -0x1.5d58ap6f)) / alpha;
}

/* MISH: x * ((e^x + 1)^2 - 1) / ((e^x + 1)^2 + 1), the exponent capped at 0x1.62e42ep5 (mish/vml_sve_la_mish.h:21-35). */
static float act_mish(float x)
{
    const float e1 = expf(x < 0x1.62e42ep5f ? x : 0x1.62e42ep5f) + 1.0f;
    const float e2 = e1 * e1;
    return x * ((e2 - 1.0f) / (e2 + 1.0f));
}

/* Every kind of the forward table (src/dnn/src/kudnn_eltwise.cpp:333-400), f32 math of the kernels' f32 sources. */
float oracle_act_f32(int kind, float x, float alpha, float beta)
{
    switch (kind) {
        case O_ACT_RELU: return act_relu(x, alpha);
        case O_ACT_SWISH: return act_swish(x, alpha);
        case O_ACT_GELU_TANH: return act_gelu_tanh(x);
        case O_ACT_GELU_ERF: return act_gelu_erf(x);
        case O_ACT_ABS: return fabsf(x);                          /* abs/vml_sve_la_absf.c */
        case O_ACT_EXP: return expf(x);                           /* exp/vml_sve_la_expf.c */
        case O_ACT_LINEAR: return fmaf(alpha, x, beta);           /* linear.c: svmad(alpha, x, beta) */
        case O_ACT_LOG: return logf(x);                           /* log/vml_sve_la_lnf.c */
        case O_ACT_ROUND: return nearbyintf(x);                   /* round/vml_sve_la_nearbyintf.c (svrinti) */
        case O_ACT_SQRT: return sqrtf(x);                         /* sqrt/vml_sve_la_sqrtf.c */
        case O_ACT_SQUARE: return x * x;                          /* sqr/vml_sve_la_sqrf.c */
        case O_ACT_TANH: return tanhf(x);                         /* tanh/vml_sve_la_tanhf.c */
        case O_ACT_SIGMOID: return 1.0f / (1.0f + expf(-x));      /* logistic/sigmoid.c:71-88 */
        case O_ACT_POW: return powf(x, beta) * alpha;             /* pow/vml_sve_powx_calculations.h:506-515 */
        case O_ACT_CLIP:                                          /* clip/clipf.c: <= alpha, then > beta */
            return x <= alpha ? alpha : (x > beta ? beta : x);
        case O_ACT_CLIP_V2:                                       /* clipv2/clipv2f.c: <= alpha, then >= beta */
            return x <= alpha ? alpha : (x >= beta ? beta : x);
        case O_ACT_HARDSIGMOID:                                   /* hardsigmoid: maxnm(minnm(x*a + b, 1), 0) */
            return fmaxf(fminf(fmaf(x, alpha, beta), 1.0f), 0.0f);
        case O_ACT_HARDSWISH:                                     /* hardswish: x * max(0, min(1, a*x + b)) */
            return x * fmaxf(fminf(fmaf(alpha, x, beta), 1.0f), 0.0f);
        case O_ACT_ELU:                                           /* elu/vml_sve_la_eluf.c: nmls(a, e^x, a) */
            return x > 0.0f ? x : fmaf(expf(x), alpha, -alpha);
        case O_ACT_ELU_DST: return x > 0.0f ? x : alpha * expm1f(x);  /* elu/eludstf.c */
        case O_ACT_SRELU: return act_srelu(x, alpha);
        case O_ACT_MISH: return act_mish(x);
        default: return x;
    }
}

/* bf16 store of an activation's result: RELU, CLIP, CLIP_V2, ELU, LINEAR, POW, ROUND and SRELU send finite values
 * at or above the largest bf16 to +-Inf first (SvF32CvtBf16InfSpecial in their FWD bf16 kernels); ELU_DST rounds
 * to nearest even (elu/eludstbf16.c, SveCvtU32ToU16); the others truncate (SvCvtBF16F32FullX). */
static uint16_t act_store_bf16(int kind, float y)
{
    switch (kind) {
        case O_ACT_RELU: case O_ACT_CLIP: case O_ACT_CLIP_V2: case O_ACT_ELU: case O_ACT_LINEAR: case O_ACT_POW:
        case O_ACT_ROUND: case O_ACT_SRELU:
            return oracle_f32_to_bf16_trunc_inf(y);
        case O_ACT_ELU_DST:
            return oracle_f32_to_bf16_rne(y);
        default:
            return oracle_f32_to_bf16_trunc(y);
    }
}

/* In-place activation over the tensor's elements (ActivationLayerFWD run from a copy of C back into C,
 * kudnn_linear_activationlayer.cpp:40-56). Element-wise, so the memory walk order does not matter. */
int oracle_activation(const otensor *t, void *p, int kind, float alpha, float beta)
{
    const int64_t n = total(t);
    /* dense tensor: every element sits in [0, n) */
    for (int64_t i = 0; i < n; ++i) {
        float x = ld(p, t->dtype, i);
        float y = oracle_act_f32(kind, x, alpha, beta);
        if (t->dtype == O_BF16) {
            ((uint16_t *)p)[i] = act_store_bf16(kind, y);
        } else {
            st(p, t->dtype, i, y);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* GEMM stage                                                                                      */


static void batch_slots(const otensor *t, int64_t dims[3], int64_t bs[3])
{
    int nb = t->ndims - 2;
    for (int s = 0; s < 3; ++s) {
        dims[s] = 1;
        bs[s] = 0;
    }
    for (int d = 0; d < nb; ++d) {
        dims[3 - nb + d] = t->dims[d];
        bs[3 - nb + d] = t->strides[d];
    }
}

/* Rounds alpha/beta to bf16 the way GEMMWrapper<bf16,bf16,bf16,float> does for cblas_bgemm (:222-224). */
static float bf16_round_scalar(float f) { return oracle_bf16_to_f32(oracle_f32_to_bf16_rne(f)); }

/* C = alpha * A x B + beta * C (+ bias), per the dtype rules of GEMMWrapper / ChooseImpl:
 *  - every sum is formed in f32 (double here, rounded once);
 *  - bf16 C with bias: f32 temp = f32(C), temp = alpha*AB + beta*temp, temp += bias, RNE (:208-221);
 *  - bf16 C without bias: cblas_bgemm with bf16 alpha/beta, RNE (:222-226);
 *  - f32 / f16 C: value rounded once into C's type after bias (all-f32 fallback :672-705);
 *  - s8 / u8 x s8 / u8 -> s32 with an s32 or s8 bias or none (cblas_gemm_s8s8s32 and its u8 forms, :243-324; an s8
 *    bias is ChooseImpl's wider-type match, :655-671): exact integer sum plus the bias (a row / column vector is
 *    KML's C offset, a full [M, N] bias is added afterwards: the same sum), two's-complement wrap into int32; only
 *    alpha 1 and beta 0 are restated (the scaling of an int32 result by float alpha / beta is KML-internal);
 *  - any other integer output or bias: the all-f32 fallback (:673-705): operands, C and bias read as f32, the f32
 *    value converted by ConvertFp32ToS32 / ToS8 / ToU8 (oracle_f32_to_int_sat). */
static int oracle_gemm_s8(const ogemm *g);

static int is_int8(int dt) { return dt == O_S8 || dt == O_U8; }

/* The dtype ChooseImpl sees: f32 for a tensor that BatchedExtendedGemm reordered (:722-765). A reordered integer dst
 * comes back from f32 through ReorderLayer's clamp and nearbyint (vector_convert.hpp:153-179), which gives the same
 * values as ConvertFp32ToS32 / ToS8 / ToU8, so the final store is the same either way. */
static int seen_dt(const ogemm *g, const otensor *t, int bit) { return (g->reordered & bit) ? O_F32 : t->dtype; }

int oracle_gemm(const ogemm *g)
{
    const int hasBias0 = g->bias.ndims != 0 && total(&g->bias) != 0;
    const int ea = seen_dt(g, &g->a, O_REORDERED_A), eb = seen_dt(g, &g->b, O_REORDERED_B);
    const int ec = seen_dt(g, &g->c, O_REORDERED_C);
    /* without a bias ChooseImpl sees dst's own dtype for it (the bias-less TensorInfo of kudnn_gemm.hpp) */
    const int biasDt = hasBias0 ? seen_dt(g, &g->bias, O_REORDERED_BIAS) : g->c.dtype;
    if (is_int8(ea) && is_int8(eb) && ec == O_S32 && (biasDt == O_S32 || biasDt == O_S8)) {
        return oracle_gemm_s8(g);
    }
    const int nd = g->a.ndims;
    if (nd < 2 || g->b.ndims != nd || g->c.ndims != nd) {
        return -1;
    }
    const int64_t M = g->a.dims[nd - 2], K = g->a.dims[nd - 1], N = g->b.dims[nd - 1];
    const int hasBias = g->bias.ndims != 0 && total(&g->bias) != 0;
    float alpha = g->alpha, beta = g->beta;
    if (!hasBias && ec == O_BF16 && ea == O_BF16 && eb == O_BF16) {
        alpha = bf16_round_scalar(alpha);
        beta = bf16_round_scalar(beta);
    }
    int64_t ad[3], as[3], bd[3], bs_[3], cd[3], cs[3], xd[3], xs[3] = {0, 0, 0};
    batch_slots(&g->a, ad, as);
    batch_slots(&g->b, bd, bs_);
    batch_slots(&g->c, cd, cs);
    if (hasBias) {
        batch_slots(&g->bias, xd, xs);
    }
    int64_t L[3];
    for (int s = 0; s < 3; ++s) {
        L[s] = ad[s] > bd[s] ? ad[s] : bd[s];
    }
    const int64_t a_sm = g->a.strides[nd - 2], a_sk = g->a.strides[nd - 1];
    const int64_t b_sk = g->b.strides[nd - 2], b_sn = g->b.strides[nd - 1];
    const int64_t c_sm = g->c.strides[nd - 2], c_sn = g->c.strides[nd - 1];
    const int64_t x_sm = hasBias ? g->bias.strides[nd - 2] : 0, x_sn = hasBias ? g->bias.strides[nd - 1] : 0;

    for (int64_t i0 = 0; i0 < L[0]; ++i0) {
        for (int64_t i1 = 0; i1 < L[1]; ++i1) {
            for (int64_t i2 = 0; i2 < L[2]; ++i2) {
                const int64_t ao = i0 * as[0] + i1 * as[1] + i2 * as[2];
                const int64_t bo = i0 * bs_[0] + i1 * bs_[1] + i2 * bs_[2];
                const int64_t co = i0 * cs[0] + i1 * cs[1] + i2 * cs[2];
                const int64_t xo = i0 * xs[0] + i1 * xs[1] + i2 * xs[2];
                /* B of this batch widened once to f32, [K][N] */
                float *bf = (float *)malloc((size_t)(K * N) * sizeof(float));
                if (bf == NULL) {
                    return -2;
                }
#pragma omp parallel for schedule(static)
                for (int64_t k = 0; k < K; ++k) {
                    for (int64_t n = 0; n < N; ++n) {
                        bf[k * N + n] = ld(g->pb, g->b.dtype, bo + k * b_sk + n * b_sn);
                    }
                }
#pragma omp parallel for schedule(dynamic, 1)
                for (int64_t m = 0; m < M; ++m) {
                    double *acc = (double *)calloc((size_t)N, sizeof(double));
                    for (int64_t k = 0; k < K; ++k) {
                        const double av = (double)ld(g->pa, g->a.dtype, ao + m * a_sm + k * a_sk);
                        if (av == 0.0) {
                            continue;
                        }
                        const float *brow = bf + k * N;
                        for (int64_t n = 0; n < N; ++n) {
                            acc[n] += av * (double)brow[n];
                        }
                    }
                    for (int64_t n = 0; n < N; ++n) {
                        const int64_t ci = co + m * c_sm + n * c_sn;
                        float v = (float)((double)alpha * acc[n]);
                        if (beta != 0.0f) {
                            v = v + beta * ld(g->pc, g->c.dtype, ci);
                        }
                        if (hasBias) {
                            v = v + ld(g->pbias, g->bias.dtype, xo + m * x_sm + n * x_sn);
                        }
                        st(g->pc, g->c.dtype, ci, v);
                    }
                    free(acc);
                }
                free(bf);
            }
        }
    }
    return 0;
}

/* The integer GEMMs into s32 of the registry (src/dnn/src/kudnn_gemm.cpp:243-324): cblas_gemm_s8s8s32, s8u8s32,
 * u8s8s32 and u8u8s32, all called with zero operand offsets, so the result is the exact integer sum (plus the s32
 * bias), wrapped to int32. alpha = 1 and beta = 0 only. */
static int oracle_gemm_s8(const ogemm *g)
{
    const int nd = g->a.ndims;
    const int ai = g->a.dtype == O_S8 || g->a.dtype == O_U8, bi = g->b.dtype == O_S8 || g->b.dtype == O_U8;
    if (!ai || !bi || g->alpha != 1.0f || g->beta != 0.0f) {
        return -3;
    }
    const int64_t M = g->a.dims[nd - 2], K = g->a.dims[nd - 1], N = g->b.dims[nd - 1];
    const int hasBias = g->bias.ndims != 0 && total(&g->bias) != 0;
    if (hasBias && g->bias.dtype != O_S32 && g->bias.dtype != O_S8) {
        return -3;
    }
    int64_t ad[3], as[3], bd[3], bs_[3], cd[3], cs[3], xd[3], xs[3] = {0, 0, 0};
    batch_slots(&g->a, ad, as);
    batch_slots(&g->b, bd, bs_);
    batch_slots(&g->c, cd, cs);
    if (hasBias) {
        batch_slots(&g->bias, xd, xs);
    }
    int64_t L[3];
    for (int s = 0; s < 3; ++s) {
        L[s] = ad[s] > bd[s] ? ad[s] : bd[s];
    }
    const int64_t a_sm = g->a.strides[nd - 2], a_sk = g->a.strides[nd - 1];
    const int64_t b_sk = g->b.strides[nd - 2], b_sn = g->b.strides[nd - 1];
    const int64_t c_sm = g->c.strides[nd - 2], c_sn = g->c.strides[nd - 1];
    const int64_t x_sm = hasBias ? g->bias.strides[nd - 2] : 0, x_sn = hasBias ? g->bias.strides[nd - 1] : 0;
    for (int64_t i0 = 0; i0 < L[0]; ++i0) {
        for (int64_t i1 = 0; i1 < L[1]; ++i1) {
            for (int64_t i2 = 0; i2 < L[2]; ++i2) {
                const int64_t ao = i0 * as[0] + i1 * as[1] + i2 * as[2];
                const int64_t bo = i0 * bs_[0] + i1 * bs_[1] + i2 * bs_[2];
                const int64_t co = i0 * cs[0] + i1 * cs[1] + i2 * cs[2];
                const int64_t xo = i0 * xs[0] + i1 * xs[1] + i2 * xs[2];
#pragma omp parallel for schedule(dynamic, 1)
                for (int64_t m = 0; m < M; ++m) {
                    for (int64_t n = 0; n < N; ++n) {
                        int64_t acc = 0;
                        for (int64_t k = 0; k < K; ++k) {
                            acc += ld_int(g->pa, g->a.dtype, ao + m * a_sm + k * a_sk) *
                                   ld_int(g->pb, g->b.dtype, bo + k * b_sk + n * b_sn);
                        }
                        if (hasBias) {
                            acc += ld_int(g->pbias, g->bias.dtype, xo + m * x_sm + n * x_sn);
                        }
                        ((int32_t *)g->pc)[co + m * c_sm + n * c_sn] = (int32_t)(uint32_t)(uint64_t)acc;
                    }
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* residual stage                                                                                   */

/* AddOps over flat arrays of linearRes's size (kudnn_linear_res.cpp:57-122). All three tensors share one
 * dtype, as the reference's dispatch on linearRes's type assumes (:192-200). */
int oracle_res_add(int dtype, int64_t size, const void *c, const void *res, void *out, int kind, float gamma)
{
    for (int64_t i = 0; i < size; ++i) {
        float cv = ld(c, dtype, i), rv = ld(res, dtype, i);
        float v = (kind == O_RES_IDENTIAL) ? cv + rv : fmaf(rv, gamma, cv);
        st(out, dtype, i, v);
    }
    return 0;
}

/* Binary stage of the post-op chain on logical (m, n) indices of same-shaped tensors y and src. */
int oracle_binary(const otensor *y, void *py, const otensor *src, const void *psrc, int kind, float gamma)
{
    const int nd = y->ndims;
    const int64_t n = total(y);
    for (int64_t lin = 0; lin < n; ++lin) {
        int64_t rem = lin, yo = 0, so = 0;
        for (int d = nd - 1; d >= 0; --d) {
            int64_t idx = rem % y->dims[d];
            rem /= y->dims[d];
            yo += idx * y->strides[d];
            so += idx * src->strides[d];
        }
        float v = ld(py, y->dtype, yo), s = ld(psrc, src->dtype, so);
        float r;
        if (kind == O_BIN_ADD) {
            r = v + s;
        } else if (kind == O_BIN_EXT) {
            r = fmaf(s, gamma, v);
        } else {
            r = v * s;
        }
        st(py, y->dtype, yo, r);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* composed operators                                                                              */

/* LinearActivationLayerFWD::Run: GEMM (alpha 1, beta 0) into C, then the activation in place
 * (kudnn_linear_activationlayer.cpp:40-56). The layer's activation member is built as
 * activationlayerfwd(cInfo, cInfo, kind, alpha) (:33): the layer's beta is validated but never reaches the activation,
 * which runs with its default second parameter 0 (kudnn_eltwise.hpp:68-69). */
int oracle_linear_act(const ogemm *g, int kind, float act_alpha)
{
    ogemm h = *g;
    h.alpha = 1.0f;
    h.beta = 0.0f;
    if (oracle_gemm(&h) != 0) {
        return -1;
    }
    return oracle_activation(&g->c, g->pc, kind, act_alpha, 0.0f);
}

/* LinearResFWD::Run (kudnn_linear_res.cpp:184-202): GEMM into C, then RES_MUL = C x res (second GEMM) or
 * AddOps over linearRes's size. */
int oracle_linear_res(const ogemm *g, const otensor *res, const void *pres, const otensor *lr, void *plr, int kind,
                      float gamma)
{
    ogemm h = *g;
    h.alpha = 1.0f;
    h.beta = 0.0f;
    if (oracle_gemm(&h) != 0) {
        return -1;
    }
    if (kind == O_RES_MUL) {
        ogemm m2;
        memset(&m2, 0, sizeof(m2));
        m2.a = g->c;
        m2.pa = g->pc;
        m2.b = *res;
        m2.pb = pres;
        m2.c = *lr;
        m2.pc = plr;
        m2.alpha = 1.0f;
        m2.beta = 0.0f;
        return oracle_gemm(&m2);
    }
    return oracle_res_add(lr->dtype, total(lr), g->pc, pres, plr, kind, gamma);
}

/* Post-op chain: GEMM stage, optional activation stage, optional binary stage, each stored in Y's dtype. */
int oracle_linear_postops(const ogemm *g, int act_kind, float act_alpha, float act_beta, int bin_kind,
                          const otensor *src, const void *psrc, float gamma)
{
    ogemm h = *g;
    h.alpha = 1.0f;
    h.beta = 0.0f;
    if (oracle_gemm(&h) != 0) {
        return -1;
    }
    if (act_kind != O_ACT_NONE) {
        oracle_activation(&g->c, g->pc, act_kind, act_alpha, act_beta);
    }
    if (bin_kind != O_BIN_NONE) {
        oracle_binary(&g->c, g->pc, src, psrc, bin_kind, gamma);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* seeded inputs: SplitMix64 -> uniform / Box-Muller normal, bf16 by RNE of the f32 sample            */

static uint64_t splitmix64(uint64_t *s)
{
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* uniform in [0,1) with 53 random bits */
static double u01(uint64_t *s) { return (double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0); }

/* Fills n values: dist 0 = uniform[lo, hi), dist 1 = normal(mean=lo, std=hi). dtype O_F32 / O_BF16 / O_F16. */
int oracle_fill(void *p, int dtype, int64_t n, uint64_t seed, int dist, double lo, double hi)
{
    uint64_t s = seed;
    for (int64_t i = 0; i < n; ++i) {
        double v;
        if (dist == 0) {
            v = lo + (hi - lo) * u01(&s);
        } else {
            double u1 = u01(&s), u2 = u01(&s);
            if (u1 < 1e-300) {
                u1 = 1e-300;
            }
            v = lo + hi * sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        }
        st(p, dtype, i, (float)v);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* CPU baseline: the reference tests' portable naive loop (linear_activation_gtest.cpp:66-88, f32
 * accumulation as in linear_res_gtest.cpp:123-160) for Y[M][N] = act(X[M][K] . W[N][K]^T + bias[N]) with an
 * optional residual add, parallelised over output rows as MatmulRef does (matmul_gtest.cpp:112). Used only
 * as the reported CPU baseline. */
int oracle_cpu_baseline(int dtype, int64_t M, int64_t N, int64_t K, const void *X, const void *W, const void *bias,
                        const void *R, int r_mul, void *Y, int act, float act_alpha, int threads)
{
#ifdef _OPENMP
    if (threads > 0) {
        omp_set_num_threads(threads);
    }
#else
    (void)threads;
#endif
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; ++i) {
        float *xr = (float *)malloc((size_t)K * sizeof(float));
        for (int64_t l = 0; l < K; ++l) {
            xr[l] = ld(X, dtype, i * K + l);
        }
        for (int64_t j = 0; j < N; ++j) {
            float sum = 0.0f;
            if (dtype == O_F32) {
                const float *wr = (const float *)W + j * K;
                for (int64_t l = 0; l < K; ++l) {
                    sum += xr[l] * wr[l];
                }
            } else {
                const uint16_t *wr = (const uint16_t *)W + j * K;
                for (int64_t l = 0; l < K; ++l) {
                    sum += xr[l] * u2f((uint32_t)wr[l] << 16);
                }
            }
            float v = sum + (bias ? ld(bias, dtype, j) : 0.0f);
            if (dtype == O_BF16) {
                v = oracle_bf16_to_f32(oracle_f32_to_bf16_rne(v));
            }
            if (act != O_ACT_NONE) {
                v = oracle_act_f32(act, v, act_alpha, 0.0f);
                if (dtype == O_BF16) {
                    v = oracle_bf16_to_f32(oracle_f32_to_bf16_trunc(v));
                }
            }
            if (R) {
                v = r_mul ? v * ld(R, dtype, i * N + j) : v + ld(R, dtype, i * N + j);
            }
            st(Y, dtype, i * N + j, v);
        }
        free(xr);
    }
    return 0;
}

/* The compiler flags this library was built with (the Makefile passes them), reported beside the CPU baseline. */
#ifndef ORACLE_BUILD_FLAGS
#define ORACLE_BUILD_FLAGS "unknown"
#endif
const char *oracle_build_flags(void) { return ORACLE_BUILD_FLAGS; }

int oracle_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
