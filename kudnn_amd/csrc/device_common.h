// Device helpers shared by every kernel of the Linear/GEMM path: bf16/f16 rounding, the activation
// math, and the fused register epilogue (bias, activation, residual add/ext/mul, typed stores).
//
// The epilogue reproduces the rounding points of the reference's separate passes:
//   stage 0  GEMM result  -> rounded to C's dtype (RNE for bf16: Service::ConvertFp32ToBf16 after
//            cblas_sbgemm + AddBias, src/dnn/src/kudnn_gemm.cpp:215-221, src/dnn/src/service.cpp:48-67)
//   stage 1  activation   -> computed in f32 from the stored C, bf16 result TRUNCATED (top 16 bits;
//            SvCvtBF16F32FullX, src/dnn/src/kernels/vml/vml_sve_base.h:111-118), RELU first maps
//            |x| >= 0x7f7f8000 to +-Inf (SvF32CvtBf16InfSpecial, vml_sve_base.h:97-109, relu/relu.c:225-233)
//   stage 2  residual     -> f32 math on the stored operands, RNE to bf16
//            (AddOps, src/dnn/src/kudnn_linear_res.cpp:57-122)
#ifndef KUDNN_DEVICE_COMMON_H
#define KUDNN_DEVICE_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "plan_types.h"

namespace kudnn_dev {

// ---------------------------------------------------------------------------------------------------
// scalar conversions

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return u2f(static_cast<uint32_t>(h) << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even f32 -> bf16 by gfx950's conversion instruction (v_cvt_pk_bf16_f32). Over all 2^32 inputs it
// equals (u + 0x7fff + ((u >> 16) & 1)) >> 16 for non-NaN u, and (u >> 16) | 0x40 (quiet, top payload bits kept)
// for NaN: denormals are rounded, not flushed.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

// Two RNE conversions in one instruction: lo in bits 0-15, hi in bits 16-31.
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi)
{
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// a, b <- their RNE bf16 values, as f32.
__device__ __forceinline__ void round_bf16_pair(float &a, float &b)
{
    const uint32_t p = pack_bf16x2_rne(a, b);
    a = u2f(p << 16);
    b = u2f(p & 0xffff0000u);
}

// Truncating f32 -> bf16 (keep the top 16 bits).
__device__ __forceinline__ uint16_t f32_to_bf16_trunc(float f) { return static_cast<uint16_t>(f2u(f) >> 16); }

// RELU's bf16 store: finite values at or above the largest bf16 (0x7f7f8000) become +-Inf, then truncate.
__device__ __forceinline__ uint16_t f32_to_bf16_trunc_inf(float f)
{
    const uint32_t u = f2u(f);
    const uint32_t a = u & 0x7fffffffu;
    const uint32_t inf = (u & 0x80000000u) | 0x7f800000u;
    return static_cast<uint16_t>(((a >= 0x7f7f8000u && a < 0x7f800000u) ? inf : u) >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

// Value of f after a round trip through storage of dtype dt (RNE), as the reference's typed buffers do.
__device__ __forceinline__ float round_store(int dt, float f)
{
    if (dt == KUDNN_DT_BF16) {
        return bf16_to_f32(f32_to_bf16_rne(f));
    }
    if (dt == KUDNN_DT_F16) {
        return f16_to_f32(f32_to_f16_rne(f));
    }
    return f;
}

// f32 -> integer output element, as ConvertFp32ToS32 / ToS8 / ToU8 (src/dnn/src/service.cpp:77-115): values below
// the type's minimum or above its maximum saturate, the rest round half to even (nearbyintf in the default rounding
// mode). The two inputs the reference hands to the hardware's own conversion take aarch64's saturating fcvtzs /
// fcvtzu, the target the reference is built for: NaN -> 0 and, for s32, +2^31 (== (float)INT32_MAX, so not "above"
// it) -> INT32_MAX.
__device__ __forceinline__ int32_t f32_to_int_sat(float v, int dt)
{
    const float lo = dt == KUDNN_DT_S32 ? -2147483648.0f : (dt == KUDNN_DT_S8 ? -128.0f : 0.0f);
    const float hi = dt == KUDNN_DT_S32 ? 2147483648.0f : (dt == KUDNN_DT_S8 ? 127.0f : 255.0f);
    if (v != v) {
        return 0;
    }
    if (v <= lo) {
        return dt == KUDNN_DT_S32 ? INT32_MIN : static_cast<int32_t>(lo);
    }
    if (v >= hi) {
        return dt == KUDNN_DT_S32 ? INT32_MAX : static_cast<int32_t>(hi);
    }
    return static_cast<int32_t>(__builtin_rintf(v));
}

// Element of dtype dt as f32 (8-bit integers are exact; int32 rounds to nearest even beyond 2^24, as
// static_cast<float> does in the reference's MatrixConverter).
__device__ __forceinline__ float load_elem(const void *p, int dt, int64_t idx)
{
    switch (dt) {
        case KUDNN_DT_F32: return static_cast<const float *>(p)[idx];
        case KUDNN_DT_BF16: return bf16_to_f32(static_cast<const uint16_t *>(p)[idx]);
        case KUDNN_DT_F16: return f16_to_f32(static_cast<const uint16_t *>(p)[idx]);
        case KUDNN_DT_S8: return static_cast<float>(static_cast<const int8_t *>(p)[idx]);
        case KUDNN_DT_U8: return static_cast<float>(static_cast<const uint8_t *>(p)[idx]);
        case KUDNN_DT_S32: return static_cast<float>(static_cast<const int32_t *>(p)[idx]);
        default: return 0.0f;
    }
}

// Stores a value that is already rounded to dt (exact conversion), or rounds with RNE; integer types saturate and
// round half to even (f32_to_int_sat; exact for the integer values of operand packing).
__device__ __forceinline__ void store_elem(void *p, int dt, int64_t idx, float v)
{
    switch (dt) {
        case KUDNN_DT_F32: static_cast<float *>(p)[idx] = v; break;
        case KUDNN_DT_BF16: static_cast<uint16_t *>(p)[idx] = f32_to_bf16_rne(v); break;
        case KUDNN_DT_F16: static_cast<uint16_t *>(p)[idx] = f32_to_f16_rne(v); break;
        case KUDNN_DT_S8: static_cast<int8_t *>(p)[idx] = static_cast<int8_t>(f32_to_int_sat(v, dt)); break;
        case KUDNN_DT_U8: static_cast<uint8_t *>(p)[idx] = static_cast<uint8_t>(f32_to_int_sat(v, dt)); break;
        case KUDNN_DT_S32: static_cast<int32_t *>(p)[idx] = f32_to_int_sat(v, dt); break;
        default: break;
    }
}

// ---------------------------------------------------------------------------------------------------
// activations (f32 math)

// exp via the hardware base-2 exponential: e^x = 2^(x*log2 e).
__device__ __forceinline__ float fast_exp(float x) { return __expf(x); }

// RELU: x <= 0 -> alpha*x, else x (relu/relu.c:14-25; a negative input times alpha 0 keeps its sign).
__device__ __forceinline__ float act_relu(float x, float alpha) { return (x <= 0.0f) ? x * alpha : x; }

// SWISH: x * sigmoid(alpha*x) with sigmoid(t) = 1/(1+e^{-t}); the reference saturates the exponent
// argument to [-87, 87] (vml_sve_la_sigmoid.h:37-47, swish/vml_sve_la_swishf.c:31-47).
__device__ __forceinline__ float act_swish(float x, float alpha)
{
    float t = -alpha * x;
    float s;
    if (t > 87.0f) {
        s = 0.0f;
    } else if (t < -87.0f) {
        s = 1.0f;
    } else {
        s = __builtin_amdgcn_rcpf(1.0f + fast_exp(t));
    }
    return x * s;
}

// GELU (tanh form): 0.5*x*(1 + tanh(y)), y = sqrt(2/pi)*x*(1 + 0.044715*x^2) (gelu_tanh/vml_sve_la_gelu_tanh.h:22-39).
// Evaluated through 0.5*(1 + tanh(y)) = 1/(1 + e^{-2y}) as x / (1 + 2^(x*(c0 + c1*x^2))), c0 = -2*sqrt(2/pi)*log2(e),
// c1 = 0.044715*c0: one exp2 and one reciprocal, and no cancellation near 0. The limits are those of the tanh form:
// x -> +inf gives x, x -> -inf gives -0 for finite x and NaN for -inf (-inf * 0).
__device__ __forceinline__ float act_gelu_tanh(float x)
{
    const float kC0 = -2.302208198144325f;   // -2 * sqrt(2/pi) * log2(e)
    const float kC1 = -0.1029432395800235f;   // 0.044715 * kC0
    const float z = x * fmaf(kC1, x * x, kC0);
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
}

// GELU (erf form): 0.5*x*(1 + erf(x/sqrt(2))) (gelu_erf/vml_sve_la_gelu_erf.h:20-28).
__device__ __forceinline__ float act_gelu_erf(float x)
{
    const float kInvSqrt2 = 0.7071067811865476f;
    return 0.5f * x * (1.0f + erff(x * kInvSqrt2));
}

// The remaining kinds of the reference's forward activation table (src/dnn/src/kudnn_eltwise.cpp:333-400), f32 math
// from each kernel's f32 source (kernels/vml/*): alpha and beta as ActivationLayerFWD passes them.
__device__ __forceinline__ float act_other(int kind, float x, float alpha, float beta)
{
    switch (kind) {
        case KUDNN_ACT_ABS: return fabsf(x);                       // abs/vml_sve_la_absf.c
        case KUDNN_ACT_EXP: return expf(x);                        // exp/vml_sve_la_expf.c
        case KUDNN_ACT_LINEAR: return fmaf(alpha, x, beta);        // linear.c: svmad(alpha, x, beta)
        case KUDNN_ACT_LOG: return logf(x);                        // log/vml_sve_la_lnf.c
        case KUDNN_ACT_ROUND: return rintf(x);                     // round/vml_sve_la_nearbyintf.c: ties to even
        case KUDNN_ACT_SQRT: return sqrtf(x);                      // sqrt/vml_sve_la_sqrtf.c
        case KUDNN_ACT_SQUARE: return x * x;                       // sqr/vml_sve_la_sqrf.c
        case KUDNN_ACT_TANH: return tanhf(x);                      // tanh/vml_sve_la_tanhf.c
        case KUDNN_ACT_SIGMOID: return 1.0f / (1.0f + expf(-x));   // logistic/sigmoid.c: sigmoid of -x negated
        case KUDNN_ACT_POW: return powf(x, beta) * alpha;          // pow: alpha * x^beta (powx_calculations.h:506-515)
        case KUDNN_ACT_CLIP:                                       // clip/clipf.c: <= alpha -> alpha, > beta -> beta
            return x <= alpha ? alpha : (x > beta ? beta : x);
        case KUDNN_ACT_CLIP_V2:                                    // clipv2/clipv2f.c: <= alpha -> alpha, >= beta -> beta
            return x <= alpha ? alpha : (x >= beta ? beta : x);
        case KUDNN_ACT_HARDSIGMOID:                                // hardsigmoid: minnm / maxnm (a NaN gives 1)
            return fmaxf(fminf(fmaf(x, alpha, beta), 1.0f), 0.0f);
        case KUDNN_ACT_HARDSWISH:                                  // hardswish: x * max(0, min(1, alpha*x + beta))
            return x * fmaxf(fminf(fmaf(alpha, x, beta), 1.0f), 0.0f);
        case KUDNN_ACT_ELU:                                        // elu/vml_sve_la_eluf.c: alpha*e^x - alpha, fused
            return x > 0.0f ? x : fmaf(expf(x), alpha, -alpha);
        case KUDNN_ACT_ELU_DST: return x > 0.0f ? x : alpha * expm1f(x);  // elu/eludstf.c
        case KUDNN_ACT_SRELU: {                                    // soft_relu/vml_sve_la_softrelu.h: ln(1+e^(ax))/a
            const float ax = alpha * x;
            if (ax >= 88.7228394f) {                               // exp's upper bound: the result is x
                return x;
            }
            return log1pf(expf(fmaxf(ax, -87.3365479f))) / alpha;  // ax clamped to exp's lower bound
        }
        case KUDNN_ACT_MISH: {                                     // mish: x * ((e^x+1)^2 - 1) / ((e^x+1)^2 + 1)
            const float e1 = expf(fminf(x, 44.3614197f)) + 1.0f;   // exponent capped as the reference's
            const float e2 = e1 * e1;
            return x * ((e2 - 1.0f) / (e2 + 1.0f));
        }
        default: return x;
    }
}

__device__ __forceinline__ float apply_act(int kind, float x, float alpha, float beta = 0.0f)
{
    switch (kind) {
        case KUDNN_ACT_UNIMPLEMENTED: return x;
        case KUDNN_ACT_RELU: return act_relu(x, alpha);
        case KUDNN_ACT_SWISH: return act_swish(x, alpha);
        case KUDNN_ACT_GELU_TANH: return act_gelu_tanh(x);
        case KUDNN_ACT_GELU_ERF: return act_gelu_erf(x);
        default: return act_other(kind, x, alpha, beta);
    }
}

// Rounding of an activation output stored as dt (vml bf16 kernels truncate; f16 kernels convert RNE).
__device__ __forceinline__ float act_round(int dt, int kind, float v)
{
    if (dt == KUDNN_DT_BF16) {
        // RELU, CLIP, CLIP_V2, ELU, LINEAR, POW, ROUND and SRELU send values at or above the largest bf16 to +-Inf
        // before truncating (SvF32CvtBf16InfSpecial in their FWD kernels); ELU_DST rounds to nearest even
        // (eludstbf16.c, SveCvtU32ToU16); the others truncate
        if (kind == KUDNN_ACT_ELU_DST) {
            return bf16_to_f32(f32_to_bf16_rne(v));
        }
        const bool inf = kind == KUDNN_ACT_RELU || kind == KUDNN_ACT_CLIP || kind == KUDNN_ACT_CLIP_V2 ||
                         kind == KUDNN_ACT_ELU || kind == KUDNN_ACT_LINEAR || kind == KUDNN_ACT_POW ||
                         kind == KUDNN_ACT_ROUND || kind == KUDNN_ACT_SRELU;
        uint16_t h = inf ? f32_to_bf16_trunc_inf(v) : f32_to_bf16_trunc(v);
        return bf16_to_f32(h);
    }
    if (dt == KUDNN_DT_F16) {
        return f16_to_f32(f32_to_f16_rne(v));
    }
    return v;
}

// ---------------------------------------------------------------------------------------------------
// fused epilogue

// Per-batch base offsets (in elements) of the epilogue tensors for a flattened batch index.
struct EpiBatch {
    int64_t c, bias, src, y;
    int64_t corr_m, corr_n;
};

__device__ __forceinline__ EpiBatch epi_batch_offsets(const EpiParams &e, int64_t b)
{
    int64_t i2 = b % e.bdim[2];
    int64_t t = b / e.bdim[2];
    int64_t i1 = t % e.bdim[1];
    int64_t i0 = t / e.bdim[1];
    EpiBatch o;
    o.c = i0 * e.c_bs[0] + i1 * e.c_bs[1] + i2 * e.c_bs[2];
    o.bias = i0 * e.bias_bs[0] + i1 * e.bias_bs[1] + i2 * e.bias_bs[2];
    o.src = i0 * e.src_bs[0] + i1 * e.src_bs[1] + i2 * e.src_bs[2];
    o.y = i0 * e.y_bs[0] + i1 * e.y_bs[1] + i2 * e.y_bs[2];
    o.corr_m = b * e.corr_m_bs;
    o.corr_n = b * e.corr_n_bs;
    return o;
}

// Epilogue forms (the types of every epilogue tensor, fixed at compile time in the fast paths): all bf16, all f32,
// all f16, or read at run time; EPI_FORM_I32 is the integer epilogue of s8 x s8 -> s32 (further below);
// EPI_FORM_PARTIAL stores a K slice's f32 sums and no epilogue (the ping-pong kernel's K slices).
enum { EPI_FORM_BF16 = 0, EPI_FORM_F32 = 1, EPI_FORM_GENERIC = 2, EPI_FORM_PARTIAL = 3, EPI_FORM_I32 = 4, EPI_FORM_F16 = 5 };

template <int FORM>
constexpr int form_dt()
{
    return FORM == EPI_FORM_BF16 ? KUDNN_DT_BF16 : (FORM == EPI_FORM_F16 ? KUDNN_DT_F16 : KUDNN_DT_F32);
}

// Raw bits of one element of dtype dt (f32 / s32: 32 bits; bf16 / f16: 16 bits, zero-extended; s8 sign-extended,
// u8 zero-extended).
__device__ __forceinline__ uint32_t load_raw1(const void *p, int dt, int64_t idx)
{
    switch (dt) {
        case KUDNN_DT_F32:
        case KUDNN_DT_S32: return static_cast<const uint32_t *>(p)[idx];
        case KUDNN_DT_BF16:
        case KUDNN_DT_F16: return static_cast<const uint16_t *>(p)[idx];
        case KUDNN_DT_S8: return static_cast<uint32_t>(static_cast<int32_t>(static_cast<const int8_t *>(p)[idx]));
        case KUDNN_DT_U8: return static_cast<const uint8_t *>(p)[idx];
        default: return 0u;
    }
}

__device__ __forceinline__ float raw1_to_f32(uint32_t r, int dt)
{
    switch (dt) {
        case KUDNN_DT_F32: return u2f(r);
        case KUDNN_DT_BF16: return u2f(r << 16);
        case KUDNN_DT_F16: return f16_to_f32(static_cast<uint16_t>(r));
        case KUDNN_DT_S8:
        case KUDNN_DT_S32: return static_cast<float>(static_cast<int32_t>(r));
        case KUDNN_DT_U8: return static_cast<float>(r);
        default: return 0.0f;
    }
}

// Marks x as read and rewritten here, so that nothing computed from it is moved above this point.
__device__ __forceinline__ uint32_t use_here(uint32_t x)
{
    asm volatile("" : "+v"(x));
    return x;
}

// Epilogue operands of one output element (C when beta != 0, bias, binary operand), loadable ahead of the
// accumulator so that their latency overlaps the main loop. They are kept as raw bits and converted where they are
// used (behind use_here): a conversion next to the load would make the wave wait for it before issuing the loads
// that follow.
struct EpiPre1 {
    uint32_t c, bias, src;
};

// FORM fixes the operand types (a fixed form has beta == 0 and bias / binary operand of the output's type); the
// generic form reads them from e.
template <int FORM = EPI_FORM_GENERIC>
__device__ __forceinline__ EpiPre1 epi_prefetch1(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n)
{
    EpiPre1 p{0u, 0u, 0u};
    if (FORM == EPI_FORM_GENERIC && e.beta != 0.0f) {
        p.c = load_raw1(e.c, e.c_dt, ob.c + m * e.c_sm + n * e.c_sn);
    }
    if (e.bias != nullptr) {
        p.bias = load_raw1(e.bias, FORM == EPI_FORM_GENERIC ? e.bias_dt : form_dt<FORM>(),
                           ob.bias + m * e.bias_sm + n * e.bias_sn);
    }
    if (e.bin != KUDNN_BINARY_NONE) {
        p.src = load_raw1(e.src, FORM == EPI_FORM_GENERIC ? e.src_dt : form_dt<FORM>(),
                          ob.src + m * e.src_sm + n * e.src_sn);
    }
    return p;
}

// Applies the epilogue to one accumulator value of output element (m, n), with its operands from epi_prefetch1.
__device__ __forceinline__ void epi_apply_pre(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, float acc,
                                              const EpiPre1 &p)
{
    float v = acc * e.alpha;
    if (e.beta != 0.0f) {
        v += e.beta * raw1_to_f32(use_here(p.c), e.c_dt);
    }
    if (e.bias != nullptr) {
        v += raw1_to_f32(use_here(p.bias), e.bias_dt);
    }
    v = round_store(e.c_dt, v);
    if (e.store_c) {
        store_elem(e.c, e.c_dt, ob.c + m * e.c_sm + n * e.c_sn, v);
    }
    if (e.act != KUDNN_ACT_UNIMPLEMENTED) {
        v = act_round(e.c_dt, e.act, apply_act(e.act, v, e.act_alpha, e.act_beta));
    }
    if (e.bin != KUDNN_BINARY_NONE) {
        const float sv = raw1_to_f32(use_here(p.src), e.src_dt);
        if (e.bin == KUDNN_BINARY_ADD) {
            v = v + sv;
        } else if (e.bin == KUDNN_BINARY_EXT) {
            v = fmaf(sv, e.gamma, v);
        } else {
            v = v * sv;
        }
    }
    store_elem(e.y, e.y_dt, ob.y + m * e.y_sm + n * e.y_sn, v);
}

// Applies the epilogue to one accumulator value of output element (m, n). m, n are in bounds.
__device__ __forceinline__ void epi_apply(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, float acc)
{
    epi_apply_pre(e, ob, m, n, acc, epi_prefetch1(e, ob, m, n));
}

// Epilogue for four consecutive columns n..n+3 of row m (the MFMA output layout gives each lane runs
// of four columns). Uses 8/16-byte accesses when the tensors are contiguous along n and aligned.
// Raw bits of the bias and binary operand of a run of 4 columns (m, n .. n+3), loaded ahead of the accumulators
// when the run takes the fast4 path with f32 or bf16 operands (other cases load at use). Each width has its own
// registers, so no copy (and no wait for the load) joins the two load paths.
struct EpiPre4 {
    uint2 src16, bias16;
    uint4 src32, bias32;
};

__device__ __forceinline__ EpiPre4 epi_prefetch4(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, int64_t N)
{
    EpiPre4 p{make_uint2(0u, 0u), make_uint2(0u, 0u), make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
    if (n + 3 < N && e.fast4) {
        if (e.bin != KUDNN_BINARY_NONE) {
            const int64_t si = ob.src + m * e.src_sm + n;
            if (e.src_dt == KUDNN_DT_BF16) {
                p.src16 = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(e.src) + si);
            } else if (e.src_dt == KUDNN_DT_F32) {
                p.src32 = *reinterpret_cast<const uint4 *>(static_cast<const float *>(e.src) + si);
            }
        }
        if (e.bias != nullptr && e.bias_sn != 0) {
            const int64_t bi = ob.bias + m * e.bias_sm + n * e.bias_sn;
            if (e.bias_dt == KUDNN_DT_BF16) {
                p.bias16 = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(e.bias) + bi);
            } else if (e.bias_dt == KUDNN_DT_F32) {
                p.bias32 = *reinterpret_cast<const uint4 *>(static_cast<const float *>(e.bias) + bi);
            }
        }
    }
    return p;
}

// 4 values of dtype dt (f32 or bf16) from the raw bits of epi_prefetch4.
__device__ __forceinline__ void unpack_pre4(const uint2 &r16, const uint4 &r32, int dt, float v[4])
{
    if (dt == KUDNN_DT_BF16) {
        const uint32_t x = use_here(r16.x), y = use_here(r16.y);
        v[0] = u2f(x << 16);
        v[1] = u2f(x & 0xffff0000u);
        v[2] = u2f(y << 16);
        v[3] = u2f(y & 0xffff0000u);
    } else {
        v[0] = u2f(use_here(r32.x));
        v[1] = u2f(use_here(r32.y));
        v[2] = u2f(use_here(r32.z));
        v[3] = u2f(use_here(r32.w));
    }
}

// Epilogue of the run of 4 columns (m, n .. n+3) (the columns at or past N are skipped), with operands from
// epi_prefetch4.
__device__ __forceinline__ void epi_apply4_pre(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, int64_t N,
                                               const float acc[4], const EpiPre4 &pre)
{
    if (n + 3 < N && e.fast4) {
        // fast4: y (and src / bias when present) are contiguous along n and 4-element aligned,
        // c is not re-read (beta == 0) and not separately stored unless contiguous too.
        float v[4];
        float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (e.bias != nullptr) {
            int64_t bi = ob.bias + m * e.bias_sm + n * e.bias_sn;
            if (e.bias_sn == 0) {
                float b0 = load_elem(e.bias, e.bias_dt, bi);
                bv[0] = bv[1] = bv[2] = bv[3] = b0;
            } else if (e.bias_dt == KUDNN_DT_F32 || e.bias_dt == KUDNN_DT_BF16) {
                unpack_pre4(pre.bias16, pre.bias32, e.bias_dt, bv);
            } else {
                for (int q = 0; q < 4; ++q) bv[q] = load_elem(e.bias, e.bias_dt, bi + q);
            }
        }
        for (int q = 0; q < 4; ++q) {
            v[q] = round_store(e.c_dt, acc[q] * e.alpha + bv[q]);
        }
        if (e.store_c) {
            int64_t ci = ob.c + m * e.c_sm + n;
            if (e.c_dt == KUDNN_DT_F32) {
                *reinterpret_cast<float4 *>(static_cast<float *>(e.c) + ci) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
                for (int q = 0; q < 4; ++q) store_elem(e.c, e.c_dt, ci + q, v[q]);
            }
        }
        if (e.act != KUDNN_ACT_UNIMPLEMENTED) {
            for (int q = 0; q < 4; ++q) v[q] = act_round(e.c_dt, e.act, apply_act(e.act, v[q], e.act_alpha, e.act_beta));
        }
        if (e.bin != KUDNN_BINARY_NONE) {
            int64_t si = ob.src + m * e.src_sm + n;
            float s[4];
            if (e.src_dt == KUDNN_DT_BF16 || e.src_dt == KUDNN_DT_F32) {
                unpack_pre4(pre.src16, pre.src32, e.src_dt, s);
            } else {
                for (int q = 0; q < 4; ++q) s[q] = load_elem(e.src, e.src_dt, si + q);
            }
            for (int q = 0; q < 4; ++q) {
                if (e.bin == KUDNN_BINARY_ADD) {
                    v[q] = v[q] + s[q];
                } else if (e.bin == KUDNN_BINARY_EXT) {
                    v[q] = fmaf(s[q], e.gamma, v[q]);
                } else {
                    v[q] = v[q] * s[q];
                }
            }
        }
        int64_t yi = ob.y + m * e.y_sm + n;
        if (e.y_dt == KUDNN_DT_BF16) {
            uint32_t lo = pack_bf16x2_rne(v[0], v[1]);
            uint32_t hi = pack_bf16x2_rne(v[2], v[3]);
            *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(e.y) + yi) = make_uint2(lo, hi);
        } else if (e.y_dt == KUDNN_DT_F32) {
            *reinterpret_cast<float4 *>(static_cast<float *>(e.y) + yi) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            for (int q = 0; q < 4; ++q) store_elem(e.y, e.y_dt, yi + q, v[q]);
        }
        return;
    }
    for (int q = 0; q < 4; ++q) {
        if (n + q < N) {
            epi_apply(e, ob, m, n + q, acc[q]);
        }
    }
}

__device__ __forceinline__ void epi_apply4(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, int64_t N,
                                           const float acc[4])
{
    epi_apply4_pre(e, ob, m, n, N, acc, epi_prefetch4(e, ob, m, n, N));
}

// Epilogue for eight consecutive columns n..n+7 of row m (n a multiple of 8): one 16-byte bf16 (or two
// 16-byte f32) store per call when the output rows are contiguous and 8-element aligned (fast8).
__device__ __forceinline__ void epi_apply8(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, int64_t N,
                                           const float acc[8])
{
    if (n + 7 < N && e.fast8) {
        float v[8];
        float bv[8];
        if (e.bias != nullptr) {
            const int64_t bi = ob.bias + m * e.bias_sm + n * e.bias_sn;
            if (e.bias_sn == 0) {
                const float b0 = load_elem(e.bias, e.bias_dt, bi);
#pragma unroll
                for (int q = 0; q < 8; ++q) bv[q] = b0;
            } else if (e.bias_dt == KUDNN_DT_BF16) {
                const uint4 raw = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(e.bias) + bi);
                const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    bv[2 * q] = u2f(w[q] << 16);
                    bv[2 * q + 1] = u2f(w[q] & 0xffff0000u);
                }
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) bv[q] = load_elem(e.bias, e.bias_dt, bi + q);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q) bv[q] = 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            v[q] = round_store(e.c_dt, acc[q] * e.alpha + bv[q]);
        }
        if (e.store_c) {
            const int64_t ci = ob.c + m * e.c_sm + n;
#pragma unroll
            for (int q = 0; q < 8; ++q) store_elem(e.c, e.c_dt, ci + q, v[q]);
        }
        if (e.act != KUDNN_ACT_UNIMPLEMENTED) {
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = act_round(e.c_dt, e.act, apply_act(e.act, v[q], e.act_alpha, e.act_beta));
        }
        if (e.bin != KUDNN_BINARY_NONE) {
            const int64_t si = ob.src + m * e.src_sm + n;
            float sv[8];
            if (e.src_dt == KUDNN_DT_BF16) {
                const uint4 raw = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(e.src) + si);
                const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    sv[2 * q] = u2f(w[q] << 16);
                    sv[2 * q + 1] = u2f(w[q] & 0xffff0000u);
                }
            } else if (e.src_dt == KUDNN_DT_F32) {
                const float4 t0 = *reinterpret_cast<const float4 *>(static_cast<const float *>(e.src) + si);
                const float4 t1 = *reinterpret_cast<const float4 *>(static_cast<const float *>(e.src) + si + 4);
                sv[0] = t0.x; sv[1] = t0.y; sv[2] = t0.z; sv[3] = t0.w;
                sv[4] = t1.x; sv[5] = t1.y; sv[6] = t1.z; sv[7] = t1.w;
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) sv[q] = load_elem(e.src, e.src_dt, si + q);
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if (e.bin == KUDNN_BINARY_ADD) {
                    v[q] = v[q] + sv[q];
                } else if (e.bin == KUDNN_BINARY_EXT) {
                    v[q] = fmaf(sv[q], e.gamma, v[q]);
                } else {
                    v[q] = v[q] * sv[q];
                }
            }
        }
        const int64_t yi = ob.y + m * e.y_sm + n;
        if (e.y_dt == KUDNN_DT_BF16) {
            uint32_t w[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                w[q] = pack_bf16x2_rne(v[2 * q], v[2 * q + 1]);
            }
            *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(e.y) + yi) = make_uint4(w[0], w[1], w[2], w[3]);
        } else if (e.y_dt == KUDNN_DT_F32) {
            float *yp = static_cast<float *>(e.y) + yi;
            *reinterpret_cast<float4 *>(yp) = make_float4(v[0], v[1], v[2], v[3]);
            *reinterpret_cast<float4 *>(yp + 4) = make_float4(v[4], v[5], v[6], v[7]);
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q) store_elem(e.y, e.y_dt, yi + q, v[q]);
        }
        return;
    }
    epi_apply4(e, ob, m, n, N, acc);
    epi_apply4(e, ob, m, n + 4, N, acc + 4);
}

// ---------------------------------------------------------------------------------------------------
// Epilogue with the activation and the tensor types fixed at compile time.
//
// The generic epilogue above dispatches every option at run time; inlined at the many call sites of an unrolled
// epilogue that is megabytes of code, and the jumps over the unused parts miss the instruction cache on every pass.
// A "form" fixes the types of every epilogue tensor: EPI_FORM_BF16 (C rounding, bias, binary operand and output all
// bf16) or EPI_FORM_F32 (all f32), in both cases with C not stored separately, beta == 0 and fast8 (output and binary
// operand contiguous along n, 16-byte aligned 8-column groups). Anything else is EPI_FORM_GENERIC and goes through
// epi_apply. Arithmetic and rounding are those of epi_apply.

// Host-side choice of the form for an epilogue. need8: the kernel stores 8-column groups with 16-byte accesses
// (fast8 must hold); a kernel that stores single elements passes false.
inline int epi_form(const EpiParams &e, bool need8 = true)
{
    const int dt = e.y_dt;
    if (e.acc_i32) {
        // the only epilogue of int32 accumulators (the host admits no other options); it checks fast8 itself
        return EPI_FORM_I32;
    }
    if ((need8 && !e.fast8) || e.store_c || e.beta != 0.0f) {
        return EPI_FORM_GENERIC;
    }
    if ((dt != KUDNN_DT_BF16 && dt != KUDNN_DT_F32 && dt != KUDNN_DT_F16) || e.c_dt != dt ||
        (e.bin != KUDNN_BINARY_NONE && e.src_dt != dt) || (e.bias != nullptr && e.bias_dt != dt)) {
        return EPI_FORM_GENERIC;
    }
    return dt == KUDNN_DT_BF16 ? EPI_FORM_BF16 : (dt == KUDNN_DT_F16 ? EPI_FORM_F16 : EPI_FORM_F32);
}

template <int ACT>
__device__ __forceinline__ float act_fixed(float x, float alpha)
{
    if constexpr (ACT == KUDNN_ACT_RELU) {
        return act_relu(x, alpha);
    } else if constexpr (ACT == KUDNN_ACT_SWISH) {
        return act_swish(x, alpha);
    } else if constexpr (ACT == KUDNN_ACT_GELU_TANH) {
        return act_gelu_tanh(x);
    } else if constexpr (ACT == KUDNN_ACT_GELU_ERF) {
        return act_gelu_erf(x);
    } else {
        return x;
    }
}

// Raw bits of 8 consecutive elements: one 16-byte word for bf16, two for f32.
struct Raw8 {
    uint4 lo, hi;
};

// Bias and binary operand of one 8-column group, as loaded by epi_prefetch8.
struct Pre8 {
    Raw8 src, bias;
};

template <int FORM>
__device__ __forceinline__ Raw8 load_raw8(const void *p, int64_t idx)
{
    Raw8 r{make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
    if constexpr (FORM == EPI_FORM_BF16 || FORM == EPI_FORM_F16) {
        r.lo = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p) + idx);
    } else {
        const uint4 *q = reinterpret_cast<const uint4 *>(static_cast<const float *>(p) + idx);
        r.lo = q[0];
        r.hi = q[1];
    }
    return r;
}

template <int FORM>
__device__ __forceinline__ void unpack_raw8(const Raw8 &r, float v[8])
{
    const uint32_t w[8] = {r.lo.x, r.lo.y, r.lo.z, r.lo.w, r.hi.x, r.hi.y, r.hi.z, r.hi.w};
    if constexpr (FORM == EPI_FORM_BF16) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[2 * q] = u2f(w[q] << 16);
            v[2 * q + 1] = u2f(w[q] & 0xffff0000u);
        }
    } else if constexpr (FORM == EPI_FORM_F16) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[2 * q] = f16_to_f32(static_cast<uint16_t>(w[q]));
            v[2 * q + 1] = f16_to_f32(static_cast<uint16_t>(w[q] >> 16));
        }
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = u2f(w[q]);
    }
}

// Binary operand of group (m, n .. n+7).
template <int FORM>
__device__ __forceinline__ Raw8 epi_prefetch8_src(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n)
{
    Raw8 r{};
    if (e.bin != KUDNN_BINARY_NONE) {
        r = load_raw8<FORM>(e.src, ob.src + m * e.src_sm + n);
    }
    return r;
}

// Bias of group (m, n .. n+7). A bias broadcast along n (bias_sn == 0) is one value, kept as f32 bits in lo.x.
template <int FORM>
__device__ __forceinline__ Raw8 epi_prefetch8_bias(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n)
{
    Raw8 r{};
    if (e.bias != nullptr) {
        if (e.bias_sn == 0) {
            r.lo.x = f2u(load_elem(e.bias, form_dt<FORM>(), ob.bias + m * e.bias_sm));
        } else {
            r = load_raw8<FORM>(e.bias, ob.bias + m * e.bias_sm + n);
        }
    }
    return r;
}

// Loads the binary operand and the bias of group (m, n .. n+7).
template <int FORM>
__device__ __forceinline__ Pre8 epi_prefetch8(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n)
{
    return Pre8{epi_prefetch8_src<FORM>(e, ob, m, n), epi_prefetch8_bias<FORM>(e, ob, m, n)};
}

// 16-byte store of a result that no later step of the kernel reads: non-temporal, so the L2 does not allocate lines
// for it (C3: 3 % faster than an ordinary store). Loads of the binary operand stay ordinary: made non-temporal as
// well, they were slower.
__device__ __forceinline__ void store16_stream(void *p, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3)
{
    typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t v = {w0, w1, w2, w3};
    __builtin_nontemporal_store(v, static_cast<u32x4_t *>(p));
}

// Epilogue of 8 consecutive columns of one row, all in bounds: acc are the accumulators, bv the bias values (read
// only when e.bias is set), src the binary operand's raw bits (epi_prefetch8_src), yp the output's first element.
template <int ACT, int FORM>
__device__ __forceinline__ void epi_fast8_core(const EpiParams &e, void *yp, const float acc[8], const Raw8 &src,
                                               const float bv[8])
{
    constexpr int DT = form_dt<FORM>();
    float v[8];
    if (e.bias != nullptr) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = fmaf(acc[q], e.alpha, bv[q]);
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = acc[q] * e.alpha;
    }
    if constexpr (DT == KUDNN_DT_BF16) {
#pragma unroll
        for (int q = 0; q < 4; ++q) round_bf16_pair(v[2 * q], v[2 * q + 1]);
    } else if constexpr (DT == KUDNN_DT_F16) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = round_store(DT, v[q]);
    }
    if constexpr (ACT != KUDNN_ACT_UNIMPLEMENTED) {
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = act_round(DT, ACT, act_fixed<ACT>(v[q], e.act_alpha));
    }
    if (e.bin != KUDNN_BINARY_NONE) {
        float sv[8];
        unpack_raw8<FORM>(src, sv);
        if (e.bin == KUDNN_BINARY_ADD) {
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = v[q] + sv[q];
        } else if (e.bin == KUDNN_BINARY_EXT) {
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = fmaf(sv[q], e.gamma, v[q]);
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = v[q] * sv[q];
        }
    }
    if constexpr (FORM == EPI_FORM_BF16 || FORM == EPI_FORM_F16) {
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (FORM == EPI_FORM_BF16) {
                w[q] = pack_bf16x2_rne(v[2 * q], v[2 * q + 1]);
            } else {
                w[q] = static_cast<uint32_t>(f32_to_f16_rne(v[2 * q])) |
                       (static_cast<uint32_t>(f32_to_f16_rne(v[2 * q + 1])) << 16);
            }
        }
        store16_stream(yp, w[0], w[1], w[2], w[3]);
    } else {
        float *fp = static_cast<float *>(yp);
        store16_stream(fp, f2u(v[0]), f2u(v[1]), f2u(v[2]), f2u(v[3]));
        store16_stream(fp + 4, f2u(v[4]), f2u(v[5]), f2u(v[6]), f2u(v[7]));
    }
}

// The bias values of an 8-column group from epi_prefetch8_bias's raw bits (one value broadcast when the bias has one
// column).
template <int FORM>
__device__ __forceinline__ void epi_bias8(const EpiParams &e, const Raw8 &raw, float bv[8])
{
    if (e.bias != nullptr && e.bias_sn == 0) {
#pragma unroll
        for (int q = 0; q < 8; ++q) bv[q] = u2f(raw.lo.x);
    } else {
        unpack_raw8<FORM>(raw, bv);
    }
}

// Epilogue of the 8-column group (m, n .. n+7), all in bounds, operands from epi_prefetch8.
template <int ACT, int FORM>
__device__ __forceinline__ void epi_fast8(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, const float acc[8],
                                          const Pre8 &pre)
{
    constexpr int ES = form_dt<FORM>() == KUDNN_DT_F32 ? 4 : 2;
    float bv[8];
    epi_bias8<FORM>(e, pre.bias, bv);
    epi_fast8_core<ACT, FORM>(e, static_cast<char *>(e.y) + (ob.y + m * e.y_sm + n) * ES, acc, pre.src, bv);
}

// Epilogue of one element (m, n) in a fixed form, its bias and binary operand from epi_prefetch1.
template <int ACT, int FORM>
__device__ __forceinline__ void epi_elem_pre(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, float acc,
                                             const EpiPre1 &p)
{
    constexpr int DT = form_dt<FORM>();
    float v = acc * e.alpha;
    if (e.bias != nullptr) {
        v += raw1_to_f32(use_here(p.bias), DT);
    }
    v = round_store(DT, v);
    if constexpr (ACT != KUDNN_ACT_UNIMPLEMENTED) {
        v = act_round(DT, ACT, act_fixed<ACT>(v, e.act_alpha));
    }
    if (e.bin != KUDNN_BINARY_NONE) {
        const float sv = raw1_to_f32(use_here(p.src), DT);
        if (e.bin == KUDNN_BINARY_ADD) {
            v = v + sv;
        } else if (e.bin == KUDNN_BINARY_EXT) {
            v = fmaf(sv, e.gamma, v);
        } else {
            v = v * sv;
        }
    }
    store_elem(e.y, DT, ob.y + m * e.y_sm + n * e.y_sn, v);
}

// Epilogue of one in-bounds element (m, n) in a fixed form (used at the matrix edge).
template <int ACT, int FORM>
__device__ __forceinline__ void epi_elem(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, float acc)
{
    constexpr int DT = form_dt<FORM>();
    float v = acc * e.alpha;
    if (e.bias != nullptr) {
        v += load_elem(e.bias, DT, ob.bias + m * e.bias_sm + n * e.bias_sn);
    }
    v = round_store(DT, v);
    if constexpr (ACT != KUDNN_ACT_UNIMPLEMENTED) {
        v = act_round(DT, ACT, act_fixed<ACT>(v, e.act_alpha));
    }
    if (e.bin != KUDNN_BINARY_NONE) {
        const float sv = load_elem(e.src, DT, ob.src + m * e.src_sm + n);
        if (e.bin == KUDNN_BINARY_ADD) {
            v = v + sv;
        } else if (e.bin == KUDNN_BINARY_EXT) {
            v = fmaf(sv, e.gamma, v);
        } else {
            v = v * sv;
        }
    }
    store_elem(e.y, DT, ob.y + m * e.y_sm + n, v);
}

// Epilogue for four consecutive columns n..n+3 of row m in a fixed form (EPI_FORM_BF16 or EPI_FORM_F32), with the bias
// and binary operand of epi_prefetch4; the arithmetic and rounding of epi_apply4_pre. Columns at or past N are skipped.
template <int ACT, int FORM>
__device__ __forceinline__ void epi_fixed4(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, int64_t N,
                                           const float acc[4], const EpiPre4 &pre)
{
    static_assert(FORM == EPI_FORM_BF16 || FORM == EPI_FORM_F32, "the prefetched operands are bf16 or f32");
    constexpr int DT = form_dt<FORM>();
    if (n + 3 < N && e.fast4) {
        float v[4];
        float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (e.bias != nullptr) {
            if (e.bias_sn == 0) {
                const float b0 = load_elem(e.bias, DT, ob.bias + m * e.bias_sm);
                bv[0] = bv[1] = bv[2] = bv[3] = b0;
            } else {
                unpack_pre4(pre.bias16, pre.bias32, DT, bv);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = round_store(DT, acc[q] * e.alpha + bv[q]);
        if constexpr (ACT != KUDNN_ACT_UNIMPLEMENTED) {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = act_round(DT, ACT, act_fixed<ACT>(v[q], e.act_alpha));
        }
        if (e.bin != KUDNN_BINARY_NONE) {
            float sv[4];
            unpack_pre4(pre.src16, pre.src32, DT, sv);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (e.bin == KUDNN_BINARY_ADD) {
                    v[q] = v[q] + sv[q];
                } else if (e.bin == KUDNN_BINARY_EXT) {
                    v[q] = fmaf(sv[q], e.gamma, v[q]);
                } else {
                    v[q] = v[q] * sv[q];
                }
            }
        }
        const int64_t yi = ob.y + m * e.y_sm + n;
        if constexpr (FORM == EPI_FORM_BF16) {
            *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(e.y) + yi) =
                make_uint2(pack_bf16x2_rne(v[0], v[1]), pack_bf16x2_rne(v[2], v[3]));
        } else {
            *reinterpret_cast<float4 *>(static_cast<float *>(e.y) + yi) = make_float4(v[0], v[1], v[2], v[3]);
        }
        return;
    }
#pragma unroll 1
    for (int q = 0; q < 4; ++q) {
        if (n + q < N) {
            epi_elem<ACT, FORM>(e, ob, m, n + q, acc[q]);
        }
    }
}


// Integer epilogue: s8 x s8 -> s32 (cblas_gemm_s8s8s32, src/dnn/src/kudnn_gemm.cpp:243-264, with the bias passed as
// the C offset for a row / column vector and added afterwards for a full [M, N] bias: the same sum either way).
// y = acc + bias in int32 with two's-complement wrap; alpha 1, beta 0, no activation or binary operand (the host
// rejects anything else). The bias is s32, or s8 widened exactly (ChooseImpl's wider-type match, :655-671). The
// accumulators arrive as the bit patterns of the MFMA's int32 results.
__device__ __forceinline__ uint32_t i32_bias(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n)
{
    uint32_t v = e.bias == nullptr ? 0u : load_raw1(e.bias, e.bias_dt, ob.bias + m * e.bias_sm + n * e.bias_sn);
    // u8 operands: the terms of the -128 shift (all in wrapping 32-bit arithmetic, like the accumulators)
    if (e.corr_m != nullptr) {
        v += static_cast<uint32_t>(e.corr_m[ob.corr_m + m]);
    }
    if (e.corr_n != nullptr) {
        v += static_cast<uint32_t>(e.corr_n[ob.corr_n + n]);
    }
    return v + static_cast<uint32_t>(e.corr_c);
}

// 8 consecutive columns (m, n .. n+7), all in bounds, y contiguous along n with 16-byte aligned groups (fast8; callers
// check it and use epi_i32_1 otherwise).
__device__ __forceinline__ void epi_i32_8(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, const float acc[8])
{
    uint32_t v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = f2u(acc[q]) + i32_bias(e, ob, m, n + q);
    uint4 *y = reinterpret_cast<uint4 *>(static_cast<uint32_t *>(e.y) + ob.y + m * e.y_sm + n);
    y[0] = make_uint4(v[0], v[1], v[2], v[3]);
    y[1] = make_uint4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void epi_i32_1(const EpiParams &e, const EpiBatch &ob, int64_t m, int64_t n, float acc)
{
    static_cast<uint32_t *>(e.y)[ob.y + m * e.y_sm + n * e.y_sn] = f2u(acc) + i32_bias(e, ob, m, n);
}

// XCD-aware block order. The hardware deals workgroups round-robin over the 8 XCDs (block b runs on
// XCD b % 8); this maps the hardware id to a logical id such that consecutive logical ids run on the
// same XCD and therefore share its L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks)
{
    const int kXcds = 8;
    int xcd = bid % kXcds;
    int per = nblocks / kXcds;
    int extra = nblocks % kXcds;
    return xcd * per + (xcd < extra ? xcd : extra) + bid / kXcds;
}

// Grouped tile order: walks GROUP tile-rows at a time so that co-resident blocks share A and B panels.
__device__ __forceinline__ void grouped_tile(int lid, int tilesM, int tilesN, int group, int &tm, int &tn)
{
    int perGroup = group * tilesN;
    int g = lid / perGroup;
    int firstM = g * group;
    int gsize = tilesM - firstM;
    if (gsize > group) gsize = group;
    int r = lid % perGroup;
    tm = firstM + r % gsize;
    tn = r / gsize;
}

}  // namespace kudnn_dev

#endif  // KUDNN_DEVICE_COMMON_H
