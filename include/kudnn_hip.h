/*
 * kudnn_hip.h -- C ABI of the MI355X (gfx950) implementation of KuDNN's Linear/GEMM path.
 *
 * This is the boundary between host code (the KuDNN-compatible C++ classes in libkudnn.so, or any
 * FFI such as Python ctypes) and the HIP kernels in libkudnn_hip.so. Every entry point takes plain
 * pointers, sizes and POD descriptors; no C++ types, no exceptions and no HIP headers cross it.
 *
 * Conventions
 *  - Every function returns an int status: KUDNN_STATUS_SUCCESS (0), KUDNN_STATUS_UNSUPPORTED (1) and
 *    KUDNN_STATUS_BAD_ARGUMENTS (2) carry exactly the meaning of KuDNN::Status
 *    (reference: src/dnn/include/service/kudnn_err_codes.hpp:18-22); values >= 3 are failures that the
 *    reference reports with exceptions (null pointers, allocation, HIP runtime errors).
 *    kudnn_last_error() returns a per-thread message for the last non-zero status.
 *  - Tensor descriptors hold dims, strides, dtype and layout exactly as KuDNN::TensorInfo does:
 *    dims and strides are in LOGICAL dimension order, strides of size-1 dims are 0
 *    (reference: src/dnn/include/types/kudnn_tensor_info.hpp:132-158, src/dnn/src/service.cpp:355-372).
 *  - Pointers passed to *_run may be device memory (hipMalloc, the fast path) or ordinary host memory;
 *    host pointers are staged through device buffers and the call then returns synchronously.
 *  - *_run is asynchronous on `stream` (a hipStream_t; NULL = the default stream) when every pointer is
 *    device memory. The kernel plan is fixed by *_create; the one mutable part of a handle is its device
 *    workspace (packed operands, split-K partials), which grows with hipMalloc on the first runs that need it
 *    and is then reused. Runs of one handle on several streams are correct: a run on another stream than the
 *    previous one waits (on the GPU) for that run, so they are serialised on the workspace. A cloned handle has
 *    a workspace of its own.
 */
#ifndef KUDNN_HIP_H
#define KUDNN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define KUDNN_HIP_API __attribute__((visibility("default")))
#else
#define KUDNN_HIP_API
#endif

#define KUDNN_HIP_MAX_DIMS 5

/* Status codes. 0..2 == KuDNN::Status (kudnn_err_codes.hpp:18-22). */
enum {
    KUDNN_STATUS_SUCCESS = 0,
    KUDNN_STATUS_UNSUPPORTED = 1,
    KUDNN_STATUS_BAD_ARGUMENTS = 2,
    KUDNN_STATUS_NULL_POINTER = 3,   /* reference: Service::LogicError from Run (kudnn_gemm.cpp:862-868) */
    KUDNN_STATUS_ALLOC_FAILED = 4,   /* reference: Service::BadAlloc / std::bad_alloc */
    KUDNN_STATUS_HIP_ERROR = 5,      /* HIP runtime failure (no reference counterpart) */
    KUDNN_STATUS_INTERNAL = 6
};

/* Element types; values == KuDNN::Element::TypeT (kudnn_data_type.hpp:31-39). */
enum {
    KUDNN_DT_UNDEFINED = 0,
    KUDNN_DT_F32 = 1,
    KUDNN_DT_F16 = 2,
    KUDNN_DT_BF16 = 3,
    KUDNN_DT_S32 = 4,
    KUDNN_DT_S8 = 5,
    KUDNN_DT_U8 = 6
};

/* Layouts: values == KuDNN::Layout (kudnn_layout.hpp:19-51); letters name logical dims listed from the
 * slowest physical position to the fastest. */
enum {
    KUDNN_LAYOUT_UNDEFINED = 0,
    KUDNN_LAYOUT_A, KUDNN_LAYOUT_AB, KUDNN_LAYOUT_BA,
    KUDNN_LAYOUT_ABC, KUDNN_LAYOUT_ACB, KUDNN_LAYOUT_BAC, KUDNN_LAYOUT_BCA, KUDNN_LAYOUT_CAB, KUDNN_LAYOUT_CBA,
    KUDNN_LAYOUT_ABCD, KUDNN_LAYOUT_ABDC, KUDNN_LAYOUT_ACBD, KUDNN_LAYOUT_ACDB, KUDNN_LAYOUT_ADBC,
    KUDNN_LAYOUT_ADCB, KUDNN_LAYOUT_BACD, KUDNN_LAYOUT_BCDA, KUDNN_LAYOUT_CDAB, KUDNN_LAYOUT_CDBA,
    KUDNN_LAYOUT_DCAB,
    KUDNN_LAYOUT_ABCDE, KUDNN_LAYOUT_ABCED, KUDNN_LAYOUT_ABDEC, KUDNN_LAYOUT_ACBDE, KUDNN_LAYOUT_ACDEB,
    KUDNN_LAYOUT_ADECB, KUDNN_LAYOUT_BACDE, KUDNN_LAYOUT_BCDEA, KUDNN_LAYOUT_CDEAB, KUDNN_LAYOUT_CDEBA,
    KUDNN_LAYOUT_DECAB,
    KUDNN_LAYOUT_COUNT
};

/* Activation kinds; values == KuDNN::ActivationFunction (kudnn_eltwise.hpp:24-54). */
enum {
    KUDNN_ACT_UNIMPLEMENTED = 0, KUDNN_ACT_ABS, KUDNN_ACT_EXP, KUDNN_ACT_LINEAR, KUDNN_ACT_LOG,
    KUDNN_ACT_RELU = 5, KUDNN_ACT_ROUND, KUDNN_ACT_SQRT, KUDNN_ACT_SQUARE, KUDNN_ACT_TANH, KUDNN_ACT_SIGMOID,
    KUDNN_ACT_POW, KUDNN_ACT_CLIP, KUDNN_ACT_CLIP_V2, KUDNN_ACT_HARDSIGMOID, KUDNN_ACT_HARDSWISH,
    KUDNN_ACT_EXP_DST, KUDNN_ACT_LOGISTIC_DST, KUDNN_ACT_TANH_DST, KUDNN_ACT_ELU,
    KUDNN_ACT_GELU_TANH = 20, KUDNN_ACT_CLIP_V2_DST, KUDNN_ACT_ELU_DST, KUDNN_ACT_RELU_DST, KUDNN_ACT_SQRT_DST,
    KUDNN_ACT_SWISH = 25, KUDNN_ACT_SRELU, KUDNN_ACT_GELU_ERF = 27, KUDNN_ACT_MISH
};

/* Residual kinds; values == KuDNN::ResOpsFunction (kudnn_linear_res.hpp:25-29). */
enum {
    KUDNN_RES_EXT = 0,       /* linearRes = C + gamma * res           (kudnn_linear_res.cpp:71-75) */
    KUDNN_RES_MUL = 1,       /* linearRes = C x res, a second GEMM    (kudnn_linear_res.cpp:188-190) */
    KUDNN_RES_IDENTIAL = 2   /* linearRes = C + res                   (kudnn_linear_res.cpp:66-70) */
};

/* Binary post-op of the post-op chain (extension; no reference counterpart, see kudnn_linear_postops_*). */
enum {
    KUDNN_BINARY_NONE = 0,
    KUDNN_BINARY_ADD = 1,    /* y = act + src           (RES_IDENTIAL arithmetic and rounding) */
    KUDNN_BINARY_EXT = 2,    /* y = act + gamma * src   (RES_EXT arithmetic and rounding)      */
    KUDNN_BINARY_MUL = 3     /* y = act * src, element-wise                                    */
};

/* POD mirror of KuDNN::TensorInfo. ndims == 0 means "no tensor" (the reference's Shape{0} sentinel,
 * kudnn_gemm.cpp:895-898). */
typedef struct kudnn_tensor_desc {
    int32_t ndims;
    int32_t dtype;
    int32_t layout;
    int32_t reserved;
    int64_t dims[KUDNN_HIP_MAX_DIMS];
    int64_t strides[KUDNN_HIP_MAX_DIMS];
} kudnn_tensor_desc;

typedef struct kudnn_gemm_plan *kudnn_gemm_t;
typedef struct kudnn_linear_act_plan *kudnn_linear_act_t;
typedef struct kudnn_linear_res_plan *kudnn_linear_res_t;
typedef struct kudnn_linear_postops_plan *kudnn_linear_postops_t;

/* ---- library ------------------------------------------------------------------------------------ */

/* Message for the last non-zero status returned on this thread ("" if none). */
KUDNN_HIP_API const char *kudnn_last_error(void);
/* Library version string. */
KUDNN_HIP_API const char *kudnn_version(void);
/* Waits for all work queued on `stream` (NULL = default stream). */
KUDNN_HIP_API int kudnn_stream_synchronize(void *stream);

/* ---- tensor descriptors --------------------------------------------------------------------------- */

/* Dense descriptor: replaces TensorInfo(shape, type, layout)
 * (kudnn_tensor_info.hpp:136-142; strides from kudnn_tensor_info.cpp:141-325). */
KUDNN_HIP_API int kudnn_tensor_desc_init(kudnn_tensor_desc *desc, int32_t ndims, const int64_t *dims,
                                         int32_t dtype, int32_t layout);
/* Strided descriptor: replaces TensorInfo(shape, type, layout, strides)
 * (kudnn_tensor_info.hpp:144-152; checks of kudnn_tensor_info.cpp:328-376). */
KUDNN_HIP_API int kudnn_tensor_desc_init_strided(kudnn_tensor_desc *desc, int32_t ndims, const int64_t *dims,
                                                 int32_t dtype, int32_t layout, const int64_t *strides);
/* 1 if the descriptor has minimum (dense) strides: TensorInfo::IsDense (kudnn_tensor_info.hpp:182-187). */
KUDNN_HIP_API int kudnn_tensor_desc_is_dense(const kudnn_tensor_desc *desc);

/* ---- threading API (accepted and validated; the GPU path does not use host threads) ----------------- */
/* Replaces KuDNN::Threading::* (kudnn_threading.hpp:29-35; semantics of threading_impl.cpp:44-175). */
KUDNN_HIP_API int kudnn_threading_get_max_num_threads(void);
KUDNN_HIP_API int kudnn_threading_set_max_num_threads(int n);
KUDNN_HIP_API int kudnn_threading_set_fixed_num_threads(int n);
KUDNN_HIP_API int kudnn_threading_set_num_threads_local(int n);
KUDNN_HIP_API int kudnn_threading_should_calculate_opt_threads(void);
KUDNN_HIP_API int kudnn_threading_set_env_mode(int mode);
KUDNN_HIP_API int kudnn_threading_get_control_status(void);

/* ---- Gemm: C = alpha * A x B + beta * C + bias ---------------------------------------------------- */
/* bias may be NULL or have ndims == 0 for "no bias". */

/* Replaces Gemm::ValidateInput (kudnn_gemm.hpp:31-34; rules of kudnn_gemm.cpp:384-476). */
KUDNN_HIP_API int kudnn_gemm_validate(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b,
                                      const kudnn_tensor_desc *c, const kudnn_tensor_desc *bias, int num_threads);
/* Replaces the Gemm constructor (kudnn_gemm.hpp:36-39, kudnn_gemm.cpp:830-857): validates and builds the
 * kernel plan (dispatcher choice, tile configuration, workspace size). */
KUDNN_HIP_API int kudnn_gemm_create(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b,
                                    const kudnn_tensor_desc *c, const kudnn_tensor_desc *bias, int num_threads,
                                    kudnn_gemm_t *plan);
/* Replaces Gemm::Run (kudnn_gemm.hpp:43-46, kudnn_gemm.cpp:859-876). */
KUDNN_HIP_API int kudnn_gemm_run(kudnn_gemm_t plan, const void *a, const void *b, void *c, const void *bias,
                                 float alpha, float beta, int num_threads, void *stream);
/* Replaces the Gemm copy constructor (kudnn_gemm.cpp:900). */
KUDNN_HIP_API int kudnn_gemm_clone(kudnn_gemm_t plan, kudnn_gemm_t *copy);
/* Replaces ~Gemm (kudnn_gemm.cpp:885). NULL is accepted. */
KUDNN_HIP_API int kudnn_gemm_destroy(kudnn_gemm_t plan);

/* ---- LinearActivationLayerFWD: C = act(A x B + bias) ---------------------------------------------- */

/* Replaces LinearActivationLayerFWD::ValidateInput (kudnn_linear_activationlayer.hpp:33-41,
 * kudnn_linear_activationlayer.cpp:115-135). */
KUDNN_HIP_API int kudnn_linear_act_validate(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b,
                                            const kudnn_tensor_desc *c, const kudnn_tensor_desc *bias, float alpha,
                                            float beta, int kind, int num_threads);
/* Replaces the LinearActivationLayerFWD constructor (kudnn_linear_activationlayer.hpp:43-51,
 * kudnn_linear_activationlayer.cpp:30-38). `alpha` is the activation parameter (RELU slope, SWISH alpha). As in the
 * reference, `beta` is only validated: the activation is built with (kind, alpha) (:33) and runs with its second
 * parameter 0, so e.g. CLIP's upper bound is 0 here; kudnn_linear_postops_* takes both parameters. */
KUDNN_HIP_API int kudnn_linear_act_create(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b,
                                          const kudnn_tensor_desc *c, const kudnn_tensor_desc *bias, float alpha,
                                          float beta, int kind, int num_threads, kudnn_linear_act_t *plan);
/* Replaces LinearActivationLayerFWD::Run (kudnn_linear_activationlayer.hpp:57-58,
 * kudnn_linear_activationlayer.cpp:40-56), fused into one kernel. */
KUDNN_HIP_API int kudnn_linear_act_run(kudnn_linear_act_t plan, const void *a, const void *b, void *c,
                                       const void *bias, int num_threads, void *stream);
KUDNN_HIP_API int kudnn_linear_act_clone(kudnn_linear_act_t plan, kudnn_linear_act_t *copy);
KUDNN_HIP_API int kudnn_linear_act_destroy(kudnn_linear_act_t plan);

/* ---- LinearResFWD: C = A x B + bias, then linearRes = C + res | C + gamma*res | C x res ------------- */

/* Replaces LinearResFWD::ValidateInput (kudnn_linear_res.hpp:39-48, kudnn_linear_res.cpp:136-166). */
KUDNN_HIP_API int kudnn_linear_res_validate(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b,
                                            const kudnn_tensor_desc *c, const kudnn_tensor_desc *bias,
                                            const kudnn_tensor_desc *res, const kudnn_tensor_desc *linear_res,
                                            int kind, int num_threads);
/* Replaces the LinearResFWD constructor (kudnn_linear_res.hpp:50-57, kudnn_linear_res.cpp:170-182). */
KUDNN_HIP_API int kudnn_linear_res_create(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b,
                                          const kudnn_tensor_desc *c, const kudnn_tensor_desc *bias,
                                          const kudnn_tensor_desc *res, const kudnn_tensor_desc *linear_res,
                                          float alpha, float beta, float gamma, int kind, int num_threads,
                                          kudnn_linear_res_t *plan);
/* Replaces LinearResFWD::Run (kudnn_linear_res.hpp:67-71, kudnn_linear_res.cpp:184-202). Writes both C and
 * linearRes, as the reference does; gamma is the Run argument (the constructor's is ignored). */
KUDNN_HIP_API int kudnn_linear_res_run(kudnn_linear_res_t plan, const void *a, const void *b, void *c,
                                       const void *bias, const void *res, void *linear_res, float gamma,
                                       int num_threads, void *stream);
KUDNN_HIP_API int kudnn_linear_res_clone(kudnn_linear_res_t plan, kudnn_linear_res_t *copy);
KUDNN_HIP_API int kudnn_linear_res_destroy(kudnn_linear_res_t plan);

/* ---- Linear with a post-op chain: Y = binary(act(A x B + bias), src) -------------------------------- */
/* Extension with no single reference counterpart: it fuses the composition LinearActivationLayerFWD
 * (kudnn_linear_activationlayer.cpp:40-56) followed by a LinearResFWD-style binary op
 * (kudnn_linear_res.cpp:57-122) or an element-wise multiply. Every stage rounds to Y's dtype exactly where
 * the composed reference ops store their outputs. act_kind == KUDNN_ACT_UNIMPLEMENTED means no activation.
 * `src` (binary operand) has Y's shape; it may be NULL/ndims 0 when binary_kind == KUDNN_BINARY_NONE. */
KUDNN_HIP_API int kudnn_linear_postops_create(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b,
                                              const kudnn_tensor_desc *y, const kudnn_tensor_desc *bias,
                                              int act_kind, float act_alpha, float act_beta, int binary_kind,
                                              const kudnn_tensor_desc *src, float gamma, int num_threads,
                                              kudnn_linear_postops_t *plan);
KUDNN_HIP_API int kudnn_linear_postops_run(kudnn_linear_postops_t plan, const void *a, const void *b, void *y,
                                           const void *bias, const void *src, float gamma, void *stream);
KUDNN_HIP_API int kudnn_linear_postops_destroy(kudnn_linear_postops_t plan);
/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): runs a plan made by kudnn_linear_postops_create exactly as
 * kudnn_linear_postops_run does (same kernels, same results), but calls no hipMalloc, hipFree or other allocating
 * routine. Its workspace (operand packs, split-K partials and arrival counters) is a static device array of 64 MiB
 * per GPU, held from library load until the process ends; a plan that needs more than 64 MiB - 512 bytes of
 * workspace (e.g. a pack of a weight larger than that) is refused with KUDNN_STATUS_UNSUPPORTED, and every buffer
 * must be device memory (host pointers: KUDNN_STATUS_BAD_ARGUMENTS). All calls on one GPU share that array: calls
 * that overlap on one GPU (several streams, or several threads) race and must be serialised by the caller. */
KUDNN_HIP_API int kudnn_linear_postops_run_noalloc(kudnn_linear_postops_t plan, const void *a, const void *b,
                                                   void *y, const void *bias, const void *src, float gamma,
                                                   void *stream);

/* ---- introspection ---------------------------------------------------------------------------------- */
/* Name of the kernel family the dispatcher chose for a plan ("mfma_bf16_256x256", "skinny_bf16_nt", ...).
 * Writes at most `len` bytes including the terminating NUL. */
KUDNN_HIP_API int kudnn_plan_describe(const void *plan, char *buf, int len);
/* Digest of the source files the ping-pong GEMM kernel was compiled from (16 hex digits; "unknown" when built
 * without one). No counterpart in the reference: it lets a measurement record say which kernel build its counters
 * came from, so counters captured from another build are not reported as this one's. */
KUDNN_HIP_API const char *kudnn_pingpong_source_digest(void);

#ifdef __cplusplus
}
#endif

#endif /* KUDNN_HIP_H */
