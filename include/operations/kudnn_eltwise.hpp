// Activation kinds of the KuDNN C++ API (same enumerators and order as KuDNN's ActivationFunction,
// src/dnn/include/operations/kudnn_eltwise.hpp:24-54; values == KUDNN_ACT_* of kudnn_hip.h).
//
// On the MI355X path activations are fused into the Linear/GEMM epilogue: LinearActivationLayerFWD runs
// RELU, SWISH, GELU_TANH and GELU_ERF inside the GEMM kernel. The stand-alone ActivationLayerFWD/BWD
// operators of KuDNN are not part of this build.
#ifndef KUDNN_ELTWISE_HPP
#define KUDNN_ELTWISE_HPP

namespace KuDNN {

enum class ActivationFunction {
    UNIMPLEMENTED,
    ABS,
    EXP,
    LINEAR,
    LOG,
    RELU,
    ROUND,
    SQRT,
    SQUARE,
    TANH,
    SIGMOID,
    POW,
    CLIP,
    CLIP_V2,
    HARDSIGMOID,
    HARDSWISH,
    EXP_DST,
    LOGISTIC_DST,
    TANH_DST,
    ELU,
    GELU_TANH,
    CLIP_V2_DST,
    ELU_DST,
    RELU_DST,
    SQRT_DST,
    SWISH,
    SRELU,
    GELU_ERF,
    MISH
};

}  // namespace KuDNN

#endif  // KUDNN_ELTWISE_HPP
