// LinearActivationLayerFWD: C = act(A x B + bias), act in {RELU, SWISH, GELU_TANH, GELU_ERF} fused into the
// GEMM epilogue. Same class and signatures as KuDNN (src/dnn/include/operations/kudnn_linear_activationlayer.hpp:31-63).
// `alpha` is the activation parameter (RELU negative slope, SWISH x*sigmoid(alpha*x)); beta is validated only.
// Rounding follows KuDNN's separate passes: the GEMM result is stored in C's type (round to nearest even),
// the activation is computed in fp32 from that value and a bf16 result is truncated.
// Other ActivationFunction kinds that KuDNN's eltwise layer accepts throw Unsupported here.
#ifndef KUDNN_LINEAR_ACTIVATIONLAYER_HPP
#define KUDNN_LINEAR_ACTIVATIONLAYER_HPP

#include <memory>

#include "operations/kudnn_eltwise.hpp"
#include "operations/kudnn_gemm.hpp"
#include "service/kudnn_err_codes.hpp"
#include "types/kudnn_tensor_info.hpp"

namespace KuDNN {

namespace Detail {
class LinearActivationLayerFWDImpl;
}  // namespace Detail

class KUDNN_API_PUBLIC LinearActivationLayerFWD final {
public:
    using SizeType = ::KuDNN::SizeType;
    static Status ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                                const TensorInfo &biasInfo, float alpha = 1.0f, float beta = 0.0f,
                                ActivationFunction kind = KuDNN::ActivationFunction::RELU,
                                int numThreads = 0) noexcept(false);
    static Status ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                                float alpha = 1.0f, float beta = 0.0f,
                                ActivationFunction kind = KuDNN::ActivationFunction::RELU,
                                int numThreads = 0) noexcept(false);
    LinearActivationLayerFWD(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                             const TensorInfo &biasInfo, float alpha = 1.0f, float beta = 0.0f,
                             ActivationFunction kind = KuDNN::ActivationFunction::RELU,
                             int numThreads = 0) noexcept(false);
    LinearActivationLayerFWD(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                             float alpha = 1.0f, float beta = 0.0f,
                             ActivationFunction kind = KuDNN::ActivationFunction::RELU,
                             int numThreads = 0) noexcept(false);
    LinearActivationLayerFWD(const LinearActivationLayerFWD &other) noexcept(false);
    LinearActivationLayerFWD(LinearActivationLayerFWD &&other) noexcept;
    LinearActivationLayerFWD &operator=(const LinearActivationLayerFWD &other) noexcept(false);
    LinearActivationLayerFWD &operator=(LinearActivationLayerFWD &&other) noexcept;
    void Run(const void *a, const void *b, void *c, const void *bias, int numThreads = 0) const noexcept(false);
    // Declared but never defined in KuDNN (a call fails to link there); here it is the no-bias Run.
    void Run(const void *a, const void *b, void *c, int numThreads = 0) const noexcept(false);
    // MI355X addition: Run ordered on `stream` (a hipStream_t; nullptr = default stream).
    void RunAsync(const void *a, const void *b, void *c, const void *bias, void *stream) const noexcept(false);
    ~LinearActivationLayerFWD() noexcept;

private:
    std::unique_ptr<Detail::LinearActivationLayerFWDImpl> pImpl;
};

}  // namespace KuDNN

#endif  // KUDNN_LINEAR_ACTIVATIONLAYER_HPP
