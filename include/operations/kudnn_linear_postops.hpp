// LinearPostOpsFWD (MI355X addition, no KuDNN counterpart): Y = binary(act(A x B + bias), src) in one kernel.
//
// It fuses what a KuDNN caller writes as LinearActivationLayerFWD followed by an element-wise pass
// (LinearResFWD's RES_IDENTIAL / RES_EXT arithmetic, or an element-wise multiply that KuDNN does not offer:
// its RES_MUL is a matrix product). Each stage rounds to Y's type exactly where the composed KuDNN
// operators store their outputs, so the result equals the composition's.
//  act    ActivationFunction::UNIMPLEMENTED = none, or RELU / SWISH / GELU_TANH / GELU_ERF
//  binary NONE, ADD (y = a + src), EXT (y = a + gamma * src), MUL (y = a * src, element-wise)
#ifndef KUDNN_LINEAR_POSTOPS_HPP
#define KUDNN_LINEAR_POSTOPS_HPP

#include <memory>

#include "operations/kudnn_eltwise.hpp"
#include "service/kudnn_err_codes.hpp"
#include "types/kudnn_tensor_info.hpp"

namespace KuDNN {

enum class BinaryPostOp { NONE = 0, ADD = 1, EXT = 2, MUL = 3 };

namespace Detail {
class LinearPostOpsFWDImpl;
}  // namespace Detail

class KUDNN_API_PUBLIC LinearPostOpsFWD final {
public:
    // biasInfo / srcInfo with total size 0 mean "none".
    LinearPostOpsFWD(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &yInfo,
                     const TensorInfo &biasInfo, ActivationFunction act, float actAlpha, BinaryPostOp binary,
                     const TensorInfo &srcInfo, int numThreads = 0) noexcept(false);
    LinearPostOpsFWD(const LinearPostOpsFWD &other) = delete;
    LinearPostOpsFWD(LinearPostOpsFWD &&other) noexcept;
    LinearPostOpsFWD &operator=(LinearPostOpsFWD &&other) noexcept;
    void Run(const void *a, const void *b, void *y, const void *bias, const void *src, float gamma = 1.0f,
             void *stream = nullptr) const noexcept(false);
    ~LinearPostOpsFWD() noexcept;

private:
    std::unique_ptr<Detail::LinearPostOpsFWDImpl> pImpl;
};

}  // namespace KuDNN

#endif  // KUDNN_LINEAR_POSTOPS_HPP
