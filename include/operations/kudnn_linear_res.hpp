// LinearResFWD: C = A x B + bias, then linearRes = C + res (RES_IDENTIAL), C + gamma * res (RES_EXT) or the
// matrix product C x res (RES_MUL). Same class and signatures as KuDNN
// (src/dnn/include/operations/kudnn_linear_res.hpp:25-77). Both C and linearRes are written, as in KuDNN;
// gamma is the Run argument (the constructor's gamma is ignored, as in KuDNN).
// On the MI355X path RES_IDENTIAL / RES_EXT are fused into the GEMM epilogue (one kernel writes C and
// linearRes); RES_MUL runs the second GEMM on the same kernels.
#ifndef KUDNN_LINEAR_RES_H
#define KUDNN_LINEAR_RES_H

#include <memory>

#include "operations/kudnn_gemm.hpp"
#include "service/kudnn_err_codes.hpp"
#include "types/kudnn_tensor_info.hpp"

namespace KuDNN {

enum class ResOpsFunction { RES_EXT, RES_MUL, RES_IDENTIAL };

namespace Detail {
class LinearResFWDImpl;
}  // namespace Detail

class KUDNN_API_PUBLIC LinearResFWD final {
public:
    using SizeType = ::KuDNN::SizeType;
    static Status ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                                const TensorInfo &biasInfo, const TensorInfo &resInfo, const TensorInfo &linearResInfo,
                                float alpha = 1.0f, float beta = 0.0f, float gamma = 1.0f,
                                ResOpsFunction kind = ResOpsFunction::RES_IDENTIAL, int numThreads = 0) noexcept(false);
    static Status ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                                const TensorInfo &res, const TensorInfo &linearRes, float alpha = 1.0f,
                                float beta = 0.0f, float gamma = 1.0f,
                                ResOpsFunction kind = ResOpsFunction::RES_IDENTIAL, int numThreads = 0) noexcept(false);
    LinearResFWD(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo, const TensorInfo &biasInfo,
                 const TensorInfo &res, const TensorInfo &linearRes, float alpha = 1.0f, float beta = 0.0f,
                 float gamma = 1.0f, ResOpsFunction kind = ResOpsFunction::RES_IDENTIAL,
                 int numThreads = 0) noexcept(false);
    LinearResFWD(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo, const TensorInfo &res,
                 const TensorInfo &linearRes, float alpha = 1.0f, float beta = 0.0f, float gamma = 1.0f,
                 ResOpsFunction kind = ResOpsFunction::RES_IDENTIAL, int numThreads = 0) noexcept(false);
    LinearResFWD(const LinearResFWD &other) noexcept(false);
    LinearResFWD(LinearResFWD &&other) noexcept;
    LinearResFWD &operator=(const LinearResFWD &other) noexcept(false);
    LinearResFWD &operator=(LinearResFWD &&other) noexcept;
    void Run(const void *a, const void *b, void *c, const void *bias, const void *res, void *linearRes,
             float gamma = 1.0f, int numThreads = 0) const noexcept(false);
    void Run(const void *a, const void *b, void *c, const void *res, void *linearRes, float gamma = 1.0f,
             int numThreads = 0) const noexcept(false);
    // MI355X addition: Run ordered on `stream` (a hipStream_t; nullptr = default stream).
    void RunAsync(const void *a, const void *b, void *c, const void *bias, const void *res, void *linearRes,
                  float gamma, void *stream) const noexcept(false);
    ~LinearResFWD() noexcept;

private:
    std::unique_ptr<Detail::LinearResFWDImpl> pImpl;
};

}  // namespace KuDNN

#endif  // KUDNN_LINEAR_RES_H
