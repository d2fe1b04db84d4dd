// Gemm: C = alpha * A x B + beta * C (+ bias), with up to three broadcast batch dims.
// Same class and signatures as KuDNN (src/dnn/include/operations/kudnn_gemm.hpp:29-51).
//
// MI355X semantics: the constructor validates the descriptors (KuDNN's rules) and builds the GPU plan once
// (kernel family, tile configuration, operand packing). Run launches it. Pointers may be device memory
// (hipMalloc; Run then returns before the GPU finishes, ordered on the default stream) or host memory
// (staged through device buffers; Run then returns with the result in place, as KuDNN does).
// RunAsync is the same call ordered on an explicit hipStream_t (passed as void*).
// numThreads is validated (0 <= numThreads <= Threading::GetMaxNumThreads()) and otherwise unused.
#ifndef KUDNN_GEMM_HPP
#define KUDNN_GEMM_HPP

#include <memory>

#include "service/kudnn_err_codes.hpp"
#include "types/kudnn_tensor_info.hpp"

namespace KuDNN {

namespace Detail {
class GemmImpl;
}  // namespace Detail

class KUDNN_API_PUBLIC Gemm final {
public:
    using SizeType = ::KuDNN::SizeType;
    static Status ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                                const TensorInfo &biasInfo, int numThreads = 0) noexcept;
    static Status ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                                int numThreads = 0) noexcept;
    Gemm(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo, const TensorInfo &biasInfo,
         int numThreads = 0) noexcept(false);
    Gemm(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo, int numThreads = 0) noexcept(false);
    Gemm(const Gemm &other) noexcept(false);
    Gemm(Gemm &&other) noexcept;
    Gemm &operator=(const Gemm &other) noexcept(false);
    Gemm &operator=(Gemm &&other) noexcept;
    void Run(const void *a, const void *b, void *c, const void *bias, float alpha = 1.0f, float beta = 0.0f,
             int numThreads = 0) const noexcept(false);
    void Run(const void *a, const void *b, void *c, float alpha = 1.0f, float beta = 0.0f, int numThreads = 0) const
        noexcept(false);
    // MI355X addition: Run ordered on `stream` (a hipStream_t; nullptr = default stream).
    void RunAsync(const void *a, const void *b, void *c, const void *bias, float alpha, float beta,
                  void *stream) const noexcept(false);
    ~Gemm() noexcept;

private:
    std::unique_ptr<Detail::GemmImpl> pImpl;
};

}  // namespace KuDNN

#endif  // KUDNN_GEMM_HPP
