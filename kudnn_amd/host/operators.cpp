// KuDNN operator classes (Gemm, LinearActivationLayerFWD, LinearResFWD, LinearPostOpsFWD) on top of the
// C ABI of libkudnn_hip.so.
//
// Each class's pImpl owns one C ABI plan: the constructor builds it (validation + dispatcher decision),
// Run executes it, copy clones it, the destructor frees it. Non-zero C ABI statuses become the exceptions
// KuDNN throws (Service::ThrowOnStatus, src/dnn/src/service.cpp:32-46):
//   UNSUPPORTED -> Service::Unsupported, BAD_ARGUMENTS / null pointers -> Service::LogicError,
//   allocation failure -> Service::BadAlloc, HIP runtime errors -> std::runtime_error.
#include <cstring>
#include <string>

#include "../../include/kudnn.hpp"
#include "../../include/kudnn_hip.h"

namespace KuDNN {

namespace {

kudnn_tensor_desc ToDesc(const TensorInfo &t)
{
    kudnn_tensor_desc d;
    std::memset(&d, 0, sizeof(d));
    const Shape dims = t.GetDims();
    const Shape strides = t.GetStrides();
    d.ndims = static_cast<int32_t>(dims.GetNumDims());
    d.dtype = static_cast<int32_t>(static_cast<Element::TypeT>(t.GetType()));
    d.layout = static_cast<int32_t>(t.GetLayout());
    for (SizeType i = 0; i < dims.GetNumDims(); ++i) {
        d.dims[i] = static_cast<int64_t>(dims[i]);
        d.strides[i] = i < strides.GetNumDims() ? static_cast<int64_t>(strides[i]) : 0;
    }
    return d;
}

// KuDNN's "no bias" descriptor: a 1-D tensor of size 0 (kudnn_gemm.cpp:895-898).
TensorInfo NoTensor(const TensorInfo &like) { return TensorInfo(Shape{0}, like.GetType(), Layout::A); }

Status ToStatus(int s) noexcept
{
    switch (s) {
        case KUDNN_STATUS_SUCCESS: return Status::SUCCESS;
        case KUDNN_STATUS_UNSUPPORTED: return Status::UNSUPPORTED;
        default: return Status::BAD_ARGUMENTS;
    }
}

void Check(int s)
{
    switch (s) {
        case KUDNN_STATUS_SUCCESS: return;
        case KUDNN_STATUS_UNSUPPORTED: throw Service::Unsupported{kudnn_last_error()};
        case KUDNN_STATUS_BAD_ARGUMENTS:
        case KUDNN_STATUS_NULL_POINTER: throw Service::LogicError{kudnn_last_error()};
        case KUDNN_STATUS_ALLOC_FAILED: throw Service::BadAlloc{};
        default: throw std::runtime_error{kudnn_last_error()};
    }
}

// Owner of one C ABI plan handle.
template <typename H, int (*Clone)(H, H *), int (*Destroy)(H)>
class Plan {
public:
    Plan() = default;
    Plan(const Plan &o) : h(nullptr)
    {
        if (o.h != nullptr) {
            Check(Clone(o.h, &h));
        }
    }
    Plan &operator=(const Plan &) = delete;
    ~Plan() { Destroy(h); }
    H h = nullptr;
};

int NoClone(kudnn_linear_postops_t, kudnn_linear_postops_t *) { return KUDNN_STATUS_UNSUPPORTED; }

}  // namespace

namespace Detail {

class GemmImpl final {
public:
    GemmImpl(const TensorInfo &a, const TensorInfo &b, const TensorInfo &c, const TensorInfo &bias, int numThreads)
    {
        const kudnn_tensor_desc da = ToDesc(a), db = ToDesc(b), dc = ToDesc(c), dbias = ToDesc(bias);
        Check(kudnn_gemm_create(&da, &db, &dc, &dbias, numThreads, &plan.h));
    }
    void Run(const void *a, const void *b, void *c, const void *bias, float alpha, float beta, int numThreads,
             void *stream) const
    {
        Check(kudnn_gemm_run(plan.h, a, b, c, bias, alpha, beta, numThreads, stream));
    }

private:
    Plan<kudnn_gemm_t, kudnn_gemm_clone, kudnn_gemm_destroy> plan;
};

class LinearActivationLayerFWDImpl final {
public:
    LinearActivationLayerFWDImpl(const TensorInfo &a, const TensorInfo &b, const TensorInfo &c, const TensorInfo &bias,
                                 float alpha, float beta, ActivationFunction kind, int numThreads)
    {
        const kudnn_tensor_desc da = ToDesc(a), db = ToDesc(b), dc = ToDesc(c), dbias = ToDesc(bias);
        Check(kudnn_linear_act_create(&da, &db, &dc, &dbias, alpha, beta, static_cast<int>(kind), numThreads,
                                      &plan.h));
    }
    void Run(const void *a, const void *b, void *c, const void *bias, int numThreads, void *stream) const
    {
        Check(kudnn_linear_act_run(plan.h, a, b, c, bias, numThreads, stream));
    }

private:
    Plan<kudnn_linear_act_t, kudnn_linear_act_clone, kudnn_linear_act_destroy> plan;
};

class LinearResFWDImpl final {
public:
    LinearResFWDImpl(const TensorInfo &a, const TensorInfo &b, const TensorInfo &c, const TensorInfo &bias,
                     const TensorInfo &res, const TensorInfo &lr, float alpha, float beta, float gamma,
                     ResOpsFunction kind, int numThreads)
    {
        const kudnn_tensor_desc da = ToDesc(a), db = ToDesc(b), dc = ToDesc(c), dbias = ToDesc(bias),
                                dres = ToDesc(res), dlr = ToDesc(lr);
        Check(kudnn_linear_res_create(&da, &db, &dc, &dbias, &dres, &dlr, alpha, beta, gamma, static_cast<int>(kind),
                                      numThreads, &plan.h));
    }
    void Run(const void *a, const void *b, void *c, const void *bias, const void *res, void *lr, float gamma,
             int numThreads, void *stream) const
    {
        Check(kudnn_linear_res_run(plan.h, a, b, c, bias, res, lr, gamma, numThreads, stream));
    }

private:
    Plan<kudnn_linear_res_t, kudnn_linear_res_clone, kudnn_linear_res_destroy> plan;
};

class LinearPostOpsFWDImpl final {
public:
    LinearPostOpsFWDImpl(const TensorInfo &a, const TensorInfo &b, const TensorInfo &y, const TensorInfo &bias,
                         ActivationFunction act, float actAlpha, BinaryPostOp binary, const TensorInfo &src,
                         int numThreads)
    {
        const kudnn_tensor_desc da = ToDesc(a), db = ToDesc(b), dy = ToDesc(y), dbias = ToDesc(bias),
                                dsrc = ToDesc(src);
        Check(kudnn_linear_postops_create(&da, &db, &dy, &dbias, static_cast<int>(act), actAlpha, 0.0f,
                                          static_cast<int>(binary), &dsrc, 1.0f, numThreads, &plan.h));
    }
    void Run(const void *a, const void *b, void *y, const void *bias, const void *src, float gamma, void *stream) const
    {
        Check(kudnn_linear_postops_run(plan.h, a, b, y, bias, src, gamma, stream));
    }

private:
    Plan<kudnn_linear_postops_t, NoClone, kudnn_linear_postops_destroy> plan;
};

}  // namespace Detail

// ---------------------------------------------------------------------------------------------------
// Gemm (kudnn_gemm.hpp)

Status Gemm::ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                           const TensorInfo &biasInfo, int numThreads) noexcept
{
    const kudnn_tensor_desc da = ToDesc(aInfo), db = ToDesc(bInfo), dc = ToDesc(cInfo), dbias = ToDesc(biasInfo);
    return ToStatus(kudnn_gemm_validate(&da, &db, &dc, &dbias, numThreads));
}

Status Gemm::ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                           int numThreads) noexcept
{
    const kudnn_tensor_desc da = ToDesc(aInfo), db = ToDesc(bInfo), dc = ToDesc(cInfo);
    return ToStatus(kudnn_gemm_validate(&da, &db, &dc, nullptr, numThreads));
}

Gemm::Gemm(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo, const TensorInfo &biasInfo,
           int numThreads) noexcept(false)
    : pImpl(new Detail::GemmImpl(aInfo, bInfo, cInfo, biasInfo, numThreads))
{
}

Gemm::Gemm(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo, int numThreads) noexcept(false)
    : Gemm(aInfo, bInfo, cInfo, NoTensor(cInfo), numThreads)
{
}

Gemm::Gemm(const Gemm &other) noexcept(false) : pImpl(new Detail::GemmImpl(*other.pImpl)) {}
Gemm::Gemm(Gemm &&other) noexcept : pImpl(std::move(other.pImpl)) {}

Gemm &Gemm::operator=(const Gemm &other) noexcept(false)
{
    if (this != &other) {
        pImpl.reset(new Detail::GemmImpl(*other.pImpl));
    }
    return *this;
}

Gemm &Gemm::operator=(Gemm &&other) noexcept
{
    if (this != &other) {
        pImpl = std::move(other.pImpl);
    }
    return *this;
}

void Gemm::Run(const void *a, const void *b, void *c, const void *bias, float alpha, float beta, int numThreads) const
    noexcept(false)
{
    pImpl->Run(a, b, c, bias, alpha, beta, numThreads, nullptr);
}

void Gemm::Run(const void *a, const void *b, void *c, float alpha, float beta, int numThreads) const noexcept(false)
{
    pImpl->Run(a, b, c, nullptr, alpha, beta, numThreads, nullptr);
}

void Gemm::RunAsync(const void *a, const void *b, void *c, const void *bias, float alpha, float beta,
                    void *stream) const noexcept(false)
{
    pImpl->Run(a, b, c, bias, alpha, beta, 0, stream);
}

Gemm::~Gemm() noexcept {}

// ---------------------------------------------------------------------------------------------------
// LinearActivationLayerFWD (kudnn_linear_activationlayer.hpp)

Status LinearActivationLayerFWD::ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo,
                                               const TensorInfo &cInfo, const TensorInfo &biasInfo, float alpha,
                                               float beta, ActivationFunction kind, int numThreads) noexcept(false)
{
    const kudnn_tensor_desc da = ToDesc(aInfo), db = ToDesc(bInfo), dc = ToDesc(cInfo), dbias = ToDesc(biasInfo);
    return ToStatus(kudnn_linear_act_validate(&da, &db, &dc, &dbias, alpha, beta, static_cast<int>(kind), numThreads));
}

Status LinearActivationLayerFWD::ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo,
                                               const TensorInfo &cInfo, float alpha, float beta,
                                               ActivationFunction kind, int numThreads) noexcept(false)
{
    return ValidateInput(aInfo, bInfo, cInfo, NoTensor(cInfo), alpha, beta, kind, numThreads);
}

LinearActivationLayerFWD::LinearActivationLayerFWD(const TensorInfo &aInfo, const TensorInfo &bInfo,
                                                   const TensorInfo &cInfo, const TensorInfo &biasInfo, float alpha,
                                                   float beta, ActivationFunction kind, int numThreads) noexcept(false)
    : pImpl(new Detail::LinearActivationLayerFWDImpl(aInfo, bInfo, cInfo, biasInfo, alpha, beta, kind, numThreads))
{
}

LinearActivationLayerFWD::LinearActivationLayerFWD(const TensorInfo &aInfo, const TensorInfo &bInfo,
                                                   const TensorInfo &cInfo, float alpha, float beta,
                                                   ActivationFunction kind, int numThreads) noexcept(false)
    : LinearActivationLayerFWD(aInfo, bInfo, cInfo, NoTensor(cInfo), alpha, beta, kind, numThreads)
{
}

LinearActivationLayerFWD::LinearActivationLayerFWD(const LinearActivationLayerFWD &other) noexcept(false)
    : pImpl(new Detail::LinearActivationLayerFWDImpl(*other.pImpl))
{
}

LinearActivationLayerFWD::LinearActivationLayerFWD(LinearActivationLayerFWD &&other) noexcept
    : pImpl(std::move(other.pImpl))
{
}

LinearActivationLayerFWD &LinearActivationLayerFWD::operator=(const LinearActivationLayerFWD &other) noexcept(false)
{
    if (this != &other) {
        pImpl.reset(new Detail::LinearActivationLayerFWDImpl(*other.pImpl));
    }
    return *this;
}

LinearActivationLayerFWD &LinearActivationLayerFWD::operator=(LinearActivationLayerFWD &&other) noexcept
{
    if (this != &other) {
        pImpl = std::move(other.pImpl);
    }
    return *this;
}

void LinearActivationLayerFWD::Run(const void *a, const void *b, void *c, const void *bias, int numThreads) const
    noexcept(false)
{
    pImpl->Run(a, b, c, bias, numThreads, nullptr);
}

void LinearActivationLayerFWD::Run(const void *a, const void *b, void *c, int numThreads) const noexcept(false)
{
    pImpl->Run(a, b, c, nullptr, numThreads, nullptr);
}

void LinearActivationLayerFWD::RunAsync(const void *a, const void *b, void *c, const void *bias, void *stream) const
    noexcept(false)
{
    pImpl->Run(a, b, c, bias, 0, stream);
}

LinearActivationLayerFWD::~LinearActivationLayerFWD() noexcept {}

// ---------------------------------------------------------------------------------------------------
// LinearResFWD (kudnn_linear_res.hpp)

Status LinearResFWD::ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                                   const TensorInfo &biasInfo, const TensorInfo &resInfo,
                                   const TensorInfo &linearResInfo, float, float, float, ResOpsFunction kind,
                                   int numThreads) noexcept(false)
{
    const kudnn_tensor_desc da = ToDesc(aInfo), db = ToDesc(bInfo), dc = ToDesc(cInfo), dbias = ToDesc(biasInfo),
                            dres = ToDesc(resInfo), dlr = ToDesc(linearResInfo);
    return ToStatus(kudnn_linear_res_validate(&da, &db, &dc, &dbias, &dres, &dlr, static_cast<int>(kind), numThreads));
}

Status LinearResFWD::ValidateInput(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                                   const TensorInfo &res, const TensorInfo &linearRes, float alpha, float beta,
                                   float gamma, ResOpsFunction kind, int numThreads) noexcept(false)
{
    return ValidateInput(aInfo, bInfo, cInfo, NoTensor(cInfo), res, linearRes, alpha, beta, gamma, kind, numThreads);
}

LinearResFWD::LinearResFWD(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                           const TensorInfo &biasInfo, const TensorInfo &res, const TensorInfo &linearRes, float alpha,
                           float beta, float gamma, ResOpsFunction kind, int numThreads) noexcept(false)
    : pImpl(new Detail::LinearResFWDImpl(aInfo, bInfo, cInfo, biasInfo, res, linearRes, alpha, beta, gamma, kind,
                                         numThreads))
{
}

LinearResFWD::LinearResFWD(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &cInfo,
                           const TensorInfo &res, const TensorInfo &linearRes, float alpha, float beta, float gamma,
                           ResOpsFunction kind, int numThreads) noexcept(false)
    : LinearResFWD(aInfo, bInfo, cInfo, NoTensor(cInfo), res, linearRes, alpha, beta, gamma, kind, numThreads)
{
}

LinearResFWD::LinearResFWD(const LinearResFWD &other) noexcept(false) : pImpl(new Detail::LinearResFWDImpl(*other.pImpl))
{
}

LinearResFWD::LinearResFWD(LinearResFWD &&other) noexcept : pImpl(std::move(other.pImpl)) {}

LinearResFWD &LinearResFWD::operator=(const LinearResFWD &other) noexcept(false)
{
    if (this != &other) {
        pImpl.reset(new Detail::LinearResFWDImpl(*other.pImpl));
    }
    return *this;
}

LinearResFWD &LinearResFWD::operator=(LinearResFWD &&other) noexcept
{
    if (this != &other) {
        pImpl = std::move(other.pImpl);
    }
    return *this;
}

void LinearResFWD::Run(const void *a, const void *b, void *c, const void *bias, const void *res, void *linearRes,
                       float gamma, int numThreads) const noexcept(false)
{
    pImpl->Run(a, b, c, bias, res, linearRes, gamma, numThreads, nullptr);
}

void LinearResFWD::Run(const void *a, const void *b, void *c, const void *res, void *linearRes, float gamma,
                       int numThreads) const noexcept(false)
{
    pImpl->Run(a, b, c, nullptr, res, linearRes, gamma, numThreads, nullptr);
}

void LinearResFWD::RunAsync(const void *a, const void *b, void *c, const void *bias, const void *res, void *linearRes,
                            float gamma, void *stream) const noexcept(false)
{
    pImpl->Run(a, b, c, bias, res, linearRes, gamma, 0, stream);
}

LinearResFWD::~LinearResFWD() noexcept {}

// ---------------------------------------------------------------------------------------------------
// LinearPostOpsFWD (kudnn_linear_postops.hpp)

LinearPostOpsFWD::LinearPostOpsFWD(const TensorInfo &aInfo, const TensorInfo &bInfo, const TensorInfo &yInfo,
                                   const TensorInfo &biasInfo, ActivationFunction act, float actAlpha,
                                   BinaryPostOp binary, const TensorInfo &srcInfo, int numThreads) noexcept(false)
    : pImpl(new Detail::LinearPostOpsFWDImpl(aInfo, bInfo, yInfo, biasInfo, act, actAlpha, binary, srcInfo, numThreads))
{
}

LinearPostOpsFWD::LinearPostOpsFWD(LinearPostOpsFWD &&other) noexcept : pImpl(std::move(other.pImpl)) {}

LinearPostOpsFWD &LinearPostOpsFWD::operator=(LinearPostOpsFWD &&other) noexcept
{
    if (this != &other) {
        pImpl = std::move(other.pImpl);
    }
    return *this;
}

void LinearPostOpsFWD::Run(const void *a, const void *b, void *y, const void *bias, const void *src, float gamma,
                           void *stream) const noexcept(false)
{
    pImpl->Run(a, b, y, bias, src, gamma, stream);
}

LinearPostOpsFWD::~LinearPostOpsFWD() noexcept {}

}  // namespace KuDNN
