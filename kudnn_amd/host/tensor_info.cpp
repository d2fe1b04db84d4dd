// TensorInfo validation, Service helpers and the Threading API of the KuDNN C++ layer (libkudnn.so).
//
// Semantics restated from KuDNN: ValidateLayout (src/dnn/src/kudnn_tensor_info.cpp:59-138),
// SetMinimumRequiredStrides (:141-325), ValidateDimsAndStrides (:328-376), GetAxisNumAccordingToLayout (:20-31),
// GetIdxForUserLayout / GetShapeAccordingToLayout / FlushStrides / AlignedAlloc (src/dnn/src/service.cpp:115-435).
// The per-layout tables of KuDNN are replaced by one permutation table (layout_table.h) shared with the
// C ABI, so both layers compute identical strides.
#include <cstdlib>
#include <string>

#include "../../include/kudnn.hpp"
#include "../../include/kudnn_hip.h"
#include "../csrc/layout_table.h"

namespace KuDNN {

namespace {

template <bool NoThrow>
typename std::conditional<NoThrow, Status, void>::type Reject(const std::string &msg)
{
    if constexpr (NoThrow) {
        (void)msg;
        return Status::BAD_ARGUMENTS;
    } else {
        throw Service::LogicError{msg};
    }
}

template <bool NoThrow>
typename std::conditional<NoThrow, Status, void>::type Accept()
{
    if constexpr (NoThrow) {
        return Status::SUCCESS;
    }
}

}  // namespace

// ---------------------------------------------------------------------------------------------------
// Service

namespace Service {

SizeType GetIdxForUserLayout(Layout l, SizeType idx) noexcept(false)
{
    const kudnn_layout::Entry *e = kudnn_layout::Lookup(static_cast<int>(l));
    if (e == nullptr) {
        throw LogicError("Shape: unknown layout");
    }
    if (idx >= static_cast<SizeType>(e->ndims)) {
        throw LogicError("Shape: index >= layout size");
    }
    return static_cast<SizeType>(e->perm[idx]);
}

Shape GetShapeAccordingToLayout(const Shape &sh, Layout parLayout) noexcept
{
    SizeType arr[MAX_DIMS] = {0, 0, 0, 0, 0};
    for (SizeType i = 0; i < sh.GetNumDims(); ++i) {
        arr[i] = sh[GetIdxForUserLayout(parLayout, i)];
    }
    return Shape(arr, sh.GetNumDims());
}

Shape FlushStrides(const Shape &dims, const Shape &strides) noexcept(false)
{
    if (dims.GetNumDims() != strides.GetNumDims()) {
        throw LogicError{"FlushStrides: dims and strides have different dimensionality"};
    }
    SizeType arr[MAX_DIMS] = {0, 0, 0, 0, 0};
    for (SizeType i = 0; i < strides.GetNumDims(); ++i) {
        arr[i] = dims[i] == 1 ? 0 : strides[i];
    }
    return Shape(arr, strides.GetNumDims());
}

void *AlignedAlloc(SizeType n, SizeType alignment) noexcept(false)
{
    if (alignment == 0 || (alignment & (alignment - 1)) != 0) {
        throw LogicError("KuDNN alignment isn't a power of 2");
    }
    if (n > std::numeric_limits<SizeType>::max() - alignment) {
        throw BadArrayNewLength();
    }
    const SizeType rounded = (n + alignment - 1) / alignment * alignment;
    if (void *p = std::aligned_alloc(alignment, rounded)) {
        return p;
    }
    throw BadAlloc();
}

void Deallocate(void *p, SizeType) noexcept { std::free(p); }

}  // namespace Service

// ---------------------------------------------------------------------------------------------------
// TensorInfo

SizeType TensorInfo::GetAxisNumAccordingToLayout(SizeType axisNum) const noexcept(false)
{
    if (axisNum > dims.GetNumDims()) {
        throw Service::LogicError{"Tensor Info: axisNum > tensor dimensionality"};
    }
    for (SizeType pos = 0; pos < dims.GetNumDims(); ++pos) {
        if (Service::GetIdxForUserLayout(layout, pos) == axisNum) {
            return pos;
        }
    }
    throw Service::LogicError{"Tensor Info: axis not found in layout"};
}

template <bool NoThrow>
typename std::conditional<NoThrow, Status, void>::type
TensorInfo::ValidateElementType(Element::Type parType) noexcept(NoThrow)
{
    if (parType == Element::TypeT::UNDEFINED) {
        return Reject<NoThrow>("Tensor Info: Undefined data type of tensor");
    }
    return Accept<NoThrow>();
}

template <bool NoThrow>
typename std::conditional<NoThrow, Status, void>::type TensorInfo::ValidateLayout(Shape parDims,
                                                                                   Layout parLayout) noexcept(NoThrow)
{
    const SizeType n = parDims.GetNumDims();
    if (n < DIM_1 || n > DIM_5) {
        return Reject<NoThrow>("Tensor Info: tensor dimensionality is incorrect");
    }
    if (!kudnn_layout::IsValidFor(static_cast<int>(parLayout), static_cast<int>(n))) {
        return Reject<NoThrow>("Tensor Info: incorrect layout for " + std::to_string(n) + "D tensor");
    }
    return Accept<NoThrow>();
}

template <bool NoThrow>
typename std::conditional<NoThrow, Status, void>::type
TensorInfo::SetMinimumRequiredStrides(Shape parDims, Layout parLayout, Shape &parStrides) noexcept(NoThrow)
{
    const SizeType n = parDims.GetNumDims();
    int64_t d[MAX_DIMS] = {0, 0, 0, 0, 0};
    int64_t s[MAX_DIMS] = {0, 0, 0, 0, 0};
    for (SizeType i = 0; i < n; ++i) {
        d[i] = static_cast<int64_t>(parDims[i]);
    }
    if (!kudnn_layout::MinStrides(static_cast<int>(parLayout), static_cast<int>(n), d, s)) {
        return Reject<NoThrow>("Tensor Info: layout wasn't processed");
    }
    SizeType out[MAX_DIMS];
    for (SizeType i = 0; i < n; ++i) {
        out[i] = static_cast<SizeType>(s[i]);
    }
    parStrides.ResetShape(out, n);
    return Accept<NoThrow>();
}

template <bool NoThrow>
typename std::conditional<NoThrow, Status, void>::type
TensorInfo::ValidateDimsAndStrides(Shape parDims, Layout parLayout, Shape parStrides) noexcept(NoThrow)
{
    if (parDims.GetNumDims() != parStrides.GetNumDims()) {
        return Reject<NoThrow>("Tensor Info: dims and strides have different dimensionality");
    }
    if constexpr (NoThrow) {
        Status st = ValidateLayout<true>(parDims, parLayout);
        if (st != Status::SUCCESS) {
            return st;
        }
    } else {
        ValidateLayout<false>(parDims, parLayout);
    }
    SizeType dimsArr[MAX_DIMS] = {1, 1, 1, 1, 1};
    for (SizeType i = 0; i < parDims.GetNumDims(); ++i) {
        dimsArr[i] = parDims[i];
    }
    if (Service::WillIntMultOverflow(dimsArr, dimsArr + parDims.GetNumDims())) {
        return Reject<NoThrow>("TensorInfo: total size doesn't fit in SizeType");
    }
    Shape minStrides = parDims;
    if constexpr (NoThrow) {
        Status st = SetMinimumRequiredStrides<true>(parDims, parLayout, minStrides);
        if (st != Status::SUCCESS) {
            return st;
        }
    } else {
        SetMinimumRequiredStrides<false>(parDims, parLayout, minStrides);
    }
    for (SizeType i = 0; i < parDims.GetNumDims(); ++i) {
        if (parStrides[i] < minStrides[i]) {
            return Reject<NoThrow>("Tensor Info: incorrect strides");
        }
    }
    return Accept<NoThrow>();
}

template void TensorInfo::ValidateElementType<false>(Element::Type) noexcept(false);
template Status TensorInfo::ValidateElementType<true>(Element::Type) noexcept(true);
template void TensorInfo::ValidateLayout<false>(Shape, Layout) noexcept(false);
template Status TensorInfo::ValidateLayout<true>(Shape, Layout) noexcept(true);
template void TensorInfo::SetMinimumRequiredStrides<false>(Shape, Layout, Shape &) noexcept(false);
template Status TensorInfo::SetMinimumRequiredStrides<true>(Shape, Layout, Shape &) noexcept(true);
template void TensorInfo::ValidateDimsAndStrides<false>(Shape, Layout, Shape) noexcept(false);
template Status TensorInfo::ValidateDimsAndStrides<true>(Shape, Layout, Shape) noexcept(true);

// ---------------------------------------------------------------------------------------------------
// Threading: the state lives in libkudnn_hip.so so that the C ABI and this layer agree on numThreads checks.

namespace Threading {

bool ShouldCalculateOptThreads() noexcept { return kudnn_threading_should_calculate_opt_threads() != 0; }
int SetMaxNumThreads(int nThreads) noexcept { return kudnn_threading_set_max_num_threads(nThreads); }
int SetFixedNumThreads(int nThreads) noexcept { return kudnn_threading_set_fixed_num_threads(nThreads); }
int GetMaxNumThreads() noexcept { return kudnn_threading_get_max_num_threads(); }
int SetNumThreadsLocal(int nThreads) noexcept { return kudnn_threading_set_num_threads_local(nThreads); }
EnvMode SetEnvMode(EnvMode mode) noexcept
{
    return static_cast<EnvMode>(kudnn_threading_set_env_mode(static_cast<int>(mode)));
}
ThreadingControl GetThreadingControlStatus() noexcept
{
    return static_cast<ThreadingControl>(kudnn_threading_get_control_status());
}

}  // namespace Threading

}  // namespace KuDNN
