// TensorInfo: dims, element type, layout and per-logical-dimension strides of one tensor
// (reference: src/dnn/include/types/kudnn_tensor_info.hpp:132-289, semantics of src/dnn/src/kudnn_tensor_info.cpp).
//  - TensorInfo(shape, type, layout): dense; strides are the minimum strides of the layout with the
//    strides of size-1 dims set to 0 (implicit broadcasting).
//  - TensorInfo(shape, type, layout, strides): explicit strides, each at least the minimum stride.
// An undefined type, a layout that does not match the rank, or too-small strides throw LogicError.
#ifndef KUDNN_TENSORINFO_HPP
#define KUDNN_TENSORINFO_HPP

#include <type_traits>

#include "service/kudnn_err_codes.hpp"
#include "service/kudnn_service.hpp"
#include "types/kudnn_data_type.hpp"
#include "types/kudnn_layout.hpp"
#include "types/kudnn_shape.hpp"
#include "types/kudnn_types.hpp"

namespace KuDNN {

constexpr SizeType DIM_1 = 1;
constexpr SizeType DIM_2 = 2;
constexpr SizeType DIM_3 = 3;
constexpr SizeType DIM_4 = 4;
constexpr SizeType DIM_5 = 5;

constexpr SizeType IDX_0 = 0;
constexpr SizeType IDX_1 = 1;
constexpr SizeType IDX_2 = 2;
constexpr SizeType IDX_3 = 3;
constexpr SizeType IDX_4 = 4;
constexpr SizeType IDX_5 = 5;

struct KUDNN_API_PUBLIC TensorInfo final {
    using SizeType = ::KuDNN::SizeType;

    TensorInfo(const Shape &shape, const Element::Type &t, const Layout &l) noexcept(false)
        : dims(shape), type(t), layout(l), stridesInfo()
    {
        ValidateElementType(type);
        ValidateLayout(dims, layout);
        SetMinimumRequiredStrides(dims, layout, stridesInfo);
    }

    TensorInfo(const Shape &shape, const Element::Type &t, const Layout &l, const Shape &strides) noexcept(false)
        : dims(shape), type(t), layout(l), stridesInfo(strides)
    {
        ValidateElementType(type);
        stridesInfo = Service::FlushStrides(dims, stridesInfo);
        ValidateDimsAndStrides(dims, layout, strides);
    }

    Shape GetDims() const noexcept { return dims; }
    SizeType GetNumDims() const noexcept { return dims.GetNumDims(); }
    SizeType GetTotalTensorSize() const noexcept { return dims.GetTotalDimsSize(); }
    Shape GetStrides() const noexcept { return stridesInfo; }
    Element::Type GetType() const noexcept { return type; }
    Layout GetLayout() const noexcept { return layout; }

    // Strides equal to the layout's minimum strides.
    bool IsDense() const noexcept
    {
        Shape minStrides = dims;
        if (SetMinimumRequiredStrides<true>(dims, layout, minStrides) != Status::SUCCESS) {
            return false;
        }
        return minStrides == stridesInfo;
    }

    // The fastest physical dimension has a stride above 1.
    bool HasStrideOverFastestDim() const noexcept
    {
        return stridesInfo[Service::GetIdxForUserLayout(layout, dims.GetNumDims() - 1)] > 1;
    }

    Layout GetStandardABXLayout() const
    {
        static const Layout byRank[] = {Layout::A, Layout::AB, Layout::ABC, Layout::ABCD, Layout::ABCDE};
        return StandardFor(byRank);
    }
    Layout GetStandardAXBLayout() const
    {
        static const Layout byRank[] = {Layout::A, Layout::AB, Layout::ACB, Layout::ACDB, Layout::ACDEB};
        return StandardFor(byRank);
    }
    Layout GetStandardBXALayout() const
    {
        static const Layout byRank[] = {Layout::A, Layout::BA, Layout::BCA, Layout::BCDA, Layout::BCDEA};
        return StandardFor(byRank);
    }

    // Physical position of logical axis `axisNum` in this tensor's layout.
    SizeType GetAxisNumAccordingToLayout(SizeType axisNum) const noexcept(false);

    template <bool areExcetionsDeclined = false>
    static typename std::conditional<areExcetionsDeclined, Status, void>::type
    ValidateElementType(Element::Type parType) noexcept(areExcetionsDeclined);

    template <bool areExcetionsDeclined = false>
    static typename std::conditional<areExcetionsDeclined, Status, void>::type
    ValidateLayout(Shape parDims, Layout parLayout) noexcept(areExcetionsDeclined);

    template <bool areExcetionsDeclined = false>
    static typename std::conditional<areExcetionsDeclined, Status, void>::type
    SetMinimumRequiredStrides(Shape parDims, Layout parLayout, Shape &parStrides) noexcept(areExcetionsDeclined);

    template <bool areExcetionsDeclined = false>
    static typename std::conditional<areExcetionsDeclined, Status, void>::type
    ValidateDimsAndStrides(Shape parDims, Layout parLayout, Shape parStrides) noexcept(areExcetionsDeclined);

private:
    Layout StandardFor(const Layout (&byRank)[5]) const
    {
        const SizeType n = dims.GetNumDims();
        if (n < DIM_1 || n > DIM_5) {
            throw Service::LogicError{"Tensor Info: tensor dimensionality is incorrect"};
        }
        return byRank[n - 1];
    }

    Shape dims;
    Element::Type type;
    Layout layout;
    Shape stridesInfo;
};

inline bool operator==(const TensorInfo &lhs, const TensorInfo &rhs) noexcept
{
    return lhs.GetDims() == rhs.GetDims() &&
           static_cast<Element::TypeT>(lhs.GetType()) == static_cast<Element::TypeT>(rhs.GetType()) &&
           lhs.GetLayout() == rhs.GetLayout() && lhs.GetStrides() == rhs.GetStrides();
}

inline bool operator!=(const TensorInfo &lhs, const TensorInfo &rhs) noexcept { return !(lhs == rhs); }

}  // namespace KuDNN

#endif  // KUDNN_TENSORINFO_HPP
