// Shape: up to five dimension sizes (reference: src/dnn/include/types/kudnn_shape.hpp:25-177).
// Behaviour kept from KuDNN: more than five dims throws LogicError; the variadic constructor throws when
// the element count times 4 bytes exceeds 3 GiB or the product overflows; indexing past the rank throws.
#ifndef KUDNN_SHAPE_HPP
#define KUDNN_SHAPE_HPP

#include <array>
#include <initializer_list>

#include "service/kudnn_exception.hpp"
#include "service/kudnn_service.hpp"
#include "types/kudnn_types.hpp"

namespace KuDNN {

constexpr SizeType MAX_DIMS = 5;

struct Shape final {
    using SizeType = ::KuDNN::SizeType;
    static constexpr SizeType NUM_MAX_DIMENSIONS = MAX_DIMS;

    Shape() noexcept : dimsArray{}, numDims{0} {}

    template <typename T>
    Shape(T *ptr, const SizeType size) noexcept(false) : dimsArray{}, numDims(0)
    {
        ResetShape(ptr, size);
    }

    template <typename... Ts>
    Shape(Ts... dims) noexcept(false) : dimsArray{}, numDims(sizeof...(dims))
    {
        CheckNumDims(sizeof...(dims));
        const SizeType vals[] = {static_cast<SizeType>(dims)...};
        for (SizeType i = 0; i < numDims; ++i) {
            dimsArray[i] = vals[i];
        }
        CheckMemoryLimit();
    }

    Shape(const std::initializer_list<SizeType> &list) noexcept(false) : dimsArray{}, numDims(0) { ResetShape(list); }

    template <typename... Ts>
    Shape &ResetShape(Ts... dims) noexcept(false)
    {
        return ResetShape(std::initializer_list<SizeType>{static_cast<SizeType>(dims)...});
    }

    Shape &ResetShape(const std::initializer_list<SizeType> &list) noexcept(false)
    {
        CheckNumDims(list.size());
        dimsArray = {};
        numDims = list.size();
        SizeType i = 0;
        for (SizeType v : list) {
            dimsArray[i++] = v;
        }
        return *this;
    }

    template <typename T>
    Shape &ResetShape(T *ptr, const SizeType size) noexcept(false)
    {
        if (ptr == nullptr) {
            throw Service::LogicError("Shape: ptr is nullptr");
        }
        CheckNumDims(size);
        dimsArray = {};
        numDims = size;
        for (SizeType i = 0; i < size; ++i) {
            dimsArray[i] = static_cast<SizeType>(ptr[i]);
        }
        return *this;
    }

    Shape &operator+=(const Shape &adder) noexcept(false)
    {
        if (adder.GetNumDims() != numDims) {
            throw Service::LogicError("Shape: different size of base and adder shapes");
        }
        for (SizeType i = 0; i < numDims; ++i) {
            dimsArray[i] += adder[i];
        }
        return *this;
    }

    Shape operator+(const Shape &adder) noexcept(false)
    {
        Shape r = *this;
        r += adder;
        return r;
    }

    SizeType operator[](SizeType id) const noexcept(false)
    {
        if (id >= numDims) {
            throw Service::LogicError("Shape: index >= num_dims");
        }
        return dimsArray[id];
    }

    SizeType &operator[](SizeType id) noexcept(false)
    {
        if (id >= numDims) {
            throw Service::LogicError("Shape: index >= num_dims");
        }
        return dimsArray[id];
    }

    SizeType GetNumDims() const noexcept { return numDims; }

    SizeType GetTotalDimsSize() const noexcept(false)
    {
        if (Service::WillIntMultOverflow(dimsArray.begin(), dimsArray.begin() + numDims)) {
            throw Service::LogicError("Shape: computing total size will cause overflow");
        }
        SizeType n = 1;
        for (SizeType i = 0; i < numDims; ++i) {
            n *= dimsArray[i];
        }
        return n;
    }

private:
    static void CheckNumDims(SizeType n) noexcept(false)
    {
        if (n > NUM_MAX_DIMENSIONS) {
            throw Service::LogicError("Shape: dims is greater than NUM_MAX_DIMENSIONS");
        }
    }
    // A single tensor may not exceed 3 GiB of 4-byte elements (signed arithmetic, as in KuDNN).
    void CheckMemoryLimit() const noexcept(false)
    {
        const long long total = static_cast<long long>(GetTotalDimsSize());
        const long long limit = 3LL * 1024 * 1024 * 1024;
        if (total * 4 > limit) {
            throw Service::LogicError("Shape: exceeded available memory limit ");
        }
    }
    std::array<SizeType, NUM_MAX_DIMENSIONS> dimsArray;
    SizeType numDims;
};

inline bool operator==(const Shape &lhs, const Shape &rhs) noexcept
{
    if (lhs.GetNumDims() != rhs.GetNumDims()) {
        return false;
    }
    for (SizeType i = 0; i < lhs.GetNumDims(); ++i) {
        if (lhs[i] != rhs[i]) {
            return false;
        }
    }
    return true;
}

inline bool operator!=(const Shape &lhs, const Shape &rhs) noexcept { return !(lhs == rhs); }

}  // namespace KuDNN

#endif  // KUDNN_SHAPE_HPP
