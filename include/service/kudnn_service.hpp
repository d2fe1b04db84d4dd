// Service helpers of the KuDNN C++ API: layout index mapping, stride flushing, overflow checks and aligned
// host allocation. Same declarations as KuDNN (src/dnn/include/service/kudnn_service.hpp:27-140).
#ifndef KUDNN_SERVICE_HPP
#define KUDNN_SERVICE_HPP

#include <cstddef>
#include <iterator>
#include <limits>
#include <type_traits>

#include "service/kudnn_exception.hpp"
#include "types/kudnn_data_type.hpp"
#include "types/kudnn_layout.hpp"
#include "types/kudnn_types.hpp"

namespace KuDNN {
namespace Service {

constexpr SizeType ALIGNMENT = 128;

// Logical dimension stored at physical position `idx` of layout `l` (throws LogicError past the layout's rank).
KUDNN_API_PUBLIC SizeType GetIdxForUserLayout(Layout l, SizeType idx) noexcept(false);

// `sh` (in logical order) permuted into physical order of `parLayout`.
KUDNN_API_PUBLIC Shape GetShapeAccordingToLayout(const Shape &sh, Layout parLayout) noexcept;

// Strides with the entries of size-1 dimensions set to 0 (implicit broadcasting).
KUDNN_API_PUBLIC Shape FlushStrides(const Shape &dims, const Shape &strides) noexcept(false);

template <typename... Ts>
struct IsAllSame : std::true_type {};
template <typename T, typename U, typename... Rest>
struct IsAllSame<T, U, Rest...>
    : std::integral_constant<bool, std::is_same<T, U>::value && IsAllSame<U, Rest...>::value> {};

// True when a * b does not fit in IntType.
template <typename IntType,
          typename std::enable_if<std::is_integral<typename std::remove_reference<IntType>::type>::value, bool>::type = true>
bool WillIntMultOverflow(IntType a, IntType b) noexcept
{
    typename std::remove_reference<IntType>::type r;
    return __builtin_mul_overflow(a, b, &r);
}

template <typename IntType, typename... Args,
          typename std::enable_if<IsAllSame<IntType, Args...>::value, bool>::type = true>
bool WillIntMultOverflow(IntType a, IntType b, Args... args) noexcept
{
    IntType r;
    if (__builtin_mul_overflow(a, b, &r)) {
        return true;
    }
    return WillIntMultOverflow(r, args...);
}

// True when the product of [begin, end) does not fit in the iterator's value type.
template <typename ForwardIt,
          typename std::enable_if<std::is_integral<typename std::iterator_traits<ForwardIt>::value_type>::value,
                                  bool>::type = true>
bool WillIntMultOverflow(ForwardIt begin, ForwardIt end) noexcept
{
    typename std::iterator_traits<ForwardIt>::value_type acc = 1;
    for (ForwardIt it = begin; it != end; ++it) {
        if (__builtin_mul_overflow(acc, *it, &acc)) {
            return true;
        }
    }
    return false;
}

// Host allocation aligned to `alignment` (a power of two); throws BadAlloc on failure.
KUDNN_API_PUBLIC void *AlignedAlloc(SizeType n, SizeType alignment = ALIGNMENT) noexcept(false);
KUDNN_API_PUBLIC void Deallocate(void *p, SizeType n = 0) noexcept;

// std::allocator-compatible wrapper of AlignedAlloc / Deallocate.
template <typename T, SizeType alignment = ALIGNMENT>
struct AlignedAllocator {
    using value_type = T;
    using pointer = T *;
    using const_pointer = const T *;
    using reference = T &;
    using const_reference = const T &;
    using size_type = ::KuDNN::SizeType;
    using difference_type = std::ptrdiff_t;

    template <typename U>
    struct rebind {
        using other = AlignedAllocator<U, alignment>;
    };

    T *allocate(SizeType n) const noexcept(false)
    {
        if (n > std::numeric_limits<SizeType>::max() / sizeof(T)) {
            throw BadArrayNewLength();
        }
        return static_cast<T *>(AlignedAlloc(n * sizeof(T), alignment));
    }
    void deallocate(T *p, SizeType n = 0) const noexcept { ::KuDNN::Service::Deallocate(p, n); }
    virtual ~AlignedAllocator() = default;
};

template <typename T>
struct Deallocator {
    void operator()(T *p, ::KuDNN::SizeType n = 0) const noexcept { ::KuDNN::Service::Deallocate(p, n); }
};

template <typename T, SizeType A1, typename U, SizeType A2>
constexpr bool operator==(const AlignedAllocator<T, A1> &, const AlignedAllocator<U, A2> &) noexcept
{
    return A1 == A2 && std::is_same<T, U>::value;
}
template <typename T, SizeType A1, typename U, SizeType A2>
constexpr bool operator!=(const AlignedAllocator<T, A1> &l, const AlignedAllocator<U, A2> &r) noexcept
{
    return !(l == r);
}

}  // namespace Service
}  // namespace KuDNN

#endif  // KUDNN_SERVICE_HPP
