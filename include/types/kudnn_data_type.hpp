// Element types and size aliases of the KuDNN C++ API (MI355X build).
// Same names and enumerator values as KuDNN's kudnn_data_type.hpp (src/dnn/include/types/kudnn_data_type.hpp:23-39),
// so that sources written against KuDNN compile unchanged.
#ifndef KUDNN_DATATYPE_HPP
#define KUDNN_DATATYPE_HPP

#include <cstddef>
#include <cstdint>

#include "service/kudnn_exception.hpp"

#define KUDNN_API_PUBLIC __attribute__((visibility("default")))

namespace KuDNN {

using SizeType = std::size_t;
using IntType = std::int64_t;

namespace Element {

enum class TypeT { UNDEFINED = 0, F32, F16, BF16, S32, S8, U8 };

// Run-time description of an element type: its enumerator plus its storage size in bytes.
struct Type final {
public:
    using SizeType = ::KuDNN::SizeType;
    Type(const TypeT &t) noexcept(false) : type{t}, size(SizeOf(t))
    {
        if (size == 0) {
            throw Service::LogicError{"Type: unsupported data type"};
        }
    }
    SizeType GetSize() const noexcept { return size; }
    SizeType GetBitwidth() const noexcept { return size * 8u; }
    operator TypeT() const noexcept { return type; }
    bool IsFP() const noexcept { return type == TypeT::F32 || type == TypeT::F16 || type == TypeT::BF16; }
    bool IsIntegral() const noexcept { return !IsFP(); }
    bool IsSigned() const noexcept { return type != TypeT::U8; }
    bool IsUnsigned() const noexcept { return !IsSigned(); }

private:
    static SizeType SizeOf(TypeT t) noexcept
    {
        switch (t) {
            case TypeT::F32: case TypeT::S32: return 4;
            case TypeT::F16: case TypeT::BF16: return 2;
            case TypeT::S8: case TypeT::U8: return 1;
            default: return 0;
        }
    }
    TypeT type;
    SizeType size;
};

// Maps a C++ element type to its enumerator (UNDEFINED for unknown types).
template <typename ElementType>
inline TypeT MatchType() { return TypeT::UNDEFINED; }
template <> inline TypeT MatchType<float>() { return TypeT::F32; }
template <> inline TypeT MatchType<std::int32_t>() { return TypeT::S32; }
template <> inline TypeT MatchType<std::int8_t>() { return TypeT::S8; }
template <> inline TypeT MatchType<std::uint8_t>() { return TypeT::U8; }
#if defined(__FLT16_MANT_DIG__)
template <> inline TypeT MatchType<_Float16>() { return TypeT::F16; }
#endif
#if defined(__BFLT16_MANT_DIG__)
template <> inline TypeT MatchType<__bf16>() { return TypeT::BF16; }
#endif

inline bool operator==(const Type &lhs, const TypeT &rhs) noexcept { return static_cast<TypeT>(lhs) == rhs; }
inline bool operator==(const TypeT &lhs, const Type &rhs) noexcept { return lhs == static_cast<TypeT>(rhs); }
inline bool operator==(const Type &lhs, const Type &rhs) noexcept
{
    return lhs.GetSize() == rhs.GetSize() && static_cast<TypeT>(lhs) == static_cast<TypeT>(rhs);
}
inline bool operator!=(const Type &lhs, const TypeT &rhs) noexcept { return !(lhs == rhs); }
inline bool operator!=(const TypeT &lhs, const Type &rhs) noexcept { return !(lhs == rhs); }
inline bool operator!=(const Type &lhs, const Type &rhs) noexcept { return !(lhs == rhs); }

}  // namespace Element
}  // namespace KuDNN

#endif  // KUDNN_DATATYPE_HPP
