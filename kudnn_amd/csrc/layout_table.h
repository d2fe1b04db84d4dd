// Layout permutation table shared by the C ABI (libkudnn_hip.so) and the C++ API (libkudnn.so).
//
// A KuDNN layout names the logical dimensions from the slowest physical position to the fastest, so
// "ACB" means physical position 0 holds logical dim 0, position 1 logical dim 2, position 2 logical dim 1.
// The reference spells this out case by case in GetIdxForUserLayout (src/dnn/src/service.cpp:115-333)
// and the per-layout stride formulas of SetMinimumRequiredStrides (src/dnn/src/kudnn_tensor_info.cpp:141-325);
// every one of those formulas is "the fastest physical dim has stride 1, each slower one the product of the
// faster dims' sizes", which is what MinStrides below computes from the permutation.
#ifndef KUDNN_LAYOUT_TABLE_H
#define KUDNN_LAYOUT_TABLE_H

#include <cstdint>

namespace kudnn_layout {

constexpr int kMaxDims = 5;

struct Entry {
    int ndims;
    int perm[kMaxDims];  // perm[physical position] = logical dim
};

// Indexed by the KuDNN::Layout / KUDNN_LAYOUT_* value (kudnn_layout.hpp:19-51).
inline const Entry *Lookup(int layout)
{
    static const Entry table[] = {
        {0, {0, 0, 0, 0, 0}},  // UNDEFINED
        {1, {0, 0, 0, 0, 0}},  // A
        {2, {0, 1, 0, 0, 0}},  // AB
        {2, {1, 0, 0, 0, 0}},  // BA
        {3, {0, 1, 2, 0, 0}},  // ABC
        {3, {0, 2, 1, 0, 0}},  // ACB
        {3, {1, 0, 2, 0, 0}},  // BAC
        {3, {1, 2, 0, 0, 0}},  // BCA
        {3, {2, 0, 1, 0, 0}},  // CAB
        {3, {2, 1, 0, 0, 0}},  // CBA
        {4, {0, 1, 2, 3, 0}},  // ABCD
        {4, {0, 1, 3, 2, 0}},  // ABDC
        {4, {0, 2, 1, 3, 0}},  // ACBD
        {4, {0, 2, 3, 1, 0}},  // ACDB
        {4, {0, 3, 1, 2, 0}},  // ADBC
        {4, {0, 3, 2, 1, 0}},  // ADCB
        {4, {1, 0, 2, 3, 0}},  // BACD
        {4, {1, 2, 3, 0, 0}},  // BCDA
        {4, {2, 3, 0, 1, 0}},  // CDAB
        {4, {2, 3, 1, 0, 0}},  // CDBA
        {4, {3, 2, 0, 1, 0}},  // DCAB
        {5, {0, 1, 2, 3, 4}},  // ABCDE
        {5, {0, 1, 2, 4, 3}},  // ABCED
        {5, {0, 1, 3, 4, 2}},  // ABDEC
        {5, {0, 2, 1, 3, 4}},  // ACBDE
        {5, {0, 2, 3, 4, 1}},  // ACDEB
        {5, {0, 3, 4, 2, 1}},  // ADECB
        {5, {1, 0, 2, 3, 4}},  // BACDE
        {5, {1, 2, 3, 4, 0}},  // BCDEA
        {5, {2, 3, 4, 0, 1}},  // CDEAB
        {5, {2, 3, 4, 1, 0}},  // CDEBA
        {5, {3, 4, 2, 0, 1}},  // DECAB
    };
    constexpr int n = static_cast<int>(sizeof(table) / sizeof(table[0]));
    if (layout <= 0 || layout >= n) {
        return nullptr;
    }
    return &table[layout];
}

// A layout is valid for a tensor when it names exactly that many dims
// (the per-ndims lists of TensorInfo::ValidateLayout, kudnn_tensor_info.cpp:59-138).
inline bool IsValidFor(int layout, int ndims)
{
    const Entry *e = Lookup(layout);
    return e != nullptr && e->ndims == ndims;
}

// The standard "ABX" layout for a dimensionality (TensorInfo::GetStandardABXLayout, kudnn_tensor_info.hpp:199-221).
inline int StandardLayout(int ndims)
{
    switch (ndims) {
        case 1: return 1;   // A
        case 2: return 2;   // AB
        case 3: return 4;   // ABC
        case 4: return 10;  // ABCD
        case 5: return 21;  // ABCDE
        default: return 0;
    }
}

// Minimum (dense) strides in logical order, with strides of size-1 dims flushed to 0 as
// Service::FlushStrides does (service.cpp:355-372). Returns false for an unknown layout/ndims pair.
inline bool MinStrides(int layout, int ndims, const int64_t *dims, int64_t *strides)
{
    const Entry *e = Lookup(layout);
    if (e == nullptr || e->ndims != ndims) {
        return false;
    }
    int64_t run = 1;
    for (int p = ndims - 1; p >= 0; --p) {
        int d = e->perm[p];
        strides[d] = run;
        run *= dims[d];
    }
    for (int d = 0; d < ndims; ++d) {
        if (dims[d] == 1) {
            strides[d] = 0;
        }
    }
    return true;
}

// Logical dim stored at a physical position: Service::GetIdxForUserLayout (service.cpp:115-333).
inline int LogicalAt(int layout, int physicalPos)
{
    const Entry *e = Lookup(layout);
    return e == nullptr ? -1 : e->perm[physicalPos];
}

}  // namespace kudnn_layout

#endif  // KUDNN_LAYOUT_TABLE_H
