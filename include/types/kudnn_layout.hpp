// Tensor layouts of the KuDNN C++ API. Letters name logical dimensions from the slowest physical position
// to the fastest. Same enumerators, order and aliases as KuDNN (src/dnn/include/types/kudnn_layout.hpp:19-64);
// the numeric values are also those of KUDNN_LAYOUT_* in kudnn_hip.h.
#ifndef KUDNN_LAYOUT_HPP
#define KUDNN_LAYOUT_HPP

namespace KuDNN {

enum class Layout {
    UNDEFINED = 0,
    A,
    AB, BA,
    ABC, ACB, BAC, BCA, CAB, CBA,
    ABCD, ABDC, ACBD, ACDB, ADBC, ADCB, BACD, BCDA, CDAB, CDBA, DCAB,
    ABCDE, ABCED, ABDEC, ACBDE, ACDEB, ADECB, BACDE, BCDEA, CDEAB, CDEBA, DECAB,
    ROW_MAJOR = AB,
    COL_MAJOR = BA,
    NCHW = ABCD,
    NHWC = ACDB,
    NCDHW = ABCDE,
    NDHWC = ACDEB,
    OIHW = ABCD,
    HWIO = CDBA,
    HWOI = CDAB,
    OHWI = ACDB,
    OHWO = BCDA,
    IOHW = BACD,
};

}  // namespace KuDNN

#endif  // KUDNN_LAYOUT_HPP
