// Status codes of the KuDNN C++ API (values == KUDNN_STATUS_SUCCESS/UNSUPPORTED/BAD_ARGUMENTS of kudnn_hip.h;
// reference: src/dnn/include/service/kudnn_err_codes.hpp:18-22).
#ifndef KUDNN_ERR_CODES
#define KUDNN_ERR_CODES

namespace KuDNN {

enum class Status { SUCCESS = 0, UNSUPPORTED, BAD_ARGUMENTS };

}  // namespace KuDNN

#endif  // KUDNN_ERR_CODES
