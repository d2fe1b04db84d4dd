// Forward declarations of the KuDNN descriptor types.
#ifndef KUDNN_TYPES_HPP
#define KUDNN_TYPES_HPP

namespace KuDNN {

struct Type;
struct Shape;
struct TensorInfo;

}  // namespace KuDNN

#endif  // KUDNN_TYPES_HPP
