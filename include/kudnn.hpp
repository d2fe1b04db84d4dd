// Umbrella header of the MI355X KuDNN Linear/GEMM library (libkudnn.so). Mirrors KuDNN's kudnn.hpp
// (src/dnn/include/kudnn.hpp:16-38) for the operators of the Linear/GEMM path; KuDNN's other operators
// (convolution, norms, softmax, RoPE, embedding, reorder, stand-alone eltwise) are not part of this build.
#ifndef KUDNN_HPP
#define KUDNN_HPP

#include "types/kudnn_data_type.hpp"
#include "types/kudnn_layout.hpp"
#include "types/kudnn_shape.hpp"
#include "types/kudnn_tensor_info.hpp"
#include "types/kudnn_types.hpp"

#include "service/kudnn_err_codes.hpp"
#include "service/kudnn_exception.hpp"
#include "service/kudnn_service.hpp"
#include "service/kudnn_threading.hpp"

#include "operations/kudnn_eltwise.hpp"
#include "operations/kudnn_gemm.hpp"
#include "operations/kudnn_linear_activationlayer.hpp"
#include "operations/kudnn_linear_postops.hpp"
#include "operations/kudnn_linear_res.hpp"

#endif  // KUDNN_HPP
