// Threading controls of the KuDNN C++ API (reference: src/dnn/include/service/kudnn_threading.hpp:20-35).
// The MI355X build runs every primitive on the GPU and starts no host threads; the settings are kept
// (and validated against the host's core count) so that numThreads arguments behave as in KuDNN:
// a Run or constructor with numThreads outside [0, GetMaxNumThreads()] is rejected with LogicError.
#ifndef KUDNN_THREADING_HPP
#define KUDNN_THREADING_HPP

#include "types/kudnn_data_type.hpp"

namespace KuDNN {
namespace Threading {

enum class EnvMode { KUDNN_THREAD_USE_ENV, KUDNN_THREAD_IGNORE_ENV };

enum class ThreadingControl { KUDNN_DEFAULT, KUDNN_MANUAL };

KUDNN_API_PUBLIC bool ShouldCalculateOptThreads() noexcept;
KUDNN_API_PUBLIC int SetMaxNumThreads(int nThreads) noexcept;
KUDNN_API_PUBLIC int SetFixedNumThreads(int nThreads) noexcept;
KUDNN_API_PUBLIC int GetMaxNumThreads() noexcept;
KUDNN_API_PUBLIC int SetNumThreadsLocal(int nThreads) noexcept;
KUDNN_API_PUBLIC EnvMode SetEnvMode(EnvMode mode) noexcept;
KUDNN_API_PUBLIC ThreadingControl GetThreadingControlStatus() noexcept;

}  // namespace Threading
}  // namespace KuDNN

#endif  // KUDNN_THREADING_HPP
