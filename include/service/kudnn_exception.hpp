// Exceptions thrown by the KuDNN C++ API. Same types and bases as KuDNN
// (src/dnn/include/service/kudnn_exception.hpp:25-51) so existing catch clauses keep working:
//   LogicError  (std::logic_error)       bad shapes, layouts, thread counts, null pointers
//   Unsupported (std::invalid_argument)  valid but unsupported dtype / kind combinations
//   BadAlloc    (std::bad_alloc)         allocation failures
// Failures of the HIP runtime (no counterpart in the CPU reference) are reported as std::runtime_error.
#ifndef KUDNN_EXCEPTION_HPP
#define KUDNN_EXCEPTION_HPP

#include <exception>
#include <new>
#include <stdexcept>
#include <string>

namespace KuDNN {
namespace Service {

struct BadAlloc : public std::bad_alloc {
    const char *what() const noexcept override { return "KuDNN allocation failed"; }
};

struct BadArrayNewLength : public std::bad_array_new_length {
    const char *what() const noexcept override { return "KuDNN bad array new length"; }
};

struct LogicError : public std::logic_error {
    explicit LogicError(const std::string &whatArg) : std::logic_error(whatArg) {}
    explicit LogicError(const char *whatArg) : std::logic_error(whatArg) {}
    LogicError(const LogicError &other) noexcept : std::logic_error(other) {}
    LogicError &operator=(const LogicError &other) noexcept = default;
};

struct Unsupported : public std::invalid_argument {
    explicit Unsupported(const std::string &whatArg) : std::invalid_argument(whatArg) {}
    explicit Unsupported(const char *whatArg) : std::invalid_argument(whatArg) {}
    Unsupported(const Unsupported &other) noexcept : std::invalid_argument(other) {}
    Unsupported &operator=(const Unsupported &other) noexcept = default;
};

}  // namespace Service
}  // namespace KuDNN

#endif  // KUDNN_EXCEPTION_HPP
