// Error mapping of the C ABI onto the exceptions the reference's callers expect
// (include/zcgvs/core/cuda_check.hpp:10-37): invalid arguments raise std::invalid_argument,
// device and runtime failures raise HipError, a std::runtime_error.
#pragma once

#include <stdexcept>
#include <string>

#include "zcgvs_hip.h"

namespace zcgvs {

class HipError : public std::runtime_error {
public:
    explicit HipError(const std::string& message) : std::runtime_error(message) {}
};

// Throws for a non-OK status of a zcgvs_* call, with the library's thread-local message.
inline void check(int status) {
    if (status == ZCGVS_OK) {
        return;
    }
    const char* message = zcgvs_last_error();
    const std::string text = message != nullptr && *message != '\0' ? message : "zcgvs: call failed";
    if (status == ZCGVS_ERR_INVALID_ARGUMENT) {
        throw std::invalid_argument(text);
    }
    throw HipError(text);
}

}  // namespace zcgvs
