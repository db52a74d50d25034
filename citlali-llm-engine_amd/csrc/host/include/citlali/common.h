// citlali/common.h -- the error type of the host layer.
//
// Same type and helper as the reference (include/citlali/common.h:1-20), so
// code written against the reference catches the same exceptions: every
// failure of the host layer or of a HIP call below it throws citlali::Error.
#pragma once

#include <stdexcept>
#include <string>

namespace citlali {

class Error : public std::runtime_error {
public:
    explicit Error(const std::string& message) : std::runtime_error(message) {}
};

// Throws Error(message) when `condition` is false.
inline void require(bool condition, const std::string& message) {
    if (!condition) throw Error(message);
}

}  // namespace citlali
