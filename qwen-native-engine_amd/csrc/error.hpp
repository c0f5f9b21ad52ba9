// Error type carried from the host code to the C ABI, where it becomes a return code and the
// thread-local message returned by qne_last_error().
#pragma once

#include <stdexcept>
#include <string>

#include "../../include/qne.h"

namespace qne {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

}  // namespace qne
