// Thread-local last-error message of libstlq_mi355, shared by its host translation units
// (stlq_mi355_last_error() returns it).
#pragma once

#include <string>

namespace stlq_mi355 {

// Stores msg as the calling thread's last error and returns code.
int SetLastError(int code, const std::string& msg);

}  // namespace stlq_mi355
