// Shared by the library's translation units: the thread-local message mg_last_error() returns.
#pragma once

#include <string>

namespace mg {
void set_last_error(const std::string& msg);
}  // namespace mg
