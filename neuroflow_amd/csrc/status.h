// status.h -- thread-local last-error message behind nflow_last_error().
#pragma once

#include <string>

namespace nfq {

// Records `msg` for nflow_last_error() on this thread and returns `code`.
int set_error(int code, const std::string& msg);

// Clears the message at the start of every entry point.
void clear_error();

}  // namespace nfq
