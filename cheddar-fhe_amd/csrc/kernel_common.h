// Error plumbing shared by the C-ABI entry points: every call returns 0 or a
// negative status and leaves a message for chd_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "cheddar_amd.h"

// invalid argument, caught on the host before any launch
#define CHD_ERR_ARG CHD_ERR_INVALID_ARGUMENT

namespace chd {
int set_error(int code, const std::string &msg);
int check_launch(const char *where);
}  // namespace chd
