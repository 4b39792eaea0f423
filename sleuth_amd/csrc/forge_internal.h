// Host-side helpers shared by the entry points of libforge_attn.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/forge_attn.h"

namespace forge {

// Records `msg` as this thread's last error and returns the rejection status (-1).
int set_error(const char* msg);
void clear_error();
// Status of the launch just issued: 0, or the hipError_t (> 0) with its text recorded.
int check_launch();

}  // namespace forge
