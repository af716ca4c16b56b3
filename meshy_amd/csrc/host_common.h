// Error reporting of libmeshy_amd, for the host-only sources (the planner and
// the host gather) as well as the kernels' sources: no device code here.
#pragma once

#include <stdint.h>

#include "../../include/meshy_amd.h"

namespace meshy {

// Records `msg` (printf-style) as the calling thread's last error and returns code.
int set_error(int code, const char* fmt, ...);
void clear_error();

}  // namespace meshy
