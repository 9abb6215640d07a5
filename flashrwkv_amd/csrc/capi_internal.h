// Internal helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>

#include "../../include/flashrwkv_amd.h"

namespace frwkv {

// Records a printf-style message as the calling thread's last error and
// returns status.
int set_error(int status, const char* fmt, ...);

// Converts a pending launch error into FRWKV_ERR_HIP with a message.
int check_launch(const char* what);

}  // namespace frwkv
