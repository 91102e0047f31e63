// api_internal.h -- host-side error state and launch checking for the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "chimere_hip.h"

namespace chimere {

// Records an error code + message for chimere_hip_get_last_error().
void set_error(int code, const char* fmt, ...);
// Records a failed launch (if any) after a kernel launch; returns true on success.
bool check_launch(const char* what);
// Validation enabled by CHIMERE_HIP_VALIDATE=1 (extra host-side checks).
bool validate_enabled();

}  // namespace chimere

#define CHIMERE_REQUIRE(cond, code, ...)            \
    do {                                            \
        if (!(cond)) {                              \
            ::chimere::set_error((code), __VA_ARGS__); \
            return;                                 \
        }                                           \
    } while (0)
