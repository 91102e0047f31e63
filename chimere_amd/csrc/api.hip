// api.hip -- error state, size helpers.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "api_internal.h"

namespace chimere {

static thread_local int g_err = CHIMERE_OK;
static thread_local char g_msg[512];

void set_error(int code, const char* fmt, ...) {
    g_err = code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof g_msg, fmt, ap);
    va_end(ap);
    if (getenv("CHIMERE_HIP_VALIDATE") && strcmp(getenv("CHIMERE_HIP_VALIDATE"), "0") != 0)
        fprintf(stderr, "[chimere_hip] error %d: %s\n", code, g_msg);
}

bool check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(CHIMERE_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
        return false;
    }
    return true;
}

bool validate_enabled() {
    static int v = -1;
    if (v < 0) {
        const char* s = getenv("CHIMERE_HIP_VALIDATE");
        v = (s && strcmp(s, "0") != 0) ? 1 : 0;
    }
    return v == 1;
}

}  // namespace chimere

extern "C" {

int chimere_q8_1_block_bytes(void) { return 36; }
int chimere_q8_1_block_elems(void) { return 32; }
int chimere_matrix_row_padding(void) { return 512; }

int chimere_hip_get_last_error(void) {
    int e = chimere::g_err;
    chimere::g_err = CHIMERE_OK;
    return e;
}

const char* chimere_hip_get_last_error_string(void) { return chimere::g_msg; }

}  // extern "C"
