// Error reporting shared by the C-ABI entry points: a nonzero gdn2_status plus
// a per-thread message (gdn2_last_error), set before anything is launched.
#pragma once

#include <hip/hip_runtime.h>

#include "gdn2.h"

namespace gdn2 {

int fail(int code, const char *fmt, ...);
int ok();
const char *last_error();
// dtype: -1 = F32 or BF16; otherwise the required dtype.
int check_view(const gdn2_view *v, const char *name, int dtype, bool data_may_be_null);
int launch_status(hipError_t e, const char *what);

}  // namespace gdn2

#define GDN2_TRY(x)                     \
    do {                                \
        int _rc = (x);                  \
        if (_rc != GDN2_OK) return _rc; \
    } while (0)
