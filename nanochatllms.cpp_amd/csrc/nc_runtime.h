// nc_runtime.h -- host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/gten_hip.h"
#include "nc_layout.h"

namespace nc {

// Records a message for nc_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);
hipStream_t stream_of(void* s);
bool initialized();

// Takes the device address of nc_matmul_2d_noalloc's staging array on
// device `dev` (the current device); called by nc_init.
int noalloc_scratch_setup(int dev);

// Checks a kernel launch; returns NC_OK or the recorded failure.
inline int launch_status(const char* what)
{
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? NC_OK : hip_fail(e, what);
}

inline bool is_act(int dt) { return dt == NC_Q8 || dt == NC_F16 || dt == NC_F32; }

}  // namespace nc

#define NC_CHECK_ARG(cond, ...)                                   \
    do {                                                          \
        if (!(cond)) return ::nc::fail(NC_ERR_ARG, __VA_ARGS__); \
    } while (0)
