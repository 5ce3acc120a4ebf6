// nc_runtime.cpp -- device, memory and error plumbing of the C-ABI.
#include "nc_runtime.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

namespace nc {

static thread_local std::string g_err;
static hipStream_t g_stream = nullptr;
static int g_device = -1;

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    return fail(NC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

hipStream_t stream_of(void* s)
{
    if (s) return static_cast<hipStream_t>(s);
    return g_stream;
}

bool initialized() { return g_device >= 0; }

}  // namespace nc

using namespace nc;

extern "C" {

int nc_init(int device)
{
    if (g_device == device) return NC_OK;
    if (g_device >= 0) return fail(NC_ERR_STATE, "nc_init: already initialized on device %d", g_device);
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= n) return fail(NC_ERR_ARG, "nc_init: device %d of %d", device, n);
    if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    if ((e = hipStreamCreate(&g_stream)) != hipSuccess) return hip_fail(e, "hipStreamCreate");
    int s = noalloc_scratch_setup(device);
    if (s) return s;
    g_device = device;
    return NC_OK;
}

const char* nc_last_error(void) { return g_err.c_str(); }

int nc_malloc(void** ptr, size_t bytes)
{
    if (!ptr) return fail(NC_ERR_ARG, "nc_malloc: null out pointer");
    *ptr = nullptr;
    if (bytes == 0) return NC_OK;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) return fail(NC_ERR_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return NC_OK;
}

int nc_free(void* ptr)
{
    if (!ptr) return NC_OK;
    hipError_t e = hipFree(ptr);
    return e == hipSuccess ? NC_OK : hip_fail(e, "hipFree");
}

int nc_memcpy_h2d(void* dst, const void* src, size_t bytes)
{
    if (!bytes) return NC_OK;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    return e == hipSuccess ? NC_OK : hip_fail(e, "nc_memcpy_h2d");
}

int nc_memcpy_d2h(void* dst, const void* src, size_t bytes)
{
    if (!bytes) return NC_OK;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
    return e == hipSuccess ? NC_OK : hip_fail(e, "nc_memcpy_d2h");
}

int nc_memset_d(void* dst, int value, size_t bytes)
{
    if (!bytes) return NC_OK;
    hipError_t e = hipMemsetAsync(dst, value, bytes, g_stream);
    return e == hipSuccess ? NC_OK : hip_fail(e, "nc_memset_d");
}

int nc_synchronize(void)
{
    if (!initialized()) return fail(NC_ERR_STATE, "nc_synchronize: nc_init not called");
    hipError_t e = hipStreamSynchronize(g_stream);
    return e == hipSuccess ? NC_OK : hip_fail(e, "hipStreamSynchronize");
}

}  // extern "C"
