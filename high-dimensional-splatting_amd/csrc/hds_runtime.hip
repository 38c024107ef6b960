// Error reporting and launch checking behind the C ABI (include/hds_rasterizer.h).
// The reference surfaces launch and execution errors as C++ exceptions with the kernel's name and
// syncs after every launch when GS_DEBUG is set (common.cuh:67-91); here the same information comes
// back as a status code plus a per-thread message, and HDS_DEBUG (or GS_DEBUG) turns the sync on.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>

#include "hds_internal.h"
#include "hds_rasterizer.h"

static thread_local char g_last_error[512] = "no error";

int hds_set_error(int status, const char* fmt, ...) {
	va_list args;
	va_start(args, fmt);
	vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
	va_end(args);
	return status;
}

bool hds_debug_sync_enabled() {
	static const bool on = std::getenv("HDS_DEBUG") != nullptr || std::getenv("GS_DEBUG") != nullptr;
	return on;
}

int hds_check_launch(const char* kernel, hipStream_t stream) {
	hipError_t err = hipGetLastError();
	if (err != hipSuccess)
		return hds_set_error(HDS_ERR_RUNTIME, "HIP kernel launch error (%s): %s", kernel, hipGetErrorString(err));
	if (!hds_debug_sync_enabled()) return HDS_OK;
	err = hipStreamSynchronize(stream);
	if (err == hipSuccess) err = hipGetLastError();
	if (err != hipSuccess)
		return hds_set_error(HDS_ERR_RUNTIME, "HIP kernel execution error (%s): %s", kernel, hipGetErrorString(err));
	return HDS_OK;
}

extern "C" const char* hds_last_error(void) { return g_last_error; }

extern "C" int hds_abi_version(void) { return HDS_ABI_VERSION; }
