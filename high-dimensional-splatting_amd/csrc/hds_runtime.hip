// Error reporting and launch checking behind the C ABI (include/hds_rasterizer.h).
// The reference surfaces launch and execution errors as C++ exceptions with the kernel's name and
// syncs after every launch when GS_DEBUG is set (common.cuh:67-91); here the same information comes
// back as a status code plus a per-thread message, and HDS_DEBUG (or GS_DEBUG) turns the sync on.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

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

// A second stream per device for kernels that run beside the caller's stream (default priority,
// non-blocking, created on first use and kept until the process ends).
int hds_side_stream(hipStream_t* out) {
	static std::mutex mutex;
	static std::vector<hipStream_t> streams;
	int device = 0;
	HDS_HIP(hipGetDevice(&device));
	std::lock_guard<std::mutex> lock(mutex);
	if ((int)streams.size() <= device) streams.resize(device + 1, nullptr);
	if (!streams[device]) HDS_HIP(hipStreamCreateWithFlags(&streams[device], hipStreamNonBlocking));
	*out = streams[device];
	return HDS_OK;
}

extern "C" const char* hds_last_error(void) { return g_last_error; }

extern "C" int hds_abi_version(void) { return HDS_ABI_VERSION; }

// Kernel timing: a pool of event pairs reused across recordings, one pair per recorded launch.
namespace {
struct ProfileRecord {
	const char* name;
	hipEvent_t start, stop;
};
std::mutex g_profile_mutex;
bool g_profile_on = false;
std::vector<ProfileRecord> g_profile;
int64_t g_profile_used = 0;
std::vector<std::string> g_profile_only;  // kernels to record; empty = all

bool profile_wanted(const char* name) {
	if (g_profile_only.empty()) return true;
	for (const std::string& k : g_profile_only)
		if (k == name) return true;
	return false;
}
}  // namespace

HdsKernelTimer::HdsKernelTimer(const char* name, hipStream_t stream) : slot_(-1), stream_(stream) {
	std::lock_guard<std::mutex> lock(g_profile_mutex);
	if (!g_profile_on || !profile_wanted(name)) return;
	if (g_profile_used == (int64_t)g_profile.size()) {
		ProfileRecord r{name, nullptr, nullptr};
		if (hipEventCreate(&r.start) != hipSuccess) return;
		if (hipEventCreate(&r.stop) != hipSuccess) {
			(void)hipEventDestroy(r.start);
			return;
		}
		g_profile.push_back(r);
	}
	ProfileRecord& r = g_profile[g_profile_used];
	r.name = name;
	if (hipEventRecord(r.start, stream) != hipSuccess) return;
	slot_ = g_profile_used++;
}

void HdsKernelTimer::stop() {
	if (slot_ < 0) return;
	std::lock_guard<std::mutex> lock(g_profile_mutex);
	(void)hipEventRecord(g_profile[slot_].stop, stream_);
	slot_ = -1;
}

extern "C" int hds_profile_begin_only(const char* kernels) {
	std::lock_guard<std::mutex> lock(g_profile_mutex);
	g_profile_only.clear();
	if (kernels) {
		const char* p = kernels;
		while (*p) {
			const char* comma = std::strchr(p, ',');
			const size_t len = comma ? (size_t)(comma - p) : std::strlen(p);
			if (len > 0) g_profile_only.emplace_back(p, len);
			p += len + (comma ? 1 : 0);
		}
	}
	g_profile_used = 0;
	g_profile_on = true;
	return HDS_OK;
}

extern "C" int hds_profile_begin(void) { return hds_profile_begin_only(nullptr); }

extern "C" int64_t hds_profile_end(void) {
	std::lock_guard<std::mutex> lock(g_profile_mutex);
	g_profile_on = false;
	for (int64_t i = 0; i < g_profile_used; i++) {
		const hipError_t e = hipEventSynchronize(g_profile[i].stop);
		if (e != hipSuccess) return -hds_set_error(HDS_ERR_RUNTIME, "hds_profile_end: %s", hipGetErrorString(e));
	}
	return g_profile_used;
}

extern "C" int hds_profile_record(int64_t i, const char** name, float* ms) {
	std::lock_guard<std::mutex> lock(g_profile_mutex);
	HDS_REQUIRE(i >= 0 && i < g_profile_used && name && ms, "hds_profile_record: no record %lld", (long long)i);
	*name = g_profile[i].name;
	HDS_HIP(hipEventElapsedTime(ms, g_profile[i].start, g_profile[i].stop));
	return HDS_OK;
}

extern "C" int hds_profile_timeline(int64_t i, const char** name, float* start_ms, float* end_ms) {
	std::lock_guard<std::mutex> lock(g_profile_mutex);
	HDS_REQUIRE(i >= 0 && i < g_profile_used && name && start_ms && end_ms, "hds_profile_timeline: no record %lld",
				(long long)i);
	*name = g_profile[i].name;
	HDS_HIP(hipEventElapsedTime(start_ms, g_profile[0].start, g_profile[i].start));
	HDS_HIP(hipEventElapsedTime(end_ms, g_profile[0].start, g_profile[i].stop));
	return HDS_OK;
}
