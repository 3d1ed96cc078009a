// Status reporting, device-limit cache and type checks shared by every entry point.
#include "clk_common.h"

#include <cstdio>

namespace clk {

namespace {
thread_local std::string g_last_error;
constexpr int kMaxDevices = 16;
int g_shared_limit[kMaxDevices] = {};
constexpr int kMaxStages = 16;
void* g_stage_events[kMaxStages] = {};
int g_stage_count = 0;

const char* type_name(int t) {
    switch (t) {
    case CLK_S32: return "S32";
    case CLK_U8: return "U8";
    case CLK_F16: return "F16";
    case CLK_F32: return "F32";
    case CLK_BF16: return "BF16";
    default: return "?";
    }
}
}  // namespace

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int ok() {
    g_last_error.clear();
    return CLK_OK;
}

int launch_status(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return fail(CLK_INTERNAL, std::string(what) + " launch: " + hipGetErrorString(err));
    }
    return ok();
}

void stage_mark(hipStream_t s, int i) {
    if (i < g_stage_count && g_stage_events[i] != nullptr) {
        (void)hipEventRecord(static_cast<hipEvent_t>(g_stage_events[i]), s);
    }
}

int shared_limit(int device) {
    if (device < 0 || device >= kMaxDevices) return 0;  // 0: unknown, callers skip the check
    if (g_shared_limit[device] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) ==
            hipSuccess) {
            g_shared_limit[device] = v;
        }
    }
    return g_shared_limit[device];
}

int check_types(const char* what, const clk_buffer* const* bufs, const int* types, int n) {
    for (int i = 0; i < n; ++i) {
        if (bufs[i] == nullptr) {
            return invalid(std::string(what) + ": buffer " + std::to_string(i) + " is missing");
        }
        if (bufs[i]->dtype != types[i]) {
            return invalid(std::string(what) + ": buffer " + std::to_string(i) + " must be " +
                           type_name(types[i]) + ", got " + type_name(bufs[i]->dtype));
        }
        if (bufs[i]->rank < 0 || (bufs[i]->rank > 0 && bufs[i]->dims == nullptr)) {
            return invalid(std::string(what) + ": buffer " + std::to_string(i) +
                           " has no dimensions");
        }
    }
    return CLK_OK;
}

}  // namespace clk

extern "C" const char* clk_last_error(void) { return clk::g_last_error.c_str(); }

extern "C" const char* clk_version(void) { return "0.6.0+gfx950"; }

extern "C" int clk_set_stage_events(void* const* events, int32_t count) {
    if (count < 0 || count > clk::kMaxStages || (count > 0 && events == nullptr)) {
        return clk::invalid("clk_set_stage_events: count must be 0.." + std::to_string(clk::kMaxStages));
    }
    for (int i = 0; i < clk::kMaxStages; ++i) clk::g_stage_events[i] = i < count ? events[i] : nullptr;
    clk::g_stage_count = count;
    return clk::ok();
}
