// Library-level C-ABI entry points: version, string ownership, device description.
#include <cstdio>
#include <cstdlib>
#include <string>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {

char *dup_string(const std::string &s) {
    char *p = static_cast<char *>(std::malloc(s.size() + 1));
    if (!p) return nullptr;
    for (size_t i = 0; i < s.size(); ++i) p[i] = (s[i] == '\0') ? ' ' : s[i];  // ffi.rs:210
    p[s.size()] = '\0';
    return p;
}

}  // namespace cfh

using namespace cfh;

extern "C" {

const char *castforge_hip_version(void) { return "castforge-hip 0.1.0 (gfx950)"; }

void castforge_hip_free_string(char *ptr) { std::free(ptr); }

int32_t castforge_hip_device_info(char **out_json, char **out_error) {
    if (out_json) *out_json = nullptr;
    return guarded(out_error, [&] {
        require(out_json != nullptr, "out_json must not be NULL");
        int dev = 0;
        check_hip(hipGetDevice(&dev), "hipGetDevice");
        hipDeviceProp_t p;
        check_hip(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
        char buf[512];
        std::snprintf(buf, sizeof buf,
                      "{\"device\":%d,\"name\":\"%s\",\"arch\":\"%s\",\"cus\":%d,"
                      "\"hbm_bytes\":%zu,\"l2_bytes\":%d,\"clock_khz\":%d,\"lds_per_block\":%zu}",
                      dev, p.name, p.gcnArchName, p.multiProcessorCount, p.totalGlobalMem,
                      p.l2CacheSize, p.clockRate, p.sharedMemPerBlock);
        *out_json = dup_string(buf);
    });
}

}  // extern "C"
