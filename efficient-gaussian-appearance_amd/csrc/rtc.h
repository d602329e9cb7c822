// hipRTC kernel specialisation and on-disk code-object cache.
#pragma once
#include <string>
#include <vector>

#include "internal.h"

namespace efgs {

struct RtcKernel {
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
};

void rtc_set_dirs(const std::string& cache_dir, const std::string& kernel_dir);

// compiles (or loads from the cache) the kernel `kernel_name` whose source is `preamble` followed by the files
// (relative to the kernel directory), for the current device
bool rtc_get_kernel(const std::string& kernel_name, const std::string& preamble, const std::vector<std::string>& files, RtcKernel& out);

// compiles into the cache for `arch` without touching a device (build step)
bool rtc_precompile(const std::string& kernel_name, const std::string& preamble, const std::vector<std::string>& files, const std::string& arch);

}  // namespace efgs
