// hipRTC specialisation of the preprocess kernels: assembles the source from a token preamble plus the
// shared headers and the kernel file, compiles it for the device architecture, caches the code object on disk
// keyed by a hash of source and options, and keeps loaded modules per device.
// Reference counterpart: B/rasterization/src/appearance.cu:78-142 (NVRTC source assembly, PTX cache).
#include "rtc.h"

#include <hip/hiprtc.h>

#include <cstdio>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>
#include <vector>

namespace efgs {

namespace {

std::mutex g_mutex;
std::string g_cache_dir;
std::string g_kernel_dir;
std::map<std::string, RtcKernel> g_loaded;  // key: device + hash

uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ull) {
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

bool read_file(const std::string& path, std::string& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::stringstream ss;
    ss << f.rdbuf();
    out = ss.str();
    return true;
}

// drops '#pragma once' lines so the headers can be concatenated into one translation unit
std::string strip_pragma_once(const std::string& s) {
    std::string out;
    out.reserve(s.size());
    std::istringstream in(s);
    std::string line;
    while (std::getline(in, line)) {
        if (line.rfind("#pragma once", 0) == 0) continue;
        out += line;
        out += '\n';
    }
    return out;
}

std::vector<std::string> compile_options(const std::string& arch) {
    return {"--offload-arch=" + arch, "-O3", "-std=c++17", "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
}

struct Prepared {
    std::string source;
    std::vector<std::string> options;
    std::string hash;
};

bool prepare(const std::string& preamble, const std::vector<std::string>& files, const std::string& kernel_dir, const std::string& arch,
             Prepared& p) {
    p.source = "#define EFGS_RTC 1\n"
               "typedef __hip_internal::uint16_t uint16_t;\n"
               "typedef __hip_internal::uint32_t uint32_t;\n"
               "typedef __hip_internal::uint64_t uint64_t;\n"
               "typedef __hip_internal::int32_t int32_t;\n" +
               preamble;
    for (const std::string& f : files) {
        std::string text;
        if (!read_file(kernel_dir + "/" + f, text)) {
            set_error("cannot read hipRTC source " + kernel_dir + "/" + f);
            return false;
        }
        p.source += "\n" + strip_pragma_once(text);
    }
    p.options = compile_options(arch);
    std::string opt_text;
    for (const auto& o : p.options) opt_text += o + " ";
    char hash[32];
    std::snprintf(hash, sizeof(hash), "%016llx", static_cast<unsigned long long>(fnv1a(opt_text, fnv1a(p.source))));
    p.hash = hash;
    return true;
}

bool compile(const std::string& kernel_name, const Prepared& p, std::string& code) {
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, p.source.c_str(), (kernel_name + ".hip").c_str(), 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
        set_error("hiprtcCreateProgram failed for " + kernel_name);
        return false;
    }
    std::vector<const char*> copts;
    for (const auto& o : p.options) copts.push_back(o.c_str());
    const hiprtcResult r = hiprtcCompileProgram(prog, static_cast<int>(copts.size()), copts.data());
    if (r != HIPRTC_SUCCESS) {
        size_t log_size = 0;
        hiprtcGetProgramLogSize(prog, &log_size);
        std::string log(log_size, '\0');
        if (log_size) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        set_error("hipRTC compilation of " + kernel_name + " failed: " + log);
        return false;
    }
    size_t code_size = 0;
    hiprtcGetCodeSize(prog, &code_size);
    code.assign(code_size, '\0');
    hiprtcGetCode(prog, &code[0]);
    hiprtcDestroyProgram(&prog);
    return true;
}

// writes through a temporary file and a rename, so concurrent readers never see a partial code object
void store(const std::string& path, const std::string& code) {
    const std::string tmp = path + ".tmp" + std::to_string(static_cast<unsigned long long>(fnv1a(path + code.substr(0, 64))));
    std::ofstream f(tmp, std::ios::binary);
    if (!f) return;
    f.write(code.data(), static_cast<std::streamsize>(code.size()));
    f.close();
    std::rename(tmp.c_str(), path.c_str());
}

std::string cache_path(const std::string& cache_dir, const std::string& kernel_name, const std::string& arch, const std::string& hash) {
    return cache_dir.empty() ? std::string() : cache_dir + "/" + kernel_name + "_" + arch + "_" + hash + ".hsaco";
}

}  // namespace

void rtc_set_dirs(const std::string& cache_dir, const std::string& kernel_dir) {
    std::lock_guard<std::mutex> lock(g_mutex);
    g_cache_dir = cache_dir;
    g_kernel_dir = kernel_dir;
}

bool rtc_get_kernel(const std::string& kernel_name, const std::string& preamble, const std::vector<std::string>& files, RtcKernel& out) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_kernel_dir.empty()) {
        set_error("hipRTC kernel directory not set (efgs_set_rtc_dirs)");
        return false;
    }
    int device = 0;
    EFGS_HIP_CHECK(hipGetDevice(&device));
    hipDeviceProp_t prop;
    EFGS_HIP_CHECK(hipGetDeviceProperties(&prop, device));
    std::string arch = prop.gcnArchName;
    const size_t colon = arch.find(':');
    if (colon != std::string::npos) arch = arch.substr(0, colon);
    Prepared p;
    if (!prepare(preamble, files, g_kernel_dir, arch, p)) return false;
    const std::string key = std::to_string(device) + ":" + p.hash;
    auto it = g_loaded.find(key);
    if (it != g_loaded.end()) {
        out = it->second;
        return true;
    }
    const std::string path = cache_path(g_cache_dir, kernel_name, arch, p.hash);
    std::string code;
    if (path.empty() || !read_file(path, code) || code.empty()) {
        if (!compile(kernel_name, p, code)) return false;
        if (!path.empty()) store(path, code);
    }
    RtcKernel k;
    EFGS_HIP_CHECK(hipModuleLoadData(&k.module, code.data()));
    EFGS_HIP_CHECK(hipModuleGetFunction(&k.function, k.module, kernel_name.c_str()));
    g_loaded[key] = k;
    out = k;
    return true;
}

bool rtc_precompile(const std::string& kernel_name, const std::string& preamble, const std::vector<std::string>& files, const std::string& arch) {
    std::string cache_dir, kernel_dir;
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        cache_dir = g_cache_dir;
        kernel_dir = g_kernel_dir;
    }
    if (cache_dir.empty() || kernel_dir.empty()) {
        set_error("hipRTC cache or kernel directory not set (efgs_set_rtc_dirs)");
        return false;
    }
    Prepared p;
    if (!prepare(preamble, files, kernel_dir, arch, p)) return false;
    const std::string path = cache_path(cache_dir, kernel_name, arch, p.hash);
    std::string code;
    if (read_file(path, code) && !code.empty()) return true;
    if (!compile(kernel_name, p, code)) return false;
    store(path, code);
    return true;
}

}  // namespace efgs
