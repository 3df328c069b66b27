// dlopen of the HIP runtime (see hip_api.hpp).

#include "hip_api.hpp"

#include <dlfcn.h>

#include <cstdlib>
#include <mutex>

#include "host.hpp"

namespace mxh {

namespace {

HipApi g_api;
std::once_flag g_once;
std::string g_fail;

void load() {
    // A runtime already in the process (e.g. one a host framework loaded) is
    // reused rather than loaded twice; otherwise the usual names, then the
    // default ROCm location. MAXIM_HIP_LIB overrides all of them.
    const char *names[] = {"libamdhip64.so.7", "libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"};
    void *so = nullptr;
    std::string path;
    if (const char *env = std::getenv("MAXIM_HIP_LIB")) {
        so = dlopen(env, RTLD_NOW | RTLD_GLOBAL);
        path = env;
    }
    for (const char *n : names) {
        if (so) break;
        so = dlopen(n, RTLD_NOW | RTLD_GLOBAL | RTLD_NOLOAD);
        path = n;
    }
    for (const char *n : names) {
        if (so) break;
        so = dlopen(n, RTLD_NOW | RTLD_GLOBAL);
        path = n;
    }
    if (!so) {
        const char *e = dlerror();
        g_fail = std::string("cannot load the HIP runtime (libamdhip64.so): ") + (e ? e : "not found");
        return;
    }
    g_api.so = so;
    g_api.path = path;
#define MXH_FN(ret, name, ...)                                                       \
    g_api.name = reinterpret_cast<ret (*)(__VA_ARGS__)>(dlsym(so, #name));           \
    if (!g_api.name) {                                                               \
        g_fail = "the HIP runtime at " + path + " has no " #name;                    \
        g_api.so = nullptr;                                                          \
        return;                                                                      \
    }
#include "hip_api.inc"
#undef MXH_FN
}

}  // namespace

HipApi &hip() {
    std::call_once(g_once, load);
    if (!g_api.so) throw mx::Error(g_fail);
    return g_api;
}

void check(hipError_t rc, const char *what) {
    if (rc == 0) return;
    const char *msg = g_api.hipGetErrorString ? g_api.hipGetErrorString(rc) : "unknown";
    throw mx::Error(std::string(what) + " failed: " + msg + " (hipError " + std::to_string(rc) + ")");
}

}  // namespace mxh
