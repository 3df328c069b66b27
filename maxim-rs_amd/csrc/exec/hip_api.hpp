// The HIP runtime, reached through dlopen: the handful of entry points the
// executor needs, declared here with their C signatures so nothing links
// against libamdhip64 at build time and no HIP header is needed on the host
// side. The counterpart of the reference's lightgpu `vm`/`ffi` layer, which
// dlopens libcuda (src/cuda.rs; README.md:17-18).
#pragma once

#include <cstddef>
#include <string>

namespace mxh {

typedef int hipError_t;
typedef struct ihipStream_t *hipStream_t;
typedef struct ihipModule_t *hipModule_t;
typedef struct ihipModuleSymbol_t *hipFunction_t;
typedef struct ihipEvent_t *hipEvent_t;
typedef struct ihipGraph *hipGraph_t;
typedef struct hipGraphExec *hipGraphExec_t;

enum { kMemcpyH2D = 1, kMemcpyD2H = 2, kMemcpyD2D = 3 };
enum { kAttrClockRate = 5, kAttrMultiprocessorCount = 63 };
enum { kCaptureModeGlobal = 0, kCaptureModeThreadLocal = 1, kCaptureModeRelaxed = 2 };

struct HipApi {
    void *so = nullptr;
    std::string path;
#define MXH_FN(ret, name, ...) ret (*name)(__VA_ARGS__) = nullptr;
#include "hip_api.inc"
#undef MXH_FN
};

// Loads the runtime once per process (thread-safe); throws on failure.
HipApi &hip();
// Throws an Error naming the call and HIP's message when rc != 0.
void check(hipError_t rc, const char *what);

}  // namespace mxh
