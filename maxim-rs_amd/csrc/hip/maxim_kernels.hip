// The gfx950 code object: every kernel the HIP executor launches, in one
// translation unit so hipcc emits one code object the host embeds.
#include "stream_ops.h"
#include "gemm.h"
#include "conv.h"
#include "conv3.h"
#include "wino.h"
#include "pointwise.h"

// The scratch of mxh_run_noalloc (channel-mean partial sums and LayerNorm
// statistics, the buffer mxh_new otherwise allocates per executor): one
// array per device, allocated when the code object is loaded and kept until
// the process ends. No kernel names it; the host looks its device address up
// once per device (hipModuleGetGlobal, the module API's symbol lookup, hence
// external linkage: a static array has no symbol to find) and passes that
// address as the kernels' scratch argument. MXK_NOALLOC_SCRATCH_FLOATS
// (kargs.h) is its size.
__device__ __align__(256) float scratch[MXK_NOALLOC_SCRATCH_FLOATS];
