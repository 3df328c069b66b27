// The gfx950 code object: every kernel the HIP executor launches, in one
// translation unit so hipcc emits one code object the host embeds.
#include "stream_ops.h"
#include "gemm.h"
#include "conv.h"
#include "conv3.h"
#include "pointwise.h"
