"""maxim_amd: Python bindings of the MI355X MAXIM executor.

`plan` wraps the plan contract (include/maxim_plan.h): the graph builder, the
packed arena, checkpoints, padding. `hip` wraps the gfx950 executor
(include/maxim_hip.h). Both are ctypes over lib/libmaxim_hip.so.
"""

from . import plan  # noqa: F401
