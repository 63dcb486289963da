"""quail_amd: Quail's packed-prompt prefill pass for Qwen3 FP8 on MI355X (gfx950).

Host side (this package): prefix tree, page arena, admission, pack layout,
the Engine primitives and the Qwen3 pipeline, readouts and the stage loop,
mirroring quail/backends/quail/executor. Device side: hand-written HIP
kernels in csrc/, built into libquail_mi355x.so and reached through the C
ABI declared in include/quail_mi355x.h.
"""

__version__ = "0.1.0"
