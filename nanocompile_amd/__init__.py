"""nanocompile_amd: an MI355X (gfx950) backend for nanocompile's int8 hot path.

The int8 projections (per-row int8 weights, per-token int8 activations, exact
int32 accumulation, an fp32 epilogue) and the fused groups around them run as
hand-written HIP kernels in one library (``_lib/libnc_hip.so``), called over
ctypes with the reference's kernel calling convention. Nothing here runs on
the CPU in place of the GPU: without the library or a device, calls raise.
"""

__all__ = ["hip", "kernels"]
