/* expf, sinf and cosf as this package's nc_math.h computes them, for make_g6.py --math nc.
 * TEST INFRASTRUCTURE ONLY: preloaded (LD_PRELOAD) into the build container's Python when it
 * runs the reference's compiled C, so that the reference's own kernels call the same
 * transcendental functions the GPU kernels do. nc_g6_math_shim lets the recorder check that
 * the preload took effect. */
#include "../../nanocompile_amd/csrc/nc_math.h"

float expf(float x) { return nc_expf(x); }
float sinf(float x) { return nc_sinf(x); }
float cosf(float x) { return nc_cosf(x); }
int nc_g6_math_shim(void) { return 1; }
