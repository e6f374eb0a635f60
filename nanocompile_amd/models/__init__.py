"""Model drivers over the HIP kernels: the callers of the int8 hot path."""
