"""Host entry points over the HIP kernels (Kernels/ of the reference)."""
