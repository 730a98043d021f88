"""Build and load libkvip_hip.so (the gfx950 HIP kernels behind the C ABI)."""
