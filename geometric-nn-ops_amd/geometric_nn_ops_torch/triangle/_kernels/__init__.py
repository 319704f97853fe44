"""Host launchers of the gfx950 HIP kernels (through the libgnn_hip.so C ABI)."""
