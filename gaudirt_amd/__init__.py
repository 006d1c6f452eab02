"""MI355X-native paged-attention path of GaudiRT (gfx950 HIP kernels behind a C ABI)."""
