"""MI355X-native HBF access-timing engine (HIP kernels behind a C ABI)."""
