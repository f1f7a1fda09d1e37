"""The MI355X (gfx950, CDNA4) provider: hand-written HIP kernels over a C ABI."""
