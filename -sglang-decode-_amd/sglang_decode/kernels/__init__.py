"""Launch wrappers over the C ABI (kernels are in ../csrc)."""
