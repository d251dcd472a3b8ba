"""MI355X (gfx950) GGUF quantized linear-layer path for gollek.

The compute lives in libgollek_hip.so (HIP kernels behind the C ABI of
include/gollek_hip.h); tensor_ops mirrors gollek's GgufTensorOps facade over
it.  Importing the package does not load the library; the first call does, and
fails loudly if it has not been built.
"""
__all__ = ["tensor_ops", "synthetic", "build"]
