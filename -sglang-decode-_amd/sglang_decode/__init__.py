"""MI355X (gfx950) persistent paged GQA decode attention for SGLang.

Importing the package does not touch the GPU or load the native library; the
library is loaded on first use by sglang_decode._lib.
"""
__version__ = "0.1.0"
