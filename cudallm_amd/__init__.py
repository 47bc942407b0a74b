"""cudallm_amd: the batch-1 decode hot path of cudallm, native to MI355X (gfx950).

The product is ``libcudallm.so`` (C ABI in ``include/cudallm/cudallm.h``; C++ host code and
hand-written HIP kernels under ``csrc/``).  This package is its Python side, mirroring the
reference's ``python/cudallm`` modules that drive the same ABI:

* ``engine``   - ctypes binding: ``Engine``, ``CudaLLMError``, ``kernel_*`` hooks.
* ``format``   - ``.cudallm`` reader / writer.
* ``quantize`` - int8 / int4 weight quantisers, run on the GPU.
* ``synth``    - seeded synthetic Llama-3.2-1B-shaped model files.
"""
from .engine import LIB_PATH, CudaLLMError, Engine

__version__ = "0.1.0"
__all__ = ["CudaLLMError", "Engine", "LIB_PATH", "__version__"]
