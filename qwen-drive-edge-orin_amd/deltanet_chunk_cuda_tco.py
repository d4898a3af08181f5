"""The reference's bf16-wmma o-pass twin under its own module name
(kernels/parity_tco.py:15-33 builds ``deltanet_chunk_cuda_tco`` from
kernels/chunk_delta_cuda_tco.cu + kernels/torch_binding_tco.cpp, with the
same op names and signatures as ``deltanet_chunk_cuda``).  Here both names
are the one gfx950 extension:

    parity_cuda.build_extension = lambda: importlib.import_module("deltanet_chunk_cuda_tco")
"""
from deltanet_chunk_cuda import chunk_prefill, chunk_prefill_debug  # noqa: F401
