"""The reference's prefill extension under its own module name.

kernels/harness/parity_cuda.py:45-62 builds ``deltanet_chunk_cuda`` from
kernels/chunk_delta_cuda.cu + kernels/torch_binding.cpp and calls its
``chunk_prefill(q, k, v, g, beta, s0)`` positionally (parity_cuda.py:69-72).
This module exposes the gfx950 extension's ops under that name, so a harness
swaps its build step for an import:

    parity_cuda.build_extension = lambda: importlib.import_module("deltanet_chunk_cuda")

with qwen-drive-edge-orin_amd/ on sys.path.  Importing raises when the
extension is not built (no fallback).
"""
from gdn_hip import load as _load

_ext = _load()

chunk_prefill = _ext.chunk_prefill
chunk_prefill_debug = _ext.chunk_prefill_debug
