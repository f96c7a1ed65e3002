"""ggml-compiler's quantized mat-mul / KV-cache attention path on MI355X (gfx950), via libgcq."""

from ._lib import GcqError, library_path, load
from .runtime import has_backend, quantize, version

__all__ = ["GcqError", "library_path", "load", "has_backend", "quantize", "version"]
