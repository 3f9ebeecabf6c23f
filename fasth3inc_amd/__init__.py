"""fasth3inc_amd -- MI355X (gfx950) implementation of fh3's Q4_K linear layer.

The product is the C-ABI library fasth3inc_amd/lib/libfh3hip.so (headers in
include/fh3/); fasth3inc_amd.fh3 is its Python binding.
"""
from . import fh3  # noqa: F401
