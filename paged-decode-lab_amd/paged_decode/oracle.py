"""Import-compatibility module for ``from paged_decode.oracle import Layout``.

The reference exposes its layout record and metadata validator from
``paged_decode.oracle`` (reference ``src/paged_decode/oracle.py:11-47``). Only
those two product-side names are re-exported here so that caller code keeps
working unchanged. The FP64 reference mathematics is not part of this package:
it lives in the repository's top-level ``oracle`` directory as test
infrastructure and is never imported by the decode path.
"""
from .layout import Layout, validate_metadata

__all__ = ["Layout", "validate_metadata"]
