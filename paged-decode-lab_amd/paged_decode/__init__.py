"""Split-K paged GQA decode attention for AMD Instinct MI355X (gfx950).

Drop-in for the ``paged_decode`` package of paged-decode-lab
(reference ``src/paged_decode/__init__.py:1-3``). Importing this package never
compiles or loads native code; ``paged_decode.runtime.load_extension`` does
that, once, at plan construction.
"""

__version__ = "0.3.0+mi355x"
