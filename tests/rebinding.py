"""The reference-side rebinding of ``load_extension()`` as INTEGRATION.md gives it.

``snippet()`` extracts the replacement function from the documentation
itself (the Python block after the ``rebinding-snippet`` marker), so the
tests that run it and the text a maintainer copies cannot drift apart.
``load_as_documented()`` runs that block in a fresh namespace and calls it,
which loads ``_C.so`` by file location under the module name the snippet
chooses, the way a reference package rebound to this build would.
"""
import os
import re
from functools import lru_cache
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
INTEGRATION = REPO / "INTEGRATION.md"
PACKAGE_ROOT = REPO / "paged-decode-lab_amd"
MARKER = "<!-- rebinding-snippet -->"


def snippet():
    """Source of the replacement ``load_extension`` (decorator included)."""
    text = INTEGRATION.read_text()
    after = text[text.index(MARKER) + len(MARKER):]
    block = re.search(r"```python\n(.*?)```", after, re.S)
    assert block is not None, "no python block after the rebinding marker"
    return block.group(1)


@lru_cache(maxsize=None)
def load_as_documented(root=PACKAGE_ROOT):
    """The extension module, loaded by the documented ``load_extension()``
    (once per root, as the reference caches its extension)."""
    namespace = {"lru_cache": lru_cache, "__name__": "paged_decode.runtime"}
    exec(compile(snippet(), str(INTEGRATION), "exec"), namespace)
    previous = os.environ.get("PAGED_DECODE_AMD")
    os.environ["PAGED_DECODE_AMD"] = str(root)
    try:
        return namespace["load_extension"]()
    finally:
        if previous is None:
            os.environ.pop("PAGED_DECODE_AMD", None)
        else:
            os.environ["PAGED_DECODE_AMD"] = previous
