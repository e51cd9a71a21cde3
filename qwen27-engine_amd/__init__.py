"""qwen27 fused per-layer ops for MI355X (gfx950): Python host binding of the C ABI in include/q27h.h.

The compute path is the HIP library lib/libq27h.so built from csrc/ (``build_library()``); this package only
hands device pointers and the current HIP stream to it. There is no fallback: if the library is missing or a
launch fails, the call raises. The directory name has a hyphen, so load it by path, e.g.

    spec = importlib.util.spec_from_file_location("qwen27_engine_amd", "<repo>/qwen27-engine_amd/__init__.py",
                                                  submodule_search_locations=["<repo>/qwen27-engine_amd"])
"""
from ._lib import LIB_PATH, Q27Error, build_library, lib  # noqa: F401
from . import gguf, ops  # noqa: F401
