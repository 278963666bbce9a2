"""silarray_amd — MI355X (gfx950) backend for the silarray GPU hot path.

The product is the C ABI library libsilgpu.so (include/silgpu.h) and the C++
front end under silarray_amd/include (sil::array, sil::gpu, sil::storage).
`silarray_amd._native` is the ctypes binding of the C ABI used by the test
suite and bench.py.
"""

from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
LIB_PATH = PACKAGE_DIR / "libsilgpu.so"
INCLUDE_DIR = PACKAGE_DIR / "include"
