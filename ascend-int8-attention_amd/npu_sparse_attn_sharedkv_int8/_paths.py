"""Package-local native library location (reference _paths.py:1-16)."""
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
NATIVE_DIR = PACKAGE_ROOT / "_native"
LIBRARY_NAME = "libsharedkv_hip.so"


def native_path(filename=LIBRARY_NAME):
    path = NATIVE_DIR / filename
    if not path.is_file():
        raise RuntimeError(
            f"Missing native library {filename}. Build it first: "
            "python -c 'import __graft_entry__ as g; g.build()' from the repository root.")
    return path
