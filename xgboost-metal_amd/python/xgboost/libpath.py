"""Locate libxgboost.so (reference python-package/xgboost/libpath.py:19-75)."""
import os
from pathlib import Path


class XGBoostLibraryNotFound(Exception):
    """Raised when the native library is missing."""


def find_lib_path() -> str:
    here = Path(__file__).resolve().parent
    candidates = [here / "lib" / "libxgboost.so"]
    env = os.environ.get("XGBOOST_HIP_LIBRARY")
    if env:
        candidates.insert(0, Path(env))
    for path in candidates:
        if path.exists():
            return str(path)
    raise XGBoostLibraryNotFound(
        "libxgboost.so was not found; build it with `python -c 'import __graft_entry__ as g; g.build()'` "
        f"(looked in {[str(c) for c in candidates]})")
