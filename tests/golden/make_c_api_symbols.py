"""Writes reference_c_api_symbols.txt: every C entry point the reference's
Python package calls (the names after `_LIB.` in python-package/xgboost/*.py).

Run in a checkout that has the reference at /root/reference:
    python tests/golden/make_c_api_symbols.py
"""
import re
from pathlib import Path

REF = Path("/root/reference/python-package/xgboost")
OUT = Path(__file__).with_name("reference_c_api_symbols.txt")


def main() -> None:
    names = set()
    for path in sorted(REF.rglob("*.py")):
        names.update(re.findall(r"_LIB\.([A-Za-z_][A-Za-z0-9_]*)", path.read_text()))
    names.discard("path")  # the loaded library's file name, not an entry point
    OUT.write_text("".join(f"{n}\n" for n in sorted(names)))
    print(f"{len(names)} names -> {OUT}")


if __name__ == "__main__":
    main()
