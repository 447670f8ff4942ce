"""Builds tests/expf_sweep.cpp (the exhaustive binary32 exp checks) with the
host g++ into a temporary folder and runs it."""
import os
import subprocess
import tempfile
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
SOURCE = ROOT / "tests" / "expf_sweep.cpp"
HEADER_DIR = ROOT / "xgboost-metal_amd" / "csrc"

_binary = None


def sweep_binary() -> Path:
    global _binary
    if _binary is None:
        out = Path(tempfile.mkdtemp(prefix="expf_sweep_")) / "expf_sweep"
        subprocess.run(["g++", "-O2", "-march=native", "-std=c++17", "-fopenmp", "-ffp-contract=off",
                        "-fno-fast-math", f"-I{HEADER_DIR}", "-o", str(out), str(SOURCE), "-lm"], check=True)
        _binary = out
    return _binary


def run(mode: str) -> str:
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(16, os.cpu_count() or 8)))
    return subprocess.run([str(sweep_binary()), mode], check=True, capture_output=True, text=True,
                          env=env).stdout
