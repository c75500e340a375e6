"""Build steps for the engine (and the CPU checker used by the tests).

    python -m bnns_to_c_amd.build          # engine + checker (+ reference C if present)

The engine is built in place with hipcc for gfx950 (csrc/Makefile), so the
shared library travels with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
ORACLE = os.path.join(ROOT, "oracle")
REFERENCE_CSRC = "/root/reference/csrc"


def _make(path: str, *targets: str, force: bool = False) -> None:
    jobs = str(min(8, os.cpu_count() or 1))
    cmd = ["make", "-C", path, "-j", jobs] + (["-B"] if force else []) + list(targets)
    subprocess.run(cmd, check=True)


def build_engine(force: bool = True) -> None:
    _make(CSRC, force=force)


def build_checker(force: bool = True) -> None:
    """CPU restatement of the reference (oracle/) and, where the reference
    sources are present, the reference C itself into oracle/_ref/, and the
    reference's CLI mains built unchanged against include/ and the engine
    (oracle/_ref/dropin/)."""
    _make(ORACLE, force=force)
    if os.path.isdir(REFERENCE_CSRC):
        _make(ORACLE, "ref", "dropin", force=force)


def build_all(force: bool = True) -> None:
    build_engine(force)
    build_checker(force)


if __name__ == "__main__":
    build_all(force="--no-force" not in sys.argv)
