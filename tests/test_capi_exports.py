"""The C-ABI library loads (no GPU needed to load it) and exports every
function include/khq.h declares, with no extra C symbols."""
import ctypes
import os
import re
import subprocess

from khq import _lib
from khq.build import LIB_PATH

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "khq.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(\w+)\(", src, flags=re.M))


def test_header_symbols_exported():
    names = declared()
    assert "launch_khq_attn_fp16" in names and len(names) == 42
    lib = ctypes.CDLL(LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    c_syms = {s for s in exported if not s.startswith("_")}
    assert c_syms == names, c_syms ^ names


def test_binding_table_matches_header():
    assert set(_lib.SIGNATURES) | {"khq_version"} == declared()
    assert _lib.version().startswith("khq-mi355x")
