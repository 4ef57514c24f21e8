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


def test_prefill_ld_vt_guard_rejects_short_last_tile():
    """The prefill kernels read V^T in 32-key tiles without a clamp, so a
    leading dimension that covers n_k only to a multiple of 16 is refused
    (-100) before anything touches the device; the fake pointers are never
    dereferenced."""
    lib = ctypes.CDLL(LIB_PATH)
    fn = lib.khq_prefill_attn_fp16
    fn.argtypes = _lib.SIGNATURES["khq_prefill_attn_fp16"]
    fn.restype = ctypes.c_int
    fake = ctypes.c_void_p(0x1000)
    for n_k in (333, 17, 48 + 16):
        short = (n_k + 15) // 16 * 16
        if short % 32 == 0:
            continue
        rc = fn(fake, fake, fake, short, n_k, 1, 1, 24, 4, 0.0625, fake, None)
        assert rc == -100, (n_k, short, rc)
