"""The kernel names bench.py reports beside its roofline (KERNEL_NAMES,
RECALL_NAMES, BATCH_ATTN_NAMES) name kernels the built HIP library holds, so
that a record's `rocprof_kernels` can be found in a rocprofv3 summary of the
same build.  Template arguments written as placeholders (EPL, G, RT, SPINOR)
match any value; every other argument must match exactly.  CPU only: reads
the library's symbol table, runs nothing on a device."""
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
LIB = os.path.join(ROOT, "shannon-prime-system_amd", "lib", "libsp_hipkv.so")
PLACEHOLDERS = {"EPL", "G", "RT", "SPINOR"}


def _kernel_symbols():
    out = subprocess.run(["nm", "-C", LIB], capture_output=True, text=True, check=True).stdout
    return [ln.split(" ", 2)[2] for ln in out.splitlines() if ln.count(" ") >= 2 and "kvd::" in ln]


def _pattern(name):
    """'kvd::k_x<EPL, G, false, 12>' -> a regex over demangled kernel symbols."""
    m = re.fullmatch(r"(kvd::[A-Za-z_0-9]+)(?:<([^>]*)>)?", name)
    assert m, name
    rx = r"(?:void )?" + re.escape(m.group(1)).replace(r"kvd::", r"kvd::(?:\(anonymous namespace\)::)?")
    if m.group(2) is not None:
        args = [a.strip() for a in m.group(2).split(",")]
        rx += "<" + ", ".join(r"[^,<>]+" if a in PLACEHOLDERS else re.escape(a) for a in args) + ">"
    return re.compile(rx + r"\(")


def _names():
    import bench
    for lst in bench.KERNEL_NAMES.values():
        yield from lst
    yield from bench.RECALL_NAMES.values()
    yield from bench.BATCH_ATTN_NAMES.values()


def _kernels(entry):
    # "[a + b]" marks float-mode launches, "(layer 0)" a note
    entry = re.sub(r"\s*\([^)]*\)\s*$", "", entry.strip().strip("[]"))
    return [k.strip() for k in entry.split(" + ")]


@pytest.mark.skipif(not os.path.exists(LIB) or not shutil.which("nm"), reason="the HIP library is not built")
def test_reported_kernel_names_exist_in_the_library():
    syms = _kernel_symbols()
    assert syms, "no kernel symbols found"
    missing = [k for e in _names() for k in _kernels(e) if not any(_pattern(k).match(s) for s in syms)]
    assert not missing, f"bench.py names kernels the library does not hold: {missing}"


def test_a_stale_template_argument_is_caught():
    syms = ["void kvd::k_attn_exact_vsum<4, 2, false, 12>(kvd::AttnArgs)"]
    assert _pattern("kvd::k_attn_exact_vsum<EPL, G, false, 12>").match(syms[0])
    assert not _pattern("kvd::k_attn_exact_vsum<EPL, G, false, 8>").match(syms[0])
