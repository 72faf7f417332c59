"""The kernels' exp against the function the reference calls.

The reference's softmax uses Rust's f32::exp, i.e. the C library's expf
(tensor.rs:745-754).  The kernels evaluate a restatement of glibc's published
table-driven expf (marian-edge_amd/csrc/ref_expf.h); here that same header is
compiled for the host and compared with the host's expf on every fp32 input,
and its 2^(i/32) table is re-derived from the mathematics."""

import re
import struct
import subprocess
from decimal import Decimal, getcontext
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "marian-edge_amd" / "csrc" / "ref_expf.h"


def _table():
    text = HEADER.read_text()
    body = text[text.index("#define MH_EXP2_TABLE_32"):text.index("namespace mh")]
    return [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ULL", body)]


def test_exp2_table_is_derived_from_the_mathematics():
    getcontext().prec = 60
    ln2 = Decimal(2).ln()
    tab = _table()
    assert len(tab) == 32
    for i, t in enumerate(tab):
        nearest = float((ln2 * i / 32).exp())  # 2^(i/32), correctly rounded
        bits = struct.unpack("<Q", struct.pack("<d", nearest))[0]
        assert t == bits - (i << 47), i


def _has_fma():
    try:
        return " fma " in Path("/proc/cpuinfo").read_text().replace("\n", " ")
    except OSError:
        return False


@pytest.mark.skipif(not _has_fma(), reason="the host C library takes its FMA path only on FMA CPUs")
def test_kernel_exp_equals_host_expf_on_every_input(tmp_path):
    exe = tmp_path / "expf_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-fopenmp", "-mfma", "-ffp-contract=off",
                    f"-I{HEADER.parent}", str(ROOT / "tests" / "expf_check.cpp"), "-o", str(exe)],
                   check=True)
    res = subprocess.run([str(exe), "1"], capture_output=True, text=True, timeout=900)
    print(res.stdout.strip())
    assert res.returncode == 0, res.stdout
    assert res.stdout.startswith(f"checked {1 << 32} mismatches 0")
