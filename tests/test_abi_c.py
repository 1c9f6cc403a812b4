"""The C ABI from C: the header is strict C, and a plain-C program linked
against libec_mi355.so encodes, reconstructs and XORs on the GPU, and codes a
checkpoint snapshot and stages it to host memory (row-major, then stripe-major on
a copy engine)."""
import os
import subprocess

import pytest

from conftest import ROOT

DEMO = os.path.join(ROOT, "megatron-lm_amd", "examples", "ec_abi_demo")


def test_header_is_strict_c(tmp_path):
    src = tmp_path / "h.c"
    src.write_text('#include "ec_mi355.h"\nint main(void) { return ec_abi_version() == EC_ABI_VERSION ? 0 : 1; }\n')
    for std in ("c99", "c11"):
        subprocess.run(["gcc", f"-std={std}", "-pedantic", "-Wall", "-Werror", "-fsyntax-only",
                        "-I", os.path.join(ROOT, "include"), str(src)], check=True)
    subprocess.run(["g++", "-std=c++11", "-pedantic", "-Wall", "-Werror", "-fsyntax-only",
                    "-x", "c++", "-I", os.path.join(ROOT, "include"), str(src)], check=True)


@pytest.mark.gpu
@pytest.mark.parametrize("nbytes", [(1 << 20) + 3, 64 << 20, 1])
def test_c_program_round_trip(nbytes):
    if not os.path.exists(DEMO):
        pytest.fail(f"{DEMO} is not built (make -C megatron-lm_amd)")
    out = subprocess.run([DEMO, str(nbytes)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert "ec_abi_demo ok" in out.stdout
