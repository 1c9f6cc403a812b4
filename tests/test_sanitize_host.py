"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer, built with
gcc/g++ on their own (no device code): the C oracle, the SIMD CPU encoder
(flat and batched) and the engine's host GF(2^8) code
(megatron-lm_amd/csrc/gf256.cpp), driven by tests/sanitize_driver.c; and the
staging entry points' multi-threaded host copies
(megatron-lm_amd/csrc/host_copy.cpp), driven by tests/sanitize_copy_driver.cpp;
and the kernels' division by a launch-time divisor (csrc/fastdiv.h), driven by
tests/fastdiv_driver.cpp."""
import os
import subprocess

from conftest import ROOT

SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
# The environment is passed through as it is; a library the environment
# preloads ahead of the ASan runtime is tolerated rather than removed.
ASAN_OPTIONS = "detect_leaks=1:verify_asan_link_order=0"


def test_host_code_is_sanitizer_clean(tmp_path):
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "oracle")]
    objs = []
    for src, cc, std in [(os.path.join(ROOT, "oracle", "ec_oracle.c"), "gcc", "-std=c11"),
                         (os.path.join(ROOT, "oracle", "ec_cpu_fast.c"), "gcc", "-std=c11"),
                         (os.path.join(ROOT, "megatron-lm_amd", "csrc", "gf256.cpp"), "g++", "-std=c++17"),
                         (os.path.join(ROOT, "tests", "sanitize_driver.c"), "gcc", "-std=c11")]:
        obj = str(tmp_path / (os.path.basename(src) + ".o"))
        subprocess.run([cc, std, *SAN, *inc, "-c", src, "-o", obj], check=True)
        objs.append(obj)
    exe = str(tmp_path / "drv")
    subprocess.run(["g++", *SAN, *objs, "-o", exe, "-pthread"], check=True)
    env = dict(os.environ, ASAN_OPTIONS=ASAN_OPTIONS, UBSAN_OPTIONS="print_stacktrace=1")
    out = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert out.returncode == 0, out.stderr[-4000:]
    assert "sanitize driver ok" in out.stdout


def test_staging_host_copies_are_sanitizer_clean(tmp_path):
    csrc = os.path.join(ROOT, "megatron-lm_amd", "csrc")
    exe = str(tmp_path / "copydrv")
    subprocess.run(["g++", "-std=c++17", *SAN, "-I", csrc,
                    os.path.join(csrc, "host_copy.cpp"),
                    os.path.join(ROOT, "tests", "sanitize_copy_driver.cpp"),
                    "-o", exe, "-pthread"], check=True)
    env = dict(os.environ, ASAN_OPTIONS=ASAN_OPTIONS, UBSAN_OPTIONS="print_stacktrace=1")
    out = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert out.returncode == 0, out.stderr[-4000:]
    assert "sanitize copy driver ok" in out.stdout


def test_fast_division_matches_hardware_divide(tmp_path):
    """The kernels' division by a launch-time divisor (csrc/fastdiv.h),
    compiled for the host, against the hardware divide."""
    csrc = os.path.join(ROOT, "megatron-lm_amd", "csrc")
    exe = str(tmp_path / "fastdiv")
    subprocess.run(["g++", "-std=c++17", *SAN, "-D__host__=", "-D__device__=",
                    "-D__forceinline__=inline", "-I", csrc,
                    os.path.join(ROOT, "tests", "fastdiv_driver.cpp"), "-o", exe], check=True)
    env = dict(os.environ, ASAN_OPTIONS=ASAN_OPTIONS, UBSAN_OPTIONS="print_stacktrace=1")
    out = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    assert "fastdiv driver ok" in out.stdout
