"""The host C++ under AddressSanitizer and UndefinedBehaviorSanitizer (CPU):
the oracle (oracle/opure_oracle.cpp) and the engine's host code -- page pool,
safetensors reader, model-directory loader and the C-ABI over them
(opure-voxelengine_amd/engine/*.cpp) -- are built with
-fsanitize=address,undefined (host code only, g++), and the CPU tests that
drive them run in a child process against those builds.  Any report fails the
child (halt on the first error), and so the test."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


def _build(tmp):
    oracle = os.path.join(tmp, "liboracle_san.so")
    subprocess.run(["g++", "-std=c++20", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", *SAN,
                    "-o", oracle, os.path.join(ROOT, "oracle", "opure_oracle.cpp")], check=True)
    eng_dir = os.path.join(ROOT, "opure-voxelengine_amd", "engine")
    lib_dir = os.path.join(ROOT, "opure-voxelengine_amd", "lib")
    engine = os.path.join(tmp, "libopure_engine_san.so")
    srcs = sorted(os.path.join(eng_dir, f) for f in os.listdir(eng_dir) if f.endswith(".cpp"))
    subprocess.run(["g++", "-std=c++20", "-fPIC", "-shared", *SAN, "-I", os.path.join(ROOT, "include"), "-I", eng_dir,
                    "-o", engine, *srcs, f"-L{lib_dir}", "-lopure_hip", f"-Wl,-rpath,{lib_dir}"], check=True)
    return oracle, engine


def test_host_code_under_asan_and_ubsan(tmp_path):
    if not os.path.exists(os.path.join(ROOT, "opure-voxelengine_amd", "lib", "libopure_hip.so")):
        pytest.skip("libopure_hip.so is not built")
    oracle, engine = _build(str(tmp_path))
    def gxx_file(name):
        return subprocess.run(["g++", f"-print-file-name={name}"], capture_output=True, text=True, check=True).stdout.strip()
    # the sanitizer runtime first; libstdc++ with it, so that its exception
    # interceptors find the real functions (python itself does not link libstdc++)
    env = dict(os.environ)
    env.update(LD_PRELOAD=f"{gxx_file('libasan.so')}:{gxx_file('libstdc++.so')}", OPURE_ORACLE_LIB=oracle, OPURE_ENGINE_LIB=engine, OMP_NUM_THREADS="4",
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    tests = ["tests/test_oracle_kernels.py", "tests/test_oracle_accept.py", "tests/test_oracle_forward.py",
             "tests/test_oracle_numerics.py", "tests/test_page_pool.py", "tests/test_loader.py"]
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-m", "not gpu and not slow", "-p", "no:cacheprovider",
                        *tests], cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "AddressSanitizer" not in r.stdout + r.stderr and "runtime error" not in r.stderr, tail
    import re
    n = re.search(r"(\d+) passed", r.stdout)
    assert n and int(n.group(1)) >= 60, tail                      # the suites ran, not just collected
