"""The C-ABI from plain C: tests/c_abi/abi_host.c is compiled with gcc as C11
against include/k3h.h and linked to the built libk3h.so, then run on the host
(argument checks only, no GPU), and the header also compiles as C++.
tests/c_abi/abi_gpu.c drives the library from a plain C host on the GPU (HIP
runtime C API for device memory, the typed call and the manifest path through
k3h_launch) against the C oracle: compiled here, run by the gpu-marked test."""
import os
import shutil
import subprocess

import pytest

import k3h
import oracle as O

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not on PATH")
def test_header_and_library_from_c(tmp_path):
    k3h.lib()  # the library exists (built by __graft_entry__.build())
    exe = tmp_path / "abi_host"
    cmd = ["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(REPO, "include"),
           os.path.join(REPO, "tests", "c_abi", "abi_host.c"), "-L", k3h.BUILD, "-lk3h",
           f"-Wl,-rpath,{k3h.BUILD}", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe), k3h.BUILD], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c-abi host checks ok" in r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not on PATH")
def test_header_compiles_as_cxx(tmp_path):
    src = tmp_path / "h.cpp"
    src.write_text('#include "k3h.h"\nint main() { return k3h_error_string(K3H_OK) ? 0 : 1; }\n')
    r = subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-fsyntax-only", "-I",
                        os.path.join(REPO, "include"), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def _build_gpu_host(tmp_path):
    k3h.lib()
    O.lib()
    lib_o = os.path.dirname(O.LIB_PATH)
    exe = tmp_path / "abi_gpu"
    cmd = ["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(ROCM, "include"), "-I", os.path.join(REPO, "include"),
           "-I", os.path.join(REPO, "oracle"), os.path.join(REPO, "tests", "c_abi", "abi_gpu.c"),
           "-L", k3h.BUILD, "-lk3h", "-L", lib_o, "-lk3oracle", "-L", os.path.join(ROCM, "lib"),
           "-lamdhip64", f"-Wl,-rpath,{k3h.BUILD}:{lib_o}:{os.path.join(ROCM, 'lib')}", "-o",
           str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


@pytest.mark.skipif(shutil.which("gcc") is None or not os.path.isdir(os.path.join(ROCM, "include")),
                    reason="gcc or the ROCm headers missing")
def test_gpu_host_program_builds(tmp_path):
    _build_gpu_host(tmp_path)


@pytest.mark.gpu
def test_c_host_gpu_parity(tmp_path):
    """Typed call and manifest launch from plain C, byte for byte against the oracle."""
    exe = _build_gpu_host(tmp_path)
    r = subprocess.run([str(exe), k3h.BUILD], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c-abi gpu parity ok" in r.stdout
