"""CPU checks of the C-ABI library: it loads, exports every function that
include/k3h.h declares, and rejects bad arguments on the host before any HIP
call (no GPU needed); plus the manifest-op argument packer."""
import ctypes
import os
import re
import struct

import pytest

import k3h

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "k3h.h")


def _declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"K3H_API\s+[\w\s\*]+?\b(k3h_\w+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    names = _declared()
    assert len(names) >= 15
    L = k3h.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the Python mirror binds all of them
    assert set(names) - set(k3h._SIGS) <= {"k3h_error_string"}


def test_code_objects_built_for_every_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("k3build", os.path.join(REPO, "kern-k3_amd", "build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    for key in b.MODULES:
        assert os.path.exists(os.path.join(k3h.BUILD, key + ".hsaco")), key


def test_error_strings():
    assert k3h.error_string(k3h.K3H_OK) == "ok"
    assert "invalid" in k3h.error_string(k3h.K3H_EINVAL)
    assert "missing" in k3h.error_string(k3h.K3H_ENOMODULE)


@pytest.fixture
def hctx():
    L = k3h.lib()
    h = ctypes.c_void_p()
    assert L.k3h_ctx_create(k3h.BUILD.encode(), ctypes.byref(h)) == 0
    yield L, h
    assert L.k3h_ctx_destroy(h) == 0


A = 0x10000  # a 16-byte-aligned stand-in address: never dereferenced by these calls


def test_host_validation_rejects_before_launch(hctx):
    L, h = hctx
    E = k3h.K3H_EINVAL
    # null context, negative sizes, misaligned pointers, out-of-range nb / eps
    assert L.k3h_residual_rms_mxfp8(None, None, A, A, A, A, A, A, None, 1e-6, 1) == E
    assert L.k3h_residual_rms_mxfp8(h, None, A, A, A, A, A, A, None, 1e-6, -1) == E
    assert L.k3h_residual_rms_mxfp8(h, None, A + 2, A, A, A, A, A, None, 1e-6, 1) == E
    assert L.k3h_residual_rms_mxfp8(h, None, A, A, A, A, A + 4, A, None, 1e-6, 1) == E
    assert L.k3h_residual_rms_mxfp8(h, None, A, A, A, A, A, A, A + 8, 1e-6, 1) == E
    assert L.k3h_residual_rms_mxfp8(h, None, A, A, A, A, A, A, None, 0.0, 1) == E
    assert L.k3h_land_add_attnres_rms(h, None, 1, A, A, A, A, A, A, A, 9, 0, 1, 1e-5) == E
    assert L.k3h_land_add_attnres_rms(h, None, 1, A, A, A, A, A, A, A, 0, 0, 1, 3e-5) == E
    assert L.k3h_land_add_attnres_rms(h, None, 1, A, A, None, None, A, A, A, 2, 0, 1, 1e-5) == E
    assert L.k3h_land_add_attnres_rms_nb(h, None, A, A, A, A, A, A, A, 0, 0, 1) == E
    assert L.k3h_moe_quant(h, None, A, A, A, 3, 7) == E  # 21 elements: not whole blocks
    assert L.k3h_attnres_rms(h, None, A + 1, A, A, A, A, 0, 0, 1, 1e-5) == E
    assert L.k3h_land_add2(h, None, A, None, A, A, 1, 1) == E


def test_empty_work_returns_ok_without_launch(hctx):
    L, h = hctx
    assert L.k3h_residual_rms_mxfp8(h, None, A, A, A, A, A, A, None, 1e-6, 0) == 0
    assert L.k3h_moe_quant(h, None, A, A, A, 0, 7168) == 0
    assert L.k3h_land_add_attnres_rms(h, None, 1, A, A, None, None, A, A, A, 0, 0, 0, 1e-5) == 0
    assert L.k3h_land_add2(h, None, A, None, A, A, 0, 0) == 0


def test_launch_rejects_bad_block():
    L = k3h.lib()
    grid = (ctypes.c_uint32 * 3)(1, 1, 1)
    blk = (ctypes.c_uint32 * 3)(2048, 1, 1)
    assert L.k3h_launch(ctypes.c_void_p(A), grid, blk, 0, None, None, 0) == k3h.K3H_EINVAL
    assert L.k3h_launch(None, grid, blk, 0, None, None, 0) == k3h.K3H_EINVAL


def test_pack_args_natural_alignment():
    kinds = ["in buffer<bf16>", "i32", "in buffer<f32>", "i32", "i64", "f32", "out buffer<u8>"]
    b = k3h.pack_args(kinds, [0x1000, 7, 0x2000, 9, -5, 1.5, None])
    assert struct.unpack_from("<Q", b, 0)[0] == 0x1000
    assert struct.unpack_from("<i", b, 8)[0] == 7
    assert struct.unpack_from("<Q", b, 16)[0] == 0x2000   # padded to 8
    assert struct.unpack_from("<i", b, 24)[0] == 9
    assert struct.unpack_from("<q", b, 32)[0] == -5      # padded to 8
    assert struct.unpack_from("<f", b, 40)[0] == 1.5
    assert struct.unpack_from("<Q", b, 48)[0] == 0       # None -> null
    assert len(b) == 56


def test_grid_expressions():
    env = {"tokens": 16384}
    assert k3h._eval_expr({"ceil_div": ["tokens", 4]}, env) == 4096
    assert k3h._eval_expr({"ceil_div": [{"mul": [{"ceil_div": ["tokens", 4]}, 112]}, 256]}, env) == 1792
    assert k3h._eval_expr({"ceil_div": [{"add": ["tokens", 3]}, 2]}, {"tokens": 5}) == 4
    with pytest.raises(ValueError):
        k3h._eval_expr({"pow": [2, 3]}, env)
