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
    assert "at once" in k3h.error_string(k3h.K3H_ERESIDENT)


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
    # barrier: slot 0 is the epoch, 1 <= nranks <= 8, units >= 1, 8-byte counters
    assert L.k3h_rs_arrive(h, None, A, A, 896, 0, 4, None) == E
    assert L.k3h_rs_arrive(h, None, A, A, 896, 1, 9, None) == E
    assert L.k3h_rs_arrive(h, None, A, A, 0, 1, 4, None) == E
    assert L.k3h_rs_arrive(h, None, A + 4, A, 896, 1, 4, None) == E
    assert L.k3h_rs_arrive(h, None, A, None, 896, 1, 4, None) == E
    assert L.k3h_rs_arrive(h, None, A, A, 896, 1, 4, A + 2) == E
    assert L.k3h_epoch_bump(h, None, A, 0) == E
    assert L.k3h_flags_init(h, None, A + 4, 372) == E


def test_empty_work_returns_ok_without_launch(hctx):
    L, h = hctx
    assert L.k3h_residual_rms_mxfp8(h, None, A, A, A, A, A, A, None, 1e-6, 0) == 0
    assert L.k3h_moe_quant(h, None, A, A, A, 0, 7168) == 0
    assert L.k3h_land_add_attnres_rms(h, None, 1, A, A, None, None, A, A, A, 0, 0, 0, 1e-5) == 0
    assert L.k3h_land_add2(h, None, A, None, A, A, 0, 0) == 0
    assert L.k3h_flags_init(h, None, A, 0) == 0


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


def test_gemm_rejects_32bit_row_offset_overflow(hctx):
    """A read in place: max_tiles * 128 * K above 2^32 - 1 is rejected before any launch."""
    L, h = hctx
    # 4682 tiles * 128 rows * 7168 bytes = 4,295,819,264 > 4,294,967,295
    assert L.k3h_moe_gemm_mx(h, None, 0, A, A, None, A, A, A, A, 4682, 1, 256, 7168, A,
                             None, None, None) == k3h.K3H_EINVAL


def test_out_gate_eps_selects_module(hctx):
    L, h = hctx
    assert L.k3h_kda_out_gate(h, None, A, A, A, A, A, 1, 1e-4) == k3h.K3H_EINVAL
    assert L.k3h_kda_out_gate(h, None, A, A, A, A, A, 0, 1e-6) == 0   # span 0: no launch
    assert L.k3h_kda_out_gate(h, None, A, A, A, A, A, 0, 1e-5) == 0


def test_wrappers_reject_undersized_buffers(monkeypatch):
    """The Python mirror checks each buffer against the size the kernel will touch.
    Without a GPU the tensor check is narrowed to its size part (the device and
    alignment parts are what host tensors would fail first); every case here is
    rejected before any call into the library."""
    import torch

    def size_only(t, name, dtypes, numel=None, align=16):
        if numel is not None and t.numel() < numel:
            raise ValueError(f"{name}: needs at least {numel} elements, has {t.numel()}")
    monkeypatch.setattr(k3h, "_dev", size_only)
    ctx = k3h.Ctx()
    i32 = lambda n: torch.zeros(n, dtype=torch.int32)
    u8 = lambda n: torch.zeros(n, dtype=torch.uint8)
    blocks, E, T, topk = 4, 56, 1024, 8
    tiles = (T * topk + 127 * E) // 128
    good = dict(blockcount=i32(blocks * E), blockoff=i32(blocks * E), cta_batch=i32(tiles),
                cta_limit=i32(tiles), num_non_exiting=i32(1), total_padded=i32(1),
                route_map=i32(tiles * 128))
    for name, small in (("blockcount", i32(1)), ("blockoff", i32(blocks * E - 1)),
                        ("cta_batch", i32(tiles - 1)), ("route_map", i32(tiles * 128 - 1))):
        args = dict(good, **{name: small})
        with pytest.raises(ValueError, match=f"{name}: needs at least"):
            ctx.moe_route_tables(args["blockcount"], blocks, E, 128, args["blockoff"],
                                 args["cta_batch"], args["cta_limit"], args["num_non_exiting"],
                                 args["total_padded"], args["route_map"], T=T, topk=topk)
    # GEMM reading A in place needs every padded row of max_tiles tiles
    K, N, mt = 256, 256, 3
    with pytest.raises(ValueError, match="a: needs at least"):
        ctx.moe_gemm_mx(ctx.GEMM_F32, u8(mt * 128 * K - 16), u8(mt * 128 * K // 32), None,
                        u8(E * N * K // 2), u8(E * N * K // 32), i32(1), i32(mt), mt, E, N, K,
                        torch.zeros(mt * 128 * N))
    with pytest.raises(ValueError, match="a_sf: needs at least"):
        ctx.moe_gemm_mx(ctx.GEMM_F32, u8(mt * 128 * K), u8(mt * 128 * K // 32 - 4), None,
                        u8(E * N * K // 2), u8(E * N * K // 32), i32(1), i32(mt), mt, E, N, K,
                        torch.zeros(mt * 128 * N))
    with pytest.raises(ValueError, match="below 2"):
        ctx.moe_gemm_mx(ctx.GEMM_F32, u8(16), u8(16), None, u8(16), u8(16), i32(1), i32(1),
                        4682, E, 256, 7168, torch.zeros(1))
    # permute with the token count given: q / sf must hold that many rows
    with pytest.raises(ValueError, match="q: needs at least"):
        ctx.moe_permute_mx(u8(10 * 1024 - 1), u8(10 * 32), i32(8), i32(1), 1024, u8(8 * 1024),
                           u8(8 * 32), tokens=10)
    ctx.close()


def test_missing_code_objects_fail_loudly(tmp_path):
    """A context over a directory without the gfx950 code objects: the typed
    calls and the entry lookup return K3H_ENOMODULE (and the Python mirror
    raises); nothing falls back to another implementation."""
    L = k3h.lib()
    h = ctypes.c_void_p()
    assert L.k3h_ctx_create(str(tmp_path).encode(), ctypes.byref(h)) == 0
    try:
        assert L.k3h_residual_rms_mxfp8(h, None, A, A, A, A, A, A, None, 1e-6, 1) == k3h.K3H_ENOMODULE
        assert L.k3h_moe_quant(h, None, A, A, A, 1, 7168) == k3h.K3H_ENOMODULE
        fn = ctypes.c_void_p()
        assert L.k3h_ctx_function(h, b"k3h_fused", b"k3h_residual_rms_mxfp8",
                                  ctypes.byref(fn)) == k3h.K3H_ENOMODULE
    finally:
        assert L.k3h_ctx_destroy(h) == 0
    with pytest.raises(k3h.K3HError):
        k3h.Ctx(str(tmp_path)).function("k3h_fused", "k3h_residual_rms_mxfp8")
