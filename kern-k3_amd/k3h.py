"""Python host side of the k3h C-ABI (``include/k3h.h``).

The operators mirror the reference's manifest op surface: each method has the
manifest op's parameters in the manifest's order (``ops.<op>.params`` of
k3-tp4-prefill-16k.json, e.g. ``moe_quant`` at line 404926) and launches the
gfx950 code object with the manifest's grid.  Tensors are torch device tensors
(torch provides the memory and the stream; the arithmetic is the HIP kernels').
Arguments are checked here and again in the C library; a failed check raises
``ValueError``, a failed launch ``K3HError``.  There is no CPU path: a missing
library or code object raises.

``ManifestOp`` runs a manifest op description verbatim: it evaluates the grid
expressions, packs the arguments by the launch's parameter kinds and calls
``k3h_launch`` -- the path the kern runtime takes for a cubin, here for a
gfx950 code object.
"""
from __future__ import annotations

import ctypes
import os
import struct
from typing import Any, Sequence

import torch  # loaded first: libk3h then binds to the HIP runtime torch already mapped

PKG = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(PKG, "build")
LIB_PATH = os.path.join(BUILD, "libk3h.so")

K3H_OK, K3H_EINVAL, K3H_ENOMODULE, K3H_ENOENTRY, K3H_ENOMEM = 0, -1, -2, -3, -4
K3H_ERESIDENT = -5

MOE_V4 = "k3_moe_prefill_v4+EP_RANKS=4+EP_STRIDED=1+TILE_SHIFT=7+SCATTER_WARPS=16"
MOE_V3 = "k3_moe_prefill_v3+EP_STRIDED=1"

H = 7168
NOALLOC_MAX_NB = 4096  # K3H_NOALLOC_MAX_NB of include/k3h.h


class K3HError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"{what}: {error_string(code)} ({code})")


_lib: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes (restype is int for all of them)
_SIGS: dict[str, list] = {
    "k3h_module_load": [_P, ctypes.c_size_t, ctypes.POINTER(_P)],
    "k3h_module_load_file": [ctypes.c_char_p, ctypes.POINTER(_P)],
    "k3h_function": [_P, ctypes.c_char_p, ctypes.POINTER(_P)],
    "k3h_launch": [_P, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32),
                   ctypes.c_uint32, _P, _P, ctypes.c_size_t],
    "k3h_module_unload": [_P],
    "k3h_runtime_version": [ctypes.POINTER(_I)],
    "k3h_ctx_create": [ctypes.c_char_p, ctypes.POINTER(_P)],
    "k3h_synth_normal": [ctypes.c_char_p, ctypes.c_size_t, _F, _F, _F, _F, _I, _P],
    "k3h_ctx_destroy": [_P],
    "k3h_ctx_function": [_P, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_P)],
    "k3h_land_add_attnres_rms": [_P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F],
    "k3h_land_add_attnres_rms_nb": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I],
    "k3h_attnres_rms": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F],
    "k3h_land_add2": [_P, _P, _P, _P, _P, _P, _I, _I],
    "k3h_moe_quant": [_P, _P, _P, _P, _P, _I, _I],
    "k3h_residual_rms_mxfp8": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I],
    "k3h_stream_copy": [_P, _P, _P, _P, ctypes.c_int64],
    "k3h_quant_fp8_amax": [_P, _P, _I, _P, _I, _P, _I],
    "k3h_quant_fp8_apply": [_P, _P, _I, _P, _P, _I, _P, _I, _P],
    "k3h_quant_fp8_tensor": [_P, _P, _I, _P, _P, _P, _P, _I, _I],
    "k3h_quant_fp8_tensor_noalloc": [_P, _P, _I, _P, _P, _P, _I, _I],
    "k3h_router_topk": [_P, _P, _I, _P, _P, _P, _P, _P, _I],
    "k3h_argmax_f32": [_P, _P, _P, _P, _P, _P, _I, _I, _I],
    "k3h_moe_route_count": [_P, _P, _I, _P, _I, _I, _I, _P],
    "k3h_moe_route_tables": [_P, _P, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P],
    "k3h_moe_route_scatter": [_P, _P, _I, _P, _P, _I, _I, _I, _P, _P],
    "k3h_moe_route": [_P, _P, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "k3h_moe_finalize": [_P, _P, _I, _P, _P, _P, _P, _I, _I],
    "k3h_moe_permute_mx": [_P, _P, _P, _P, _P, _P, _I, _I, _P, _P],
    "k3h_moe_w_shuffle": [_P, _P, _P, _P, _I, _I, _I, _I],
    "k3h_moe_sf_shuffle": [_P, _P, _P, _P, _I, _I, _I, _I],
    "k3h_span_gather": [_P, _P, _P, _P, _P, _P, ctypes.c_int64, _P, _P, _P, _P, _P, _P, _P, _I],
    "k3h_kda_out_gate": [_P, _P, _P, _P, _P, _P, _P, _I, _F],
    "k3h_mla_prep": [_P, _P, _I, _P, _P, _P, _P, _P, ctypes.c_int64, ctypes.c_int64, _P, _P, _I],
    "k3h_mla_rope_pack": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _F, _I, _I],
    "k3h_attnres_rms_push": [_P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I],
    "k3h_attnres_rms_push_stats": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P],
    "k3h_attnres_rms_push_add2": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P,
                                  _P, _P, _I],
    "k3h_land_add_attnres_rms_nb_stats": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _I],
    "k3h_land_add2_bf16": [_P, _P, _P, _P, _P, _P, _I, _I],
    "k3h_flags_init": [_P, _P, _P, _I],
    "k3h_epoch_bump": [_P, _P, _P, _I],
    "k3h_rs_arrive": [_P, _P, _P, _P, _I, _I, _I, _P],
    "k3h_rms": [_P, _P, _P, _P, _P, _I, _I],
    "k3h_land": [_P, _P, _P, _P, _I, _I, _I, _I],
    "k3h_land_situ": [_P, _P, _I, _P, _P, _I, _I],
    "k3h_situ_rms": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I],
    "k3h_moe_w_tile": [_P, _P, _P, _P, _I, _I, _I, _I],
    "k3h_moe_sf_tile": [_P, _P, _P, _P, _I, _I, _I, _I],
    "k3h_moe_gemm_mx": [_P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P],
    "k3h_moe_fc1": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I],
    "k3h_moe_fc2": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I],
}


def lib() -> ctypes.CDLL:
    """Load libk3h.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `python kern-k3_amd/build.py`")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _I
        L.k3h_error_string.argtypes = [_I]
        L.k3h_error_string.restype = ctypes.c_char_p
        _lib = L
    return _lib


def synth_normal(name: str, shape, mean: float = 0.0, std: float = 1.0, outlier_p: float = 0.0,
                 outlier_x: float = 50.0, dtype=torch.bfloat16) -> torch.Tensor:
    """Seeded synthetic input on the host (k3h_synth_normal): the tensor's own
    xoshiro256** stream, seed 24301 ^ fnv1a64(name), Box-Muller normals; bf16 or f32."""
    n = 1
    for d in shape:
        n *= int(d)
    if dtype == torch.bfloat16:
        out = torch.empty(n, dtype=torch.int16)
    elif dtype == torch.float32:
        out = torch.empty(n, dtype=torch.float32)
    else:
        raise ValueError("synth_normal: bfloat16 or float32")
    _check(lib().k3h_synth_normal(name.encode(), n, mean, std, outlier_p, outlier_x,
                                  int(dtype == torch.bfloat16), out.data_ptr() if n else None),
           "synth_normal")
    if dtype == torch.bfloat16:
        out = out.view(torch.bfloat16)
    return out.view(*shape)


def error_string(code: int) -> str:
    return lib().k3h_error_string(code).decode()


def _check(rc: int, what: str) -> None:
    if rc != K3H_OK:
        if rc == K3H_EINVAL:
            raise ValueError(f"{what}: invalid argument (rejected by libk3h)")
        raise K3HError(rc, what)


# ---------------------------------------------------------------- tensor checks
def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _dev(t: torch.Tensor, name: str, dtypes: Sequence[torch.dtype], numel: int | None = None,
         align: int = 16) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name}: expected a torch tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be a GPU tensor (got {t.device})")
    if t.dtype not in dtypes:
        raise ValueError(f"{name}: dtype {t.dtype} not in {list(dtypes)}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{name}: needs at least {numel} elements, has {t.numel()}")
    if t.data_ptr() % align:
        raise ValueError(f"{name}: must be {align}-byte aligned")


BF16 = (torch.bfloat16,)
U8 = (torch.uint8, torch.float8_e4m3fn)
F32 = (torch.float32,)
I32 = (torch.int32,)
I64 = (torch.int64,)


def _stream(stream: Any) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class Ctx:
    """A k3h context: code objects loaded on first use from ``codeobj_dir``."""

    def __init__(self, codeobj_dir: str = BUILD):
        self.L = lib()
        h = _P()
        _check(self.L.k3h_ctx_create(codeobj_dir.encode(), ctypes.byref(h)), "k3h_ctx_create")
        self.h = h
        self.dir = codeobj_dir

    def close(self) -> None:
        if self.h:
            self.L.k3h_ctx_destroy(self.h)
            self.h = None

    def function(self, module_key: str, entry: str) -> int:
        f = _P()
        _check(self.L.k3h_ctx_function(self.h, module_key.encode(), entry.encode(), ctypes.byref(f)),
               f"{module_key}:{entry}")
        return f.value

    # ------------------------------------------------------------ K1 family
    def land_add_attnres_rms(self, partial, prefix, blocks, sw, gamma, prefix2, normed, nb: int,
                             snapshot: int, B: int, eps: float = 1e-5, stream=None) -> None:
        """kern_k3_land_add_attnres_rms (k3_residual_v2.cu:295); partial bf16 or f32."""
        n = B * H
        _dev(partial, "partial", BF16 + F32, n)
        if not snapshot:
            _dev(prefix, "prefix", BF16, n)
        if nb > 0:
            _dev(blocks, "blocks", BF16, B * 8 * H)
            _dev(sw, "sw", F32, H)
        _dev(gamma, "gamma", BF16, H)
        _dev(prefix2, "prefix2", BF16, n)
        _dev(normed, "normed", BF16, n)
        _check(self.L.k3h_land_add_attnres_rms(
            self.h, _stream(stream), int(partial.dtype == torch.bfloat16), _ptr(partial),
            _ptr(prefix), _ptr(blocks), _ptr(sw), _ptr(gamma), _ptr(prefix2), _ptr(normed), nb,
            snapshot, B, eps), "land_add_attnres_rms")

    def land_add_attnres_rms_nb(self, partial, prefix, blocks, sw, gamma, prefix2, normed,
                                nb: int, snapshot: int, B: int, stream=None) -> None:
        """kern_k3_land_add_attnres_rms_nb{nb} (k3_residual_nb.cu:350-811), LAND_BF16."""
        n = B * H
        _dev(partial, "partial", BF16, n)
        if not snapshot:
            _dev(prefix, "prefix", BF16, n)
        _dev(blocks, "blocks", BF16, B * 8 * H)
        _dev(sw, "sw", F32, H)
        _dev(gamma, "gamma", BF16, H)
        _dev(prefix2, "prefix2", BF16, n)
        _dev(normed, "normed", BF16, n)
        _check(self.L.k3h_land_add_attnres_rms_nb(
            self.h, _stream(stream), _ptr(partial), _ptr(prefix), _ptr(blocks), _ptr(sw),
            _ptr(gamma), _ptr(prefix2), _ptr(normed), nb, snapshot, B), "land_add_attnres_rms_nb")

    def attnres_rms(self, prefix, blocks, sw, gamma, normed, nb: int, snapshot: int, B: int,
                    eps: float = 1e-5, stream=None) -> None:
        """kern_k3_attnres_rms (k3_residual_v2.cu:260)."""
        _dev(prefix, "prefix", BF16, B * H)
        if nb > 0 or snapshot:
            _dev(blocks, "blocks", BF16, B * 8 * H)
        if nb > 0:
            _dev(sw, "sw", F32, H)
        _dev(gamma, "gamma", BF16, H)
        _dev(normed, "normed", BF16, B * H)
        _check(self.L.k3h_attnres_rms(self.h, _stream(stream), _ptr(prefix), _ptr(blocks),
                                      _ptr(sw), _ptr(gamma), _ptr(normed), nb, snapshot, B, eps),
               "attnres_rms")

    def land_add2(self, p1, p2, prefix2, hidden, two: int, B: int, stream=None) -> None:
        """kern_k3_land_add2 (k3_residual_v2.cu:349)."""
        _dev(p1, "p1", F32, B * H)
        if two:
            _dev(p2, "p2", F32, B * H)
        _dev(prefix2, "prefix2", BF16, B * H)
        _dev(hidden, "hidden", BF16, B * H)
        _check(self.L.k3h_land_add2(self.h, _stream(stream), _ptr(p1), _ptr(p2), _ptr(prefix2),
                                    _ptr(hidden), two, B), "land_add2")

    # ------------------------------------------------------------ MXFP8
    # ------------------------------------------------------------ push family
    def _push_checks(self, blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks):
        if nb > 0 or (snapshot and nb < 8):
            _dev(blocks, "blocks", BF16, B * 8 * H)
        if nb > 0:
            _dev(sw, "sw", F32, H)
        _dev(gamma, "gamma", BF16, H)
        _dev(normed_all, "normed_all", BF16, (rank + 1) * B * H)
        if nranks > 1:
            _dev(dst_peer, "dst_peer", I64, nranks, align=8)

    def attnres_rms_push(self, prefix, blocks, sw, gamma, normed_all, dst_peer, nb: int,
                         snapshot: int, B: int, rank: int, nranks: int, version: int = 3,
                         stream=None) -> None:
        """kern_k3_attnres_rms_push of k3_residual_push (version 1) / _v3 (version 3)
        (k3_residual_push_v3.cu:324; op attnres_rms_push_first_v3).  dst_peer: int64
        tensor of every rank's normed_all device address."""
        _dev(prefix, "prefix", BF16, B * H)
        self._push_checks(blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks)
        _check(self.L.k3h_attnres_rms_push(
            self.h, _stream(stream), version, _ptr(prefix), _ptr(blocks), _ptr(sw), _ptr(gamma),
            _ptr(normed_all), _ptr(dst_peer), nb, snapshot, B, rank, nranks), "attnres_rms_push")

    def attnres_rms_push_stats(self, prefix, blocks, sw, gamma, normed_all, dst_peer, nb: int,
                               snapshot: int, B: int, rank: int, nranks: int, sw_mlp, stats,
                               stream=None) -> None:
        """kern_k3_attnres_rms_push of k3_residual_push_stats (k3_residual_push_stats.cu:354)."""
        _dev(prefix, "prefix", BF16, B * H)
        self._push_checks(blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks)
        if nb > 0:
            _dev(sw_mlp, "sw_mlp", F32, H)
            _dev(stats, "stats", F32, B * 16, align=8)
        _check(self.L.k3h_attnres_rms_push_stats(
            self.h, _stream(stream), _ptr(prefix), _ptr(blocks), _ptr(sw), _ptr(gamma),
            _ptr(normed_all), _ptr(dst_peer), nb, snapshot, B, rank, nranks, _ptr(sw_mlp),
            _ptr(stats)), "attnres_rms_push_stats")

    def attnres_rms_push_add2(self, blocks, sw, gamma, normed_all, dst_peer, nb: int,
                              snapshot: int, B: int, rank: int, nranks: int, sw_mlp, stats, p1,
                              p2, prefix2, hidden, two: int, stream=None) -> None:
        """kern_k3_attnres_rms_push of k3_residual_push_add2 (k3_residual_push_add2.cu:362;
        op attnres_rms_push_add2)."""
        self._push_checks(blocks, sw, gamma, normed_all, dst_peer, nb, snapshot, B, rank, nranks)
        if nb > 0:
            _dev(sw_mlp, "sw_mlp", F32, H)
            _dev(stats, "stats", F32, B * 16, align=8)
        _dev(p1, "p1", BF16, B * H)
        if two:
            _dev(p2, "p2", BF16, B * H)
        _dev(prefix2, "prefix2", BF16, B * H)
        _dev(hidden, "hidden", BF16, B * H)
        _check(self.L.k3h_attnres_rms_push_add2(
            self.h, _stream(stream), _ptr(blocks), _ptr(sw), _ptr(gamma), _ptr(normed_all),
            _ptr(dst_peer), nb, snapshot, B, rank, nranks, _ptr(sw_mlp), _ptr(stats), _ptr(p1),
            _ptr(p2), _ptr(prefix2), _ptr(hidden), two), "attnres_rms_push_add2")

    def land_add_attnres_rms_nb_stats(self, partial, prefix, blocks, sw, gamma, prefix2, normed,
                                      nb: int, snapshot: int, B: int, stats, nb_stats: int,
                                      stream=None) -> None:
        """kern_k3_land_add_attnres_rms_nb{nb} of k3_residual_nb_stats (LAND_BF16)
        (k3_residual_nb_stats.cu:366-811; ops land_add_attnres_rms_bf16_v2_nb4..8)."""
        n = B * H
        _dev(partial, "partial", BF16, n)
        if not snapshot:
            _dev(prefix, "prefix", BF16, n)
        _dev(blocks, "blocks", BF16, B * 8 * H)
        _dev(sw, "sw", F32, H)
        _dev(gamma, "gamma", BF16, H)
        _dev(prefix2, "prefix2", BF16, n)
        _dev(normed, "normed", BF16, n)
        if nb_stats > 0:
            _dev(stats, "stats", F32, B * 16, align=8)
        _check(self.L.k3h_land_add_attnres_rms_nb_stats(
            self.h, _stream(stream), _ptr(partial), _ptr(prefix), _ptr(blocks), _ptr(sw),
            _ptr(gamma), _ptr(prefix2), _ptr(normed), nb, snapshot, B, _ptr(stats), nb_stats),
            "land_add_attnres_rms_nb_stats")

    def land_add2_bf16(self, p1, p2, prefix2, hidden, two: int, B: int, stream=None) -> None:
        """kern_k3_land_add2_bf16 (k3_land_bf16.cu:96)."""
        _dev(p1, "p1", BF16, B * H)
        if two:
            _dev(p2, "p2", BF16, B * H)
        _dev(prefix2, "prefix2", BF16, B * H)
        _dev(hidden, "hidden", BF16, B * H)
        _check(self.L.k3h_land_add2_bf16(self.h, _stream(stream), _ptr(p1), _ptr(p2),
                                         _ptr(prefix2), _ptr(hidden), two, B), "land_add2_bf16")

    # ------------------------------------------------------------ epoch / arrival barrier
    def flags_init(self, flags, n: int, stream=None) -> None:
        """kern_k3_flags_init (k3_collectives.cu:64): flags[0 .. n) = 0."""
        _dev(flags, "flags", I64, n, align=8)
        _check(self.L.k3h_flags_init(self.h, _stream(stream), _ptr(flags), n), "flags_init")

    def epoch_bump(self, flags, units: int, stream=None) -> None:
        """kern_k3_epoch_bump (k3_collectives.cu:74): flags[0] += units."""
        _dev(flags, "flags", I64, 1, align=8)
        _check(self.L.k3h_epoch_bump(self.h, _stream(stream), _ptr(flags), units), "epoch_bump")

    def rs_arrive(self, flags, flags_peer, units: int, slot: int, nranks: int, missing=None,
                  stream=None) -> None:
        """kern_k3_rs_arrive1 (k3_rs_arrive_v2.cu:41): flags[slot] += units, then wait until
        every rank's flags[slot] (flags_peer: int64 tensor of device addresses) reaches
        flags[0].  With ``missing`` (int32 [1]) the mask of ranks that never arrived is
        written there."""
        _dev(flags, "flags", I64, slot + 1, align=8)
        _dev(flags_peer, "flags_peer", I64, nranks, align=8)
        if missing is not None:
            _dev(missing, "missing", I32, 1, align=4)
        _check(self.L.k3h_rs_arrive(self.h, _stream(stream), _ptr(flags), _ptr(flags_peer), units,
                                    slot, nranks, _ptr(missing)), "rs_arrive")

    # ------------------------------------------------------------ landing kernels
    def rms(self, x, gamma, o, h: int, B: int, stream=None) -> None:
        """kern_k3_rms (k3_land.cu:104; l0 op rms)."""
        al = 16 if h % 8 == 0 else 2
        _dev(x, "x", BF16, B * h, align=al)
        _dev(gamma, "gamma", BF16, h, align=al)
        _dev(o, "o", BF16, B * h, align=al)
        _check(self.L.k3h_rms(self.h, _stream(stream), _ptr(x), _ptr(gamma), _ptr(o), h, B), "rms")

    def land(self, p, o, n: int, off: int, ldc: int, B: int, stream=None) -> None:
        """kern_k3_land (k3_land.cu:168; l0 op land_n3584)."""
        vec = (n | off | ldc) % 4 == 0
        _dev(p, "p", F32, B * ldc, align=16 if vec else 4)
        _dev(o, "o", BF16, B * n, align=8 if vec else 2)
        _check(self.L.k3h_land(self.h, _stream(stream), _ptr(p), _ptr(o), n, off, ldc, B), "land")

    def land_situ(self, p, act, n: int, B: int, variant: str | None = None, stream=None) -> None:
        """SiTU landing: p f32 -> kern_k3_land_situ (op land_situ_n33792); p bf16 ->
        kern_k3_land_situ_bf16 (variant "land_bf16", default) or kern_k3_situ_bf16
        (variant "situ_bf16", l0 op land_situ_n33792)."""
        vec = n % 8 == 0
        if p.dtype == torch.float32:
            mode = 0
        else:
            mode = 2 if variant == "situ_bf16" else 1
        _dev(p, "p", F32 if mode == 0 else BF16, B * 2 * n, align=16 if vec else 2)
        _dev(act, "act", BF16, B * n, align=16 if vec else 2)
        _check(self.L.k3h_land_situ(self.h, _stream(stream), mode, _ptr(p), _ptr(act), n, B),
               "land_situ")

    def situ_rms(self, sp, act, lat, gam, ln, n: int, B: int, h: int, L: int, tokens: int,
                 stream=None) -> None:
        """kern_k3_situ_rms_bf16 (k3_land_fused.cu:151; op land_situ_rms)."""
        a_s, a_l = (16 if n % 8 == 0 else 2), (16 if h % 8 == 0 else 2)
        _dev(sp, "sp", BF16, B * 2 * n, align=a_s)
        _dev(act, "act", BF16, B * n, align=a_s)
        _dev(lat, "lat", BF16, L * h, align=a_l)
        _dev(gam, "gam", BF16, h, align=a_l)
        _dev(ln, "ln", BF16, L * h, align=a_l)
        _check(self.L.k3h_situ_rms(self.h, _stream(stream), _ptr(sp), _ptr(act), _ptr(lat),
                                   _ptr(gam), _ptr(ln), n, B, h, L, tokens), "situ_rms")

    def moe_quant(self, x, q, sf, rows: int, cols: int, stream=None) -> None:
        """kern_k3_moe_quant (k3_moe_prefill_v4.cu:111): manifest op moe_quant."""
        n = rows * cols
        if n % 32:
            raise ValueError("moe_quant: rows * cols must be a multiple of 32")
        _dev(x, "x", BF16, n)
        _dev(q, "q", U8, n, align=8)
        _dev(sf, "sf", U8, n // 32, align=1)
        _check(self.L.k3h_moe_quant(self.h, _stream(stream), _ptr(x), _ptr(q), _ptr(sf), rows,
                                    cols), "moe_quant")

    def residual_rms_mxfp8(self, x, residual, gamma, residual_out, q, sf, normed=None,
                           eps: float = 1e-6, B: int | None = None, stream=None) -> None:
        """Fused residual add + RMSNorm + MXFP8 (K1b nb=0 composed with moe_quant)."""
        B = x.shape[0] if B is None else B
        n = B * H
        _dev(x, "x", BF16, n)
        _dev(residual, "residual", BF16, n)
        _dev(gamma, "gamma", BF16, H)
        _dev(residual_out, "residual_out", BF16, n)
        _dev(q, "q", U8, n, align=8)
        _dev(sf, "sf", U8, n // 32, align=4)
        if normed is not None:
            _dev(normed, "normed", BF16, n)
        _check(self.L.k3h_residual_rms_mxfp8(self.h, _stream(stream), _ptr(x), _ptr(residual),
                                             _ptr(gamma), _ptr(residual_out), _ptr(q), _ptr(sf),
                                             _ptr(normed), eps, B), "residual_rms_mxfp8")


    # ------------------------------------------------------------ per-tensor fp8
    def quant_fp8_tensor(self, x, y, scale_out, partials, n: int, v2: bool = True,
                         stream=None) -> None:
        """Manifest op quant_fp8_tensor (params x, y, scale_out, partials, n): amax + apply."""
        nb = partials.numel()
        _dev(x, "x", BF16, n)
        _dev(y, "y", U8, n, align=8)
        _dev(scale_out, "scale_out", F32, 1, align=4)
        _dev(partials, "partials", F32, 1, align=4)
        _check(self.L.k3h_quant_fp8_tensor(self.h, _stream(stream), int(v2), _ptr(x), _ptr(y),
                                           _ptr(scale_out), _ptr(partials), n, nb),
               "quant_fp8_tensor")

    def quant_fp8_tensor_noalloc(self, x, y, scale_out, n: int, nb: int = 2048, v2: bool = True,
                                 stream=None) -> None:
        """quant_fp8_tensor with the amax partials in the library's per-GPU device array
        (no caller buffer, no allocation); nb <= NOALLOC_MAX_NB.  Calls that overlap on
        one GPU share that array and race."""
        if not 1 <= nb <= NOALLOC_MAX_NB:
            raise ValueError(f"quant_fp8_tensor_noalloc: nb must be in [1, {NOALLOC_MAX_NB}]")
        _dev(x, "x", BF16, n)
        _dev(y, "y", U8, n, align=8)
        _dev(scale_out, "scale_out", F32, 1, align=4)
        _check(self.L.k3h_quant_fp8_tensor_noalloc(self.h, _stream(stream), int(v2), _ptr(x),
                                                   _ptr(y), _ptr(scale_out), n, nb),
               "quant_fp8_tensor_noalloc")

    def quant_fp8_amax(self, x, n: int, partials, v2: bool = True, stream=None) -> None:
        _dev(x, "x", BF16, n)
        _dev(partials, "partials", F32, 1, align=4)
        _check(self.L.k3h_quant_fp8_amax(self.h, _stream(stream), int(v2), _ptr(x), n,
                                         _ptr(partials), partials.numel()), "quant_fp8_amax")

    # ------------------------------------------------------------ MoE router
    def router_topk(self, S, bias, rs, idx, wts, B: int, topk: int = 16, stream=None) -> None:
        """Manifest op router_topk (S, bias, rs, idx, wts, B) -- kern_k3_router_topk."""
        _dev(S, "S", F32, B * 224, align=4)
        _dev(bias, "bias", F32, 224, align=4)
        _dev(rs, "rs", BF16, 1, align=2)
        _dev(idx, "idx", I32, B * topk, align=4)
        _dev(wts, "wts", F32, B * topk, align=4)
        _check(self.L.k3h_router_topk(self.h, _stream(stream), topk, _ptr(S), _ptr(bias), _ptr(rs),
                                      _ptr(idx), _ptr(wts), B), "router_topk")

    def argmax_f32(self, logits, pmax, pidx, out, B: int, n: int, parts: int, stream=None) -> None:
        _dev(logits, "logits", F32, B * n, align=4)
        _dev(pmax, "pmax", F32, B * parts, align=4)
        _dev(pidx, "pidx", I32, B * parts, align=4)
        _dev(out, "out", I64, B, align=8)
        _check(self.L.k3h_argmax_f32(self.h, _stream(stream), _ptr(logits), _ptr(pmax), _ptr(pidx),
                                     _ptr(out), B, n, parts), "argmax_f32")

    # ------------------------------------------------------------ EP routing
    def moe_route_count(self, ids, T: int, rank: int, E: int, blockcount, topk: int = 16,
                        stream=None) -> None:
        _dev(ids, "ids", I32, T * topk, align=4)
        _dev(blockcount, "blockcount", I32, -(-T // 256) * E, align=4)
        _check(self.L.k3h_moe_route_count(self.h, _stream(stream), topk, _ptr(ids), T, rank, E,
                                          _ptr(blockcount)), "moe_route_count")

    def moe_route_tables(self, blockcount, blocks: int, E: int, tile: int, blockoff, cta_batch,
                         cta_limit, num_non_exiting, total_padded, route_map, stream=None,
                         T: int | None = None, topk: int = 16) -> None:
        """Tables of the counting sort over `blocks` 256-token blocks.  The route
        tiles number at most (T*topk + (tile-1)*E) // tile (every expert's last
        tile may be partial), which sizes cta_batch / cta_limit and route_map
        (T defaults to blocks*256)."""
        T = blocks * 256 if T is None else T
        if T > blocks * 256:
            raise ValueError("moe_route_tables: T exceeds blocks * 256")
        max_tiles = (T * topk + (tile - 1) * E) // tile
        _dev(blockcount, "blockcount", I32, blocks * E, align=4)
        _dev(blockoff, "blockoff", I32, blocks * E, align=4)
        _dev(cta_batch, "cta_batch", I32, max_tiles, align=4)
        _dev(cta_limit, "cta_limit", I32, max_tiles, align=4)
        _dev(num_non_exiting, "num_non_exiting", I32, 1, align=4)
        _dev(total_padded, "total_padded", I32, 1, align=4)
        _dev(route_map, "route_map", I32, max_tiles * tile, align=4)
        _check(self.L.k3h_moe_route_tables(self.h, _stream(stream), _ptr(blockcount), blocks, E, tile,
                                           _ptr(blockoff), _ptr(cta_batch), _ptr(cta_limit),
                                           _ptr(num_non_exiting), _ptr(total_padded),
                                           _ptr(route_map)), "moe_route_tables")

    def moe_route_scatter(self, ids, blockoff, T: int, rank: int, E: int, route_map, exp2perm,
                          topk: int = 16, stream=None) -> None:
        _dev(ids, "ids", I32, T * topk, align=4)
        _dev(blockoff, "blockoff", I32, -(-T // 256) * E, align=4)
        _dev(route_map, "route_map", I32, 1, align=4)
        _dev(exp2perm, "exp2perm", I32, T * topk, align=4)
        _check(self.L.k3h_moe_route_scatter(self.h, _stream(stream), topk, _ptr(ids), _ptr(blockoff),
                                            T, rank, E, _ptr(route_map), _ptr(exp2perm)),
               "moe_route_scatter")

    def moe_route(self, ids, T: int, rank: int, E: int, blockcount, blockoff, cta_batch, cta_limit,
                  num_non_exiting, total_padded, route_map, exp2perm, sync, topk: int = 16,
                  stream=None) -> None:
        """route_count -> route_tables -> route_scatter in one launch (T <= 65536).
        sync: 2 int32 zeroed before the first call (each call leaves them zero)."""
        blocks = -(-T // 256)
        max_tiles = (T * topk + 127 * E) // 128 if T > 0 else 0  # T = 0 writes no table row
        if blocks > 256:
            raise ValueError("moe_route: T above 65536 (use the three-launch chain)")
        if T > 0:
            _dev(ids, "ids", I32, T * topk, align=4)
            _dev(exp2perm, "exp2perm", I32, T * topk, align=4)
        _dev(blockcount, "blockcount", I32, blocks * E, align=4)
        _dev(blockoff, "blockoff", I32, blocks * E, align=4)
        _dev(cta_batch, "cta_batch", I32, max(1, max_tiles), align=4)
        _dev(cta_limit, "cta_limit", I32, max(1, max_tiles), align=4)
        _dev(num_non_exiting, "num_non_exiting", I32, 1, align=4)
        _dev(total_padded, "total_padded", I32, 1, align=4)
        _dev(route_map, "route_map", I32, max(1, max_tiles * 128), align=4)
        _dev(sync, "sync", I32, 2, align=4)
        _check(self.L.k3h_moe_route(self.h, _stream(stream), topk, _ptr(ids), T, rank, E,
                                    _ptr(blockcount), _ptr(blockoff), _ptr(cta_batch),
                                    _ptr(cta_limit), _ptr(num_non_exiting), _ptr(total_padded),
                                    _ptr(route_map), _ptr(exp2perm), _ptr(sync)), "moe_route")

    def moe_finalize(self, fc2, exp2perm, wts, out, T: int, cols: int, topk: int = 16,
                     stream=None) -> None:
        _dev(fc2, "fc2", BF16, cols)
        _dev(exp2perm, "exp2perm", I32, T * topk, align=4)
        _dev(wts, "wts", F32, T * topk, align=4)
        _dev(out, "out", BF16, T * cols)
        _check(self.L.k3h_moe_finalize(self.h, _stream(stream), topk, _ptr(fc2), _ptr(exp2perm),
                                       _ptr(wts), _ptr(out), T, cols), "moe_finalize")

    def moe_permute_mx(self, q, sf, route_map, total_padded, cols: int, pq, psf,
                       stream=None, tokens: int | None = None) -> None:
        """pq[r] = q[route_map[r]], psf[r] = sf[route_map[r]] for r < total_padded[0]
        (a device value), at most the rows pq / psf hold.  route_map entries index
        rows of q / sf: with `tokens` given, q and sf must hold that many rows (the
        entries are device values, so the host checks the capacity it is told)."""
        if cols <= 0 or cols % 32:
            raise ValueError("moe_permute_mx: cols must be a positive multiple of 32")
        max_rows = min(pq.numel() // cols, psf.numel() // (cols // 32), route_map.numel())
        rows_in = 1 if tokens is None else tokens
        _dev(q, "q", U8, rows_in * cols)
        _dev(sf, "sf", U8, rows_in * (cols // 32), align=4)
        _dev(route_map, "route_map", I32, 1, align=4)
        _dev(total_padded, "total_padded", I32, 1, align=4)
        _dev(pq, "pq", U8, 1)
        _dev(psf, "psf", U8, 1, align=4)
        _check(self.L.k3h_moe_permute_mx(self.h, _stream(stream), _ptr(q), _ptr(sf), _ptr(route_map),
                                         _ptr(total_padded), max_rows, cols, _ptr(pq), _ptr(psf)),
               "moe_permute_mx")

    def moe_w_shuffle(self, src, dst, experts: int, n: int, row_bytes: int, gated: int,
                      stream=None) -> None:
        _dev(src, "src", U8, experts * n * row_bytes)
        _dev(dst, "dst", U8, experts * n * row_bytes)
        _check(self.L.k3h_moe_w_shuffle(self.h, _stream(stream), _ptr(src), _ptr(dst), experts, n,
                                        row_bytes, gated), "moe_w_shuffle")

    def moe_sf_shuffle(self, src, dst, experts: int, n: int, kg: int, gated: int,
                       stream=None) -> None:
        _dev(src, "src", U8, experts * n * kg, align=1)
        _dev(dst, "dst", U8, experts * n * kg, align=1)
        _check(self.L.k3h_moe_sf_shuffle(self.h, _stream(stream), _ptr(src), _ptr(dst), experts, n,
                                         kg, gated), "moe_sf_shuffle")

    # ------------------------------------------------------------ KDA
    def span_gather(self, partial, cw, kda_base, line_index, line_bytes: int, wsm_partial, span_q,
                    span_k, span_v, span_beta, span_flow, span_at, span: int, stream=None) -> None:
        """Manifest op span_gather_v2 -- kern_k3_span_gather, HEADS = 24."""
        inner = 3072
        _dev(partial, "partial", BF16, 4 * inner)
        _dev(cw, "cw", F32, 12 * inner)
        _dev(kda_base, "kda_base", (kda_base.dtype,))
        _dev(line_index, "line_index", I32, 1, align=4)
        _dev(wsm_partial, "wsm_partial", F32, 256)
        for nm, t in (("span_q", span_q), ("span_k", span_k), ("span_v", span_v)):
            _dev(t, nm, BF16, span * inner)
        _dev(span_beta, "span_beta", BF16, 24 * span, align=2)
        _dev(span_flow, "span_flow", BF16, span * 128)
        _dev(span_at, "span_at", I32, 1, align=4)
        _check(self.L.k3h_span_gather(self.h, _stream(stream), _ptr(partial), _ptr(cw), _ptr(kda_base),
                                      _ptr(line_index), line_bytes, _ptr(wsm_partial), _ptr(span_q),
                                      _ptr(span_k), _ptr(span_v), _ptr(span_beta), _ptr(span_flow),
                                      _ptr(span_at), span), "span_gather")

    def kda_out_gate(self, attn, gate_partial, gamma_o, gated, span_at, span: int,
                     stream=None, eps: float = 1e-5) -> None:
        """Manifest op kda_out_gate_v2 -- kern_k3_kda_out_gate, HEADS = 24; eps picks the
        module (1e-5, or 1e-6 for the +K11_RMS_EPS=1e-6f build)."""
        _dev(attn, "attn", BF16, span * 3072)
        _dev(gate_partial, "gate_partial", BF16, 4 * 3072)
        _dev(gamma_o, "gamma_o", F32, 128)
        _dev(gated, "gated", BF16, 3072)
        _dev(span_at, "span_at", I32, 1, align=4)
        _check(self.L.k3h_kda_out_gate(self.h, _stream(stream), _ptr(attn), _ptr(gate_partial),
                                       _ptr(gamma_o), _ptr(gated), _ptr(span_at), span, eps),
               "kda_out_gate")

    # ------------------------------------------------------------ MLA
    def mla_prep(self, partial, gamma_q_a, gamma_kv_a, slot_mapping, slab, layer_off: int,
                 q_norm, mla_gate, B: int, page_stride: int = 884736, stream=None) -> None:
        """Manifest op mla_prep (partial, gamma_q_a, gamma_kv_a, slot_mapping, state kv,
        layer_off, q_norm, mla_gate, B): head launch then gate launch."""
        _dev(partial, "partial", BF16 + F32, B * 5184)
        _dev(gamma_q_a, "gamma_q_a", BF16, 1536, align=8)
        _dev(gamma_kv_a, "gamma_kv_a", BF16, 512, align=8)
        _dev(slot_mapping, "slot_mapping", I64, B, align=8)
        _dev(slab, "slab", BF16, 1, align=8)
        _dev(q_norm, "q_norm", BF16, B * 1536, align=8)
        _dev(mla_gate, "mla_gate", BF16, B * 3072)
        _check(self.L.k3h_mla_prep(self.h, _stream(stream), int(partial.dtype == torch.bfloat16),
                                   _ptr(partial), _ptr(gamma_q_a), _ptr(gamma_kv_a),
                                   _ptr(slot_mapping), _ptr(slab), layer_off, page_stride,
                                   _ptr(q_norm), _ptr(mla_gate), B), "mla_prep")

    def mla_rope_pack(self, latent, k_rope, q, gamma_kv, positions, latent_out, q_out, T: int,
                      H: int, theta: float = 50000.0, eps: float = 1e-6, stream=None) -> None:
        _dev(latent, "latent", BF16, T * 512)
        _dev(k_rope, "k_rope", BF16, T * 64)
        _dev(q, "q", BF16, T * H * 192)
        _dev(gamma_kv, "gamma_kv", BF16, 512)
        _dev(positions, "positions", I64, T, align=8)
        _dev(latent_out, "latent_out", BF16, T * 576)
        _dev(q_out, "q_out", BF16, T * H * 192)
        _check(self.L.k3h_mla_rope_pack(self.h, _stream(stream), _ptr(latent), _ptr(k_rope), _ptr(q),
                                        _ptr(gamma_kv), _ptr(positions), _ptr(latent_out),
                                        _ptr(q_out), theta, eps, T, H), "mla_rope_pack")

    # ------------------------------------------------------------ MoE expert GEMMs
    GEMM_F32, GEMM_BF16, GEMM_SITU_MX, GEMM_F32_SITU_TILING = 0, 1, 2, 3

    def moe_w_tile(self, src, dst, experts: int, n: int, k: int, gated: int, stream=None) -> None:
        """Row-major e2m1 weights [experts, n, k/2] -> the MFMA-operand tiled layout."""
        nbytes = experts * n * k // 2
        _dev(src, "src", U8, nbytes)
        _dev(dst, "dst", U8, nbytes)
        _check(self.L.k3h_moe_w_tile(self.h, _stream(stream), _ptr(src), _ptr(dst), experts, n, k,
                                     gated), "moe_w_tile")

    def moe_sf_tile(self, src, dst, experts: int, n: int, k: int, gated: int, stream=None) -> None:
        """E8M0 scales [experts, n, k/32] -> the tiled scale layout."""
        nbytes = experts * n * k // 32
        _dev(src, "src", U8, nbytes, align=1)
        _dev(dst, "dst", U8, nbytes, align=8)
        _check(self.L.k3h_moe_sf_tile(self.h, _stream(stream), _ptr(src), _ptr(dst), experts, n, k,
                                      gated), "moe_sf_tile")

    def moe_gemm_mx(self, epilogue: int, a, a_sf, a_rows, wt, wsf, num_tiles, cta_batch,
                    max_tiles: int, E: int, N: int, K: int, out, out_sf=None, alpha=None,
                    beta=None, stream=None) -> None:
        """MX GEMM over the route tiles (epilogue GEMM_F32 / GEMM_BF16 / GEMM_SITU_MX, or
        GEMM_F32_SITU_TILING: the f32 accumulators of the GEMM_SITU_MX kernel's own tiling)."""
        rows = max_tiles * 128
        if a_rows is None:
            # A is read in place: one row per padded row of every tile (32-bit row offsets)
            if rows * K > 0xFFFFFFFF:
                raise ValueError("moe_gemm_mx: max_tiles * 128 * K must stay below 2^32")
            _dev(a, "a", U8, rows * K, align=16)
            _dev(a_sf, "a_sf", U8, rows * K // 32, align=4)
        else:
            _dev(a, "a", U8, K, align=16)
            _dev(a_sf, "a_sf", U8, K // 32, align=4)
            _dev(a_rows, "a_rows", I32, rows, align=4)
        _dev(wt, "wt", U8, E * N * K // 2)
        _dev(wsf, "wsf", U8, E * N * K // 32, align=8)
        _dev(num_tiles, "num_tiles", I32, 1, align=4)
        _dev(cta_batch, "cta_batch", I32, max_tiles, align=4)
        if epilogue == self.GEMM_F32:
            _dev(out, "out", F32, rows * N, align=4)
        elif epilogue == self.GEMM_F32_SITU_TILING:
            _dev(out, "out", F32, rows * N, align=16)
        elif epilogue == self.GEMM_BF16:
            _dev(out, "out", BF16, rows * N, align=16)
        else:
            _dev(out, "out", U8, rows * N // 2, align=16)
            _dev(out_sf, "out_sf", U8, rows * N // 64, align=2)
            _dev(alpha, "alpha", F32, E, align=4)
            _dev(beta, "beta", F32, E, align=4)
        _check(self.L.k3h_moe_gemm_mx(self.h, _stream(stream), epilogue, _ptr(a), _ptr(a_sf),
                                      _ptr(a_rows), _ptr(wt), _ptr(wsf), _ptr(num_tiles),
                                      _ptr(cta_batch), max_tiles, E, N, K, _ptr(out), _ptr(out_sf),
                                      _ptr(alpha), _ptr(beta)), "moe_gemm_mx")

    # ------------------------------------------------------------ measurement
    def stream_copy(self, src, dst, stream=None) -> None:
        """dst <- src with 16-byte non-temporal loads/stores (the HBM copy ceiling)."""
        nbytes = src.numel() * src.element_size()
        if nbytes % 16 or dst.numel() * dst.element_size() < nbytes:
            raise ValueError("stream_copy: size must be a multiple of 16 bytes and fit dst")
        _dev(src, "src", (src.dtype,))
        _dev(dst, "dst", (dst.dtype,))
        _check(self.L.k3h_stream_copy(self.h, _stream(stream), _ptr(src), _ptr(dst), nbytes // 16),
               "stream_copy")


# ---------------------------------------------------------------- manifest ops
def _eval_expr(e: Any, env: dict[str, int]) -> int:
    """Grid expressions of the manifest: ints, variable names, ceil_div/mul/add."""
    if isinstance(e, int):
        return e
    if isinstance(e, str):
        return int(env[e])
    if isinstance(e, dict) and len(e) == 1:
        (op, args), = e.items()
        v = [_eval_expr(a, env) for a in args]
        if op == "ceil_div":
            return -(-v[0] // v[1])
        if op == "mul":
            return v[0] * v[1]
        if op == "add":
            return v[0] + v[1]
    raise ValueError(f"unsupported grid expression {e!r}")


def pack_args(kinds: Sequence[str], values: Sequence[Any]) -> bytes:
    """Pack launch arguments at natural alignment (buffers/state/i64: 8 B; i32/f32: 4 B)."""
    out = bytearray()
    for kind, v in zip(kinds, values):
        k = kind.split()[-1]
        if k.startswith("buffer") or k == "state":
            fmt, al = "<Q", 8
            v = 0 if v is None else (v.data_ptr() if isinstance(v, torch.Tensor) else int(v))
        elif k == "i64":
            fmt, al = "<q", 8
        elif k == "i32":
            fmt, al = "<i", 4
        elif k == "f32":
            fmt, al = "<f", 4
        else:
            raise ValueError(f"unsupported parameter kind {kind!r}")
        out += b"\0" * ((-len(out)) % al)
        out += struct.pack(fmt, v)
    return bytes(out)


class ManifestOp:
    """One manifest op (``ops.<name>``) executed launch by launch through k3h_launch."""

    def __init__(self, ctx: Ctx, name: str, spec: dict):
        self.ctx, self.name, self.spec = ctx, name, spec
        self.params = spec["params"]

    def __call__(self, args: Sequence[Any], env: dict[str, int], stream=None) -> None:
        if len(args) != len(self.params):
            raise ValueError(f"{self.name}: {len(self.params)} arguments expected")
        L = self.ctx.L
        for ln in self.spec["impl"]["launches"]:
            kinds = ln.get("params", self.params)
            if "args" in ln:
                vals = []
                for a in ln["args"]:
                    (k, v), = a.items()
                    if k == "param":
                        vals.append(args[v])
                    elif k == "rank":  # this process's rank in group v ("tp" / "ep")
                        vals.append(int(env[f"rank_{v}"]))
                    else:
                        vals.append(v)
            else:
                vals = list(args)
            buf = pack_args(kinds, vals)
            fn = self.ctx.function(ln["module"], ln["entry"])
            grid = (ctypes.c_uint32 * 3)(*[_eval_expr(g, env) for g in ln["grid"]])
            block = (ctypes.c_uint32 * 3)(*ln["block"])
            cbuf = ctypes.create_string_buffer(buf, len(buf))
            _check(L.k3h_launch(fn, grid, block, ln.get("shared_mem", 0), _stream(stream),
                                ctypes.cast(cbuf, _P), len(buf)),
                   f"{self.name}:{ln['entry']}")
