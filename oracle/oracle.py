"""numpy front end of the C oracle (``libk3oracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and
the CPU-baseline leg of ``bench.py``; the product path never loads it.

bf16 arrays are ``np.uint16`` bit patterns; e4m3 / E8M0 arrays ``np.uint8``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ODIR = os.path.dirname(os.path.abspath(__file__))
# K3_ORACLE_LIB: another build of the same sources (bench.py's CPU baseline times a
# build made with -march=native on the host it runs on)
LIB_PATH = os.environ.get("K3_ORACLE_LIB") or os.path.join(ODIR, "libk3oracle.so")
H = 7168

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-s", "-C", ODIR], check=True)
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.k3o_bf2f.restype = ctypes.c_float
        _lib.k3o_bf2f.argtypes = [ctypes.c_uint16]
        _lib.k3o_f2bf.restype = ctypes.c_uint16
        _lib.k3o_f2bf.argtypes = [ctypes.c_float]
        _lib.k3o_e4m3.restype = ctypes.c_uint8
        _lib.k3o_e4m3.argtypes = [ctypes.c_float]
        _lib.k3o_e4m3_decode.restype = ctypes.c_float
        _lib.k3o_e4m3_decode.argtypes = [ctypes.c_uint8]
        _lib.k3o_expf.restype = ctypes.c_float
        _lib.k3o_expf.argtypes = [ctypes.c_float]
        _lib.k3o_sigmoid.restype = ctypes.c_float
        _lib.k3o_sigmoid.argtypes = [ctypes.c_float]
        _lib.k3o_mx_exp.restype = ctypes.c_int
        _lib.k3o_mx_exp.argtypes = [ctypes.c_float]
        _lib.k3o_num_threads.restype = ctypes.c_int
        _lib.k3o_situ.restype = ctypes.c_float
        _lib.k3o_situ.argtypes = [ctypes.c_float, ctypes.c_float]
        _lib.k3o_e2m1_decode.restype = ctypes.c_float
        _lib.k3o_e2m1_decode.argtypes = [ctypes.c_uint8]
        _lib.k3o_rs_arrive.restype = ctypes.c_uint
        _lib.k3o_rs_arrive.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_longlong]
        _lib.k3o_epoch_bump.argtypes = [ctypes.c_void_p, ctypes.c_int]
        _lib.k3o_flags_init.argtypes = [ctypes.c_void_p, ctypes.c_int]
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def num_threads() -> int:
    return lib().k3o_num_threads()


# ---------------------------------------------------------------- numerics
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().k3o_f2bf_n(_p(x), _p(y), ctypes.c_size_t(x.size))
    return y


def e4m3(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint8)
    lib().k3o_e4m3_n(_p(x), _p(y), ctypes.c_size_t(x.size))
    return y


def e4m3_decode(c: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.k3o_e4m3_decode(int(v)) for v in c.ravel()], np.float32).reshape(c.shape)


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().k3o_expf_n(_p(x), _p(y), ctypes.c_size_t(x.size))
    return y


def mx_exp(amax: float) -> int:
    return lib().k3o_mx_exp(float(amax))


# ---------------------------------------------------------------- K1 family
def land_add_attnres_rms(partial, prefix, blocks, sw, gamma, nb, snapshot, B, eps=1e-5):
    """Returns (prefix2, normed); partial uint16 (bf16) or float32."""
    prefix2 = np.empty((B, H), np.uint16)
    normed = np.empty((B, H), np.uint16)
    bf = partial.dtype == np.uint16
    lib().k3o_land_add_attnres_rms(
        _p(partial) if bf else None, None if bf else _p(partial), _p(prefix), _p(blocks), _p(sw),
        _p(gamma), _p(prefix2), _p(normed), nb, snapshot, B, ctypes.c_float(eps))
    return prefix2, normed


def attnres_rms(prefix, blocks, sw, gamma, nb, snapshot, B, eps=1e-5):
    """Returns (blocks_out, normed); blocks is copied, not modified."""
    blocks_out = None if blocks is None else blocks.copy()
    normed = np.empty((B, H), np.uint16)
    lib().k3o_attnres_rms(_p(prefix), _p(blocks_out), _p(sw), _p(gamma), _p(normed), nb, snapshot,
                          B, ctypes.c_float(eps))
    return blocks_out, normed


def land_add2(p1, p2, prefix2, two, B):
    hidden = np.empty((B, H), np.uint16)
    lib().k3o_land_add2(_p(p1), _p(p2), _p(prefix2), _p(hidden), two, B)
    return hidden


def land_add2_bf16(p1, p2, prefix2, two, B):
    """kern_k3_land_add2_bf16: bf16 partials (uint16)."""
    hidden = np.empty((B, H), np.uint16)
    lib().k3o_land_add2_bf16(_p(p1), _p(p2), _p(prefix2), _p(hidden), two, B)
    return hidden


def attnres_rms_stats(prefix, blocks, sw, gamma, nb, snapshot, B, sw_mlp=None, eps=1e-5):
    """res_in of the push family: returns (blocks_out, normed, stats [B, 8, 2] or None)."""
    blocks_out = None if blocks is None else blocks.copy()
    normed = np.empty((B, H), np.uint16)
    stats = None if sw_mlp is None else np.zeros((B, 8, 2), np.float32)
    lib().k3o_attnres_rms_stats(_p(prefix), _p(blocks_out), _p(sw), _p(gamma), _p(normed), nb,
                                snapshot, B, ctypes.c_float(eps),
                                None if sw_mlp is None else _p(np.ascontiguousarray(sw_mlp, np.float32)),
                                _p(stats))
    return blocks_out, normed, stats


def land_add_attnres_rms_stats(partial, prefix, blocks, sw, gamma, nb, snapshot, B, stats,
                               nb_stats, eps=1e-5):
    """res_mlp with res_in's candidate statistics; returns (prefix2, normed)."""
    prefix2 = np.empty((B, H), np.uint16)
    normed = np.empty((B, H), np.uint16)
    bf = partial.dtype == np.uint16
    lib().k3o_land_add_attnres_rms_stats(
        _p(partial) if bf else None, None if bf else _p(partial), _p(prefix), _p(blocks), _p(sw),
        _p(gamma), _p(prefix2), _p(normed), nb, snapshot, B, ctypes.c_float(eps),
        None if stats is None else _p(np.ascontiguousarray(stats, np.float32)), nb_stats)
    return prefix2, normed


# ---------------------------------------------------------------- MXFP8
def moe_quant(x, rows, cols):
    n = rows * cols
    q = np.empty(n, np.uint8)
    sf = np.empty(n // 32, np.uint8)
    lib().k3o_moe_quant(_p(np.ascontiguousarray(x)), _p(q), _p(sf), rows, cols)
    return q.reshape(rows, cols), sf.reshape(rows, cols // 32)


def par_copy(a):
    """A copy of array a whose pages the OpenMP threads touch first."""
    a = np.ascontiguousarray(a)
    out = np.empty_like(a)
    lib().k3o_par_copy(_p(out), _p(a), ctypes.c_size_t(a.nbytes))
    return out


def residual_rms_mxfp8(x, residual, gamma, B, eps=1e-6, want_normed=True, out=None):
    """out: optional (res_out, q, sf, normed) arrays to write (allocated by the caller)."""
    if out is not None:
        res_out, q, sf, normed = out
    else:
        res_out = np.empty((B, H), np.uint16)
        q = np.empty((B, H), np.uint8)
        sf = np.empty((B, H // 32), np.uint8)
        normed = np.empty((B, H), np.uint16) if want_normed else None
    lib().k3o_residual_rms_mxfp8(_p(x), _p(residual), _p(gamma), _p(res_out), _p(q), _p(sf),
                                 _p(normed), B, ctypes.c_float(eps))
    return res_out, q, sf, normed


def quant_fp8_amax(x, n, nb_grid, v2=True):
    partials = np.empty(nb_grid, np.float32)
    lib().k3o_quant_fp8_amax(_p(x), n, _p(partials), nb_grid, int(v2))
    return partials


def quant_fp8_apply(x, n, partials, nb):
    y = np.empty(n, np.uint8)
    scale = np.empty(1, np.float32)
    lib().k3o_quant_fp8_apply(_p(x), _p(y), n, _p(partials), nb, _p(scale))
    return y, scale


# ---------------------------------------------------------------- router / argmax
def sigmoid(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().k3o_sigmoid_n(_p(x), _p(y), ctypes.c_size_t(x.size))
    return y


def router_topk(S, bias, rs_bf16, B, topk):
    idx = np.empty((B, topk), np.int32)
    wts = np.empty((B, topk), np.float32)
    rs = np.ascontiguousarray(np.array([rs_bf16], np.uint16).reshape(-1)[:1])
    lib().k3o_router_topk(_p(np.ascontiguousarray(S, np.float32)), _p(np.ascontiguousarray(bias, np.float32)),
                          _p(rs), _p(idx), _p(wts), B, topk)
    return idx, wts


def argmax_partial(logits, B, n, parts):
    pmax = np.empty(B * parts, np.float32)
    pidx = np.empty(B * parts, np.int32)
    lib().k3o_argmax_partial(_p(np.ascontiguousarray(logits, np.float32)), _p(pmax), _p(pidx), B, n, parts)
    return pmax, pidx


def argmax_final(pmax, pidx, B, parts):
    out = np.empty(B, np.int64)
    lib().k3o_argmax_final(_p(pmax), _p(pidx), _p(out), B, parts)
    return out


# ---------------------------------------------------------------- EP routing
def local_expert(i, rank, E, ep_ranks=4, strided=1):
    return lib().k3o_local_expert(int(i), rank, E, ep_ranks, strided)


def route_count(ids, T, topk, rank, E, ep_ranks=4, strided=1):
    nblk = (T + 255) // 256
    bc = np.empty(nblk * E, np.int32)
    lib().k3o_route_count(_p(np.ascontiguousarray(ids, np.int32)), T, topk, rank, E, ep_ranks, strided, _p(bc))
    return bc


def route_tables(blockcount, blocks, E, tile, route_map_len):
    """Returns dict of blockoff, cta_batch, cta_limit, num_non_exiting, total_padded and
    route_map (padding rows only; other rows -1 sentinel as the oracle leaves them)."""
    blockoff = np.empty(blocks * E, np.int32)
    nmax = route_map_len // tile + 1
    cta_batch = np.full(nmax, -1, np.int32)
    cta_limit = np.full(nmax, -1, np.int32)
    nne = np.zeros(1, np.int32)
    tp = np.zeros(1, np.int32)
    rmap = np.full(route_map_len, -1, np.int32)
    lib().k3o_route_tables(_p(np.ascontiguousarray(blockcount, np.int32)), blocks, E, tile, _p(blockoff),
                           _p(cta_batch), _p(cta_limit), _p(nne), _p(tp), _p(rmap))
    return dict(blockoff=blockoff, cta_batch=cta_batch, cta_limit=cta_limit,
                num_non_exiting=int(nne[0]), total_padded=int(tp[0]), route_map=rmap)


def route_scatter(ids, blockoff, T, topk, rank, E, route_map, ep_ranks=4, strided=1):
    rmap = route_map.copy()
    e2p = np.empty(T * topk, np.int32)
    lib().k3o_route_scatter(_p(np.ascontiguousarray(ids, np.int32)), _p(blockoff), T, topk, rank, E,
                            ep_ranks, strided, _p(rmap), _p(e2p))
    return rmap, e2p


def moe_permute_mx(q, sf, route_map, total_padded, cols):
    pq = np.empty((total_padded, cols), np.uint8)
    psf = np.empty((total_padded, cols // 32), np.uint8)
    lib().k3o_moe_permute_mx(_p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(sf)),
                             _p(np.ascontiguousarray(route_map, np.int32)), total_padded, cols, _p(pq), _p(psf))
    return pq, psf


def moe_finalize(fc2, exp2perm, wts, T, topk, cols):
    out = np.empty((T, cols), np.uint16)
    lib().k3o_moe_finalize(_p(np.ascontiguousarray(fc2)), _p(np.ascontiguousarray(exp2perm, np.int32)),
                           _p(np.ascontiguousarray(wts, np.float32)), _p(out), T, topk, cols)
    return out


def moe_w_shuffle(src, experts, n, row_bytes, gated):
    dst = np.empty_like(src)
    lib().k3o_moe_w_shuffle(_p(src), _p(dst), experts, n, row_bytes, gated)
    return dst


def moe_sf_shuffle(src, experts, n, kg, gated):
    dst = np.empty_like(src)
    lib().k3o_moe_sf_shuffle(_p(src), _p(dst), experts, n, kg, gated)
    return dst


# ---------------------------------------------------------------- KDA
def span_gather(partial, cw, win, wsm, at, span, heads=24):
    """Returns (q, k, v, beta, flow, new_win); win [3, 3, inner] bf16 is not modified."""
    inner = heads * 128
    w = np.ascontiguousarray(win, np.uint16).copy()
    q = np.empty((span, inner), np.uint16)
    k = np.empty((span, inner), np.uint16)
    v = np.empty((span, inner), np.uint16)
    beta = np.empty(heads * span, np.uint16)
    flow = np.empty((span, 128), np.uint16)
    lib().k3o_span_gather(_p(np.ascontiguousarray(partial)), _p(np.ascontiguousarray(cw, np.float32)),
                          _p(w), _p(np.ascontiguousarray(wsm, np.float32)), _p(q), _p(k), _p(v),
                          _p(beta), _p(flow), at, span, heads)
    return q, k, v, beta, flow, w


def kda_out_gate(attn, gate_partial, gamma_o, gated_in, at, span, heads=24, eps=1e-5):
    """eps is the module's K11_RMS_EPS (1e-5, or 1e-6 for config 3)."""
    gated = np.ascontiguousarray(gated_in, np.uint16).copy()
    lib().k3o_kda_out_gate(_p(np.ascontiguousarray(attn)), _p(np.ascontiguousarray(gate_partial)),
                           _p(np.ascontiguousarray(gamma_o, np.float32)), _p(gated), at, span, heads,
                           ctypes.c_float(eps))
    return gated


# ---------------------------------------------------------------- MLA
def mla_prep(partial, gamma_q_a, gamma_kv_a, slot_mapping, slab_in, layer_off, page_stride, B,
             inner=3072, mla_fused=5184):
    """Returns (slab, q_norm, mla_gate); partial float32 or uint16 (bf16) [B, mla_fused]."""
    slab = np.ascontiguousarray(slab_in, np.uint16).copy()
    q_norm = np.empty((B, 1536), np.uint16)
    gate = np.empty((B, inner), np.uint16)
    bf = partial.dtype == np.uint16
    partial = np.ascontiguousarray(partial)
    lib().k3o_mla_prep(None if bf else _p(partial), _p(partial) if bf else None, mla_fused, inner,
                       _p(gamma_q_a), _p(gamma_kv_a), _p(np.ascontiguousarray(slot_mapping, np.int64)),
                       _p(slab), ctypes.c_longlong(layer_off), ctypes.c_longlong(page_stride),
                       _p(q_norm), _p(gate), B)
    return slab, q_norm, gate


def mla_rope_pack(latent, k_rope, q, gamma_kv, positions, T, H, theta=50000.0, eps=1e-6):
    lat = np.empty((T, 576), np.uint16)
    qo = np.empty((T, H, 192), np.uint16)
    lib().k3o_mla_rope_pack(_p(np.ascontiguousarray(latent)), _p(np.ascontiguousarray(k_rope)),
                            _p(np.ascontiguousarray(q)), _p(gamma_kv),
                            _p(np.ascontiguousarray(positions, np.int64)), _p(lat), _p(qo),
                            ctypes.c_float(theta), ctypes.c_float(eps), T, H)
    return lat, qo


# ---------------------------------------------------------------- landing kernels
def rms(x, gamma, h, B):
    o = np.zeros((B, h), np.uint16)
    lib().k3o_rms(_p(np.ascontiguousarray(x)), _p(np.ascontiguousarray(gamma)), _p(o), h, B)
    return o


def land(p, n, off, ldc, B):
    o = np.empty((B, n), np.uint16)
    lib().k3o_land(_p(np.ascontiguousarray(p, np.float32)), _p(o), n, off, ldc, B)
    return o


def situ(g, u):
    """Exact SiTU of f32 operands (elementwise), as the f32 value that lands."""
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    y = np.empty_like(g)
    lib().k3o_situ_n(_p(g), _p(u), _p(y), ctypes.c_size_t(g.size))
    return y


def land_situ(p, n, B):
    """p float32 or uint16 (bf16) [B, 2n] -> act [B, n] bf16."""
    act = np.empty((B, n), np.uint16)
    p = np.ascontiguousarray(p)
    f32 = p.dtype == np.float32
    lib().k3o_land_situ(_p(p) if f32 else None, None if f32 else _p(p), _p(act), n, B)
    return act


def situ_rms(sp, lat, gam, n, B, h, L, tokens, act_in=None, ln_in=None):
    """kern_k3_situ_rms_bf16: returns (act, ln); rows outside the grid keep act_in / ln_in."""
    act = np.zeros((B, n), np.uint16) if act_in is None else np.array(act_in, np.uint16)
    ln = np.zeros((L, h), np.uint16) if ln_in is None else np.array(ln_in, np.uint16)
    lib().k3o_situ_rms(_p(np.ascontiguousarray(sp)), _p(act), _p(np.ascontiguousarray(lat)),
                       _p(np.ascontiguousarray(gam)), _p(ln), n, B, h, L, tokens)
    return act, ln


# ---------------------------------------------------------------- MoE expert GEMMs
def e2m1_decode(nib):
    nib = np.asarray(nib, np.uint8)
    f = np.vectorize(lambda v: lib().k3o_e2m1_decode(int(v)), otypes=[np.float32])
    return f(nib)


def moe_gemm_mx(a, a_sf, a_rows, w, w_sf, num_tiles, cta_batch, E, N, K, magnitude=False):
    """Double-precision MX GEMM over the route tiles t < num_tiles (rows [128 t, 128 t + 128),
    expert cta_batch[t]); rows of skipped tiles are NaN.  magnitude=True returns sum |a w|."""
    assert K <= 8192 and K % 32 == 0 and N > 0
    out = np.full((num_tiles * 128, N), np.nan, np.float64)
    fn = lib().k3o_moe_gemm_mx_abs if magnitude else lib().k3o_moe_gemm_mx
    rows = None if a_rows is None else np.ascontiguousarray(a_rows, np.int32)
    fn(_p(np.ascontiguousarray(a, np.uint8)), _p(np.ascontiguousarray(a_sf, np.uint8)), _p(rows),
       _p(np.ascontiguousarray(w, np.uint8)), _p(np.ascontiguousarray(w_sf, np.uint8)),
       int(num_tiles), _p(np.ascontiguousarray(cta_batch, np.int32)), E, N, K, _p(out))
    return out


def situ_ab(g, u, alpha, beta):
    """Exact gated activation of f32 operands with per-call alpha / beta (f32 value that lands)."""
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    y = np.empty_like(g)
    lib().k3o_situ_ab_n(_p(g), _p(u), _p(y), ctypes.c_size_t(g.size), ctypes.c_float(alpha),
                        ctypes.c_float(beta))
    return y


def moe_fc1_epilogue(c, alpha_rows, beta_rows):
    """fc1 epilogue on f32 accumulators c [rows, N] in weight-row order ([up | gate]):
    u = bf16(c[:, :N/2]), g = bf16(c[:, N/2:]), x = bf16(situ(g, u; alpha, beta)) per row's
    expert, then MX quantisation of x -> (q [rows, N/2], sf [rows, N/64])."""
    c = np.ascontiguousarray(c, np.float32)
    rows, N = c.shape
    half = N // 2
    bf = lambda v: (((v.view(np.uint32).astype(np.uint64) + 0x7FFF +
                      ((v.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16))
    up16, gate16 = bf(np.ascontiguousarray(c[:, :half])), bf(np.ascontiguousarray(c[:, half:]))
    u = (up16.astype(np.uint32) << 16).view(np.float32)
    g = (gate16.astype(np.uint32) << 16).view(np.float32)
    alpha_rows = np.asarray(alpha_rows, np.float32)
    beta_rows = np.asarray(beta_rows, np.float32)
    if rows and (alpha_rows == alpha_rows[0]).all() and (beta_rows == beta_rows[0]).all():
        x = situ_ab(g, u, float(alpha_rows[0]), float(beta_rows[0]))  # one call for every row
    else:
        x = np.empty((rows, half), np.float32)
        for r in range(rows):
            x[r] = situ_ab(g[r], u[r], float(alpha_rows[r]), float(beta_rows[r]))
    x16 = bf(x)
    return moe_quant(x16, rows, half)


# ---- epoch / arrival barrier (host threads play the ranks)
def flags_init(flags: np.ndarray) -> None:
    """kern_k3_flags_init: every counter of a uint64 array to 0."""
    assert flags.dtype == np.uint64
    lib().k3o_flags_init(_p(flags), flags.size)


def epoch_bump(flags: np.ndarray, units: int) -> None:
    """kern_k3_epoch_bump: flags[0] += units."""
    lib().k3o_epoch_bump(_p(flags), units)


def rs_arrive(flags: np.ndarray, flags_peer: np.ndarray, units: int, slot: int, nranks: int,
              spin_ns: int) -> int:
    """kern_k3_rs_arrive1: flags[slot] += units, then wait (at most spin_ns) until every
    rank's counter (flags_peer: uint64 addresses) reaches flags[0]; returns the mask of
    the ranks given up on.  The GIL is released for the call (ctypes), so threads can
    play the ranks."""
    assert flags.dtype == np.uint64 and flags_peer.dtype == np.uint64
    return int(lib().k3o_rs_arrive(_p(flags), _p(flags_peer), units, slot, nranks, spin_ns))

