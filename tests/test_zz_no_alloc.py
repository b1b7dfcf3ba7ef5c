"""GPU: the allocation-free entry k3h_quant_fp8_tensor_noalloc (amax partials in
the library's per-GPU device array) against the allocating entry
k3h_quant_fp8_tensor (partials in a caller buffer), both called through the
C-ABI on the same inputs: the e4m3 payload and the scale bit-exact.  Two calls
in a row, the second over a smaller, ragged input with fewer partials, so stale
partials of the first call would show; device free memory is unchanged across
the second allocation-free call (the first call on a device resolves the
array's address, a one-time set-up)."""
import ctypes

import numpy as np
import pytest
import torch

import k3h

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _inputs(n, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn(n, generator=g, device="cuda")
    out = torch.rand(n, generator=g, device="cuda") < 0.001
    return torch.where(out, x * 50.0, x).to(torch.bfloat16)


def _pair(ctx, x, n, nb, v2):
    """Both entries through the C-ABI; returns (y_alloc, scale_alloc, y_noalloc, scale_noalloc)."""
    L, s = ctx.L, torch.cuda.current_stream().cuda_stream
    y0 = torch.full((n,), 0x5a, dtype=torch.uint8, device="cuda")
    y1 = torch.full((n,), 0xa5, dtype=torch.uint8, device="cuda")
    sc0 = torch.zeros(1, dtype=torch.float32, device="cuda")
    sc1 = torch.zeros(1, dtype=torch.float32, device="cuda")
    parts = torch.empty(nb, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    assert L.k3h_quant_fp8_tensor(ctx.h, s, v2, x.data_ptr(), y0.data_ptr(), sc0.data_ptr(),
                                  parts.data_ptr(), n, nb) == 0
    free0 = torch.cuda.mem_get_info()[0]
    assert L.k3h_quant_fp8_tensor_noalloc(ctx.h, s, v2, x.data_ptr(), y1.data_ptr(),
                                          sc1.data_ptr(), n, nb) == 0
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    return y0, sc0, y1, sc1, free0, free1


@pytest.mark.parametrize("v2", [1, 0])
def test_noalloc_matches_allocating_entry(ctx, v2):
    for i, (n, nb) in enumerate([(16384 * 7168, 2048), (1_000_003, 300)]):
        _case(f"quant_fp8_tensor_noalloc v2={v2} call {i + 1}: n={n} nb={nb}")
        x = _inputs(n, 9100 + 10 * v2 + i)
        y0, sc0, y1, sc1, free0, free1 = _pair(ctx, x, n, nb, v2)
        assert sc0.item() > 0 and sc1.view(torch.int32).item() == sc0.view(torch.int32).item()
        ndiff = int((y0 != y1).sum().item())
        print(f"  scale {sc1.item():.6g}, payload bytes differing: {ndiff}", flush=True)
        assert ndiff == 0
        if i == 1:
            assert free1 == free0, "the allocation-free entry changed device free memory"


def test_noalloc_rejects_too_many_partials(ctx):
    x = torch.zeros(64, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros(64, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(1, dtype=torch.float32, device="cuda")
    rc = ctx.L.k3h_quant_fp8_tensor_noalloc(ctx.h, None, 1, x.data_ptr(), y.data_ptr(),
                                            sc.data_ptr(), 64, k3h.NOALLOC_MAX_NB + 1)
    assert rc == k3h.K3H_EINVAL
    with pytest.raises(ValueError):
        ctx.quant_fp8_tensor_noalloc(x, y, sc, 64, nb=k3h.NOALLOC_MAX_NB + 1)
