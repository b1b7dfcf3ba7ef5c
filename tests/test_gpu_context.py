"""GPU: one k3h context shared by host threads.  The context loads code objects
lazily under its own lock; concurrent first lookups must all return the same
function handle and leave the context usable."""
import threading

import pytest
import torch

import k3h

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def test_context_shared_by_threads():
    """One fresh context, eight host threads looking up entries of several module
    keys at once (the first lookups load the code objects): every thread gets the
    same handle for the same (key, entry), and a launch through it works."""
    _case("context lookups from eight threads")
    c = k3h.Ctx()
    names = [("k3h_fused", "k3h_residual_rms_mxfp8"), ("k3h_fused", "k3h_stream_copy"),
             ("k3_land", "kern_k3_rms"), ("k3_rs_arrive_v2", "kern_k3_rs_arrive1"),
             ("k3_collectives", "kern_k3_epoch_bump"), ("k3h_probe", "k3h_probe_read_u4")]
    got, errors = {}, []

    def body(i):
        try:
            for k in range(len(names)):
                key = names[(i + k) % len(names)]
                got.setdefault(key, set()).add(c.function(*key))
        except BaseException as e:
            errors.append(e)

    ts = [threading.Thread(target=body, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(60)
    assert not errors, errors
    assert all(len(v) == 1 for v in got.values()) and len(got) == len(names)
    flags = torch.zeros(4, dtype=torch.int64, device="cuda")
    c.epoch_bump(flags, 3)
    torch.cuda.synchronize()
    assert int(flags[0]) == 3
    c.close()
