"""dsmoe_forward_noalloc (static device scratch, no context, no allocation)
against dsmoe_forward on the same inputs: routing, weights and both outputs
bit for bit, on two calls in a row, the second with fewer tokens (the static
scratch keeps the first call's contents; the row counters of the fused mid
quantization must be back at zero)."""
import ctypes
import dataclasses
import sys

import numpy as np
import pytest

import dsmoe
from dsmoe import configs as C

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _bits(t):
    return t.detach().cpu().numpy().view(np.uint8)


def _case(name):
    if name == "c2_noshared":
        case = C.CASES["c2"]
        return dataclasses.replace(case, cfg=dataclasses.replace(case.cfg, shared_fmt=-1))
    return C.CASES[name]


@pytest.mark.parametrize("name,Ts", [("c1", [8, 3]), ("c2", [5, 1]), ("c2_noshared", [8, 2])])
def test_noalloc_equals_forward(gpu, name, Ts):
    import torch
    case = _case(name)
    cfg = case.cfg
    d, k = cfg.d_model, cfg.top_k
    w = C.make_weights(case, device=gpu)
    lay = dsmoe.MoeLayer(cfg, 8)
    for call, T in enumerate(Ts):
        say(f"noalloc vs forward {name} call={call} T={T}")
        x = C.make_x(case, T=T, step=call, device=gpu)
        outs = []
        for run in ("forward", "noalloc"):
            so = torch.full((T, d), float("nan"), device=gpu)
            ro = torch.full((T, d), float("nan"), device=gpu)
            sel = torch.full((T, k), -7, dtype=torch.int32, device=gpu)
            wt = torch.full((T, k), float("nan"), device=gpu)
            if run == "forward":
                lay.forward(w, x, so, ro, sel, wt)
            else:
                dsmoe.forward_noalloc(cfg, w, x, so, ro, sel, wt)
            torch.cuda.synchronize()
            outs.append([_bits(t) for t in (so, ro, sel, wt)])
        for a, b in zip(*outs):
            assert np.array_equal(a, b), f"{name} call {call}: noalloc differs from forward"
    lay.close()


def test_noalloc_rejects_more_than_8_tokens(gpu):
    import torch
    case = C.CASES["c1"]
    cfg = case.cfg
    w = C.make_weights(case, device=gpu)
    x = C.make_x(case, T=9, device=gpu)
    so = torch.empty(9, cfg.d_model, device=gpu)
    ro = torch.empty(9, cfg.d_model, device=gpu)
    c, wc = cfg.c(), w.c()
    rc = dsmoe.lib().dsmoe_forward_noalloc(ctypes.byref(c), ctypes.byref(wc), dsmoe._p(x), 9, dsmoe._p(so),
                                           dsmoe._p(ro), None, None, None)
    assert rc == 2  # DSMOE_ERR_UNSUPPORTED
    assert b"T must be in 0..8" in dsmoe.lib().dsmoe_last_error()


def test_noalloc_under_graph_capture(gpu):
    """dsmoe_forward_noalloc captured into a HIP graph after the device's
    set-up (an eager call), replayed several times with eager work and
    synchronizations between the replays: every replay gives the eager
    call's bits."""
    import torch
    case = C.CASES["c1"]
    cfg = case.cfg
    d, k, T = cfg.d_model, cfg.top_k, 2
    say(f"noalloc graph capture c1 T={T}")
    w = C.make_weights(case, device=gpu)
    x = C.make_x(case, T=T, device=gpu)
    so, ro = torch.empty(T, d, device=gpu), torch.empty(T, d, device=gpu)
    sel = torch.empty(T, k, dtype=torch.int32, device=gpu)
    wt = torch.empty(T, k, device=gpu)
    dsmoe.forward_noalloc(cfg, w, x, so, ro, sel, wt)  # set-up happens here, outside capture
    torch.cuda.synchronize()
    want = [_bits(t).copy() for t in (so, ro, sel, wt)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        dsmoe.forward_noalloc(cfg, w, x, so, ro, sel, wt, stream=s)
    torch.cuda.synchronize()
    for rep in range(3):
        for t in (so, ro, wt):
            t.fill_(float("nan"))
        sel.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(want, [_bits(t) for t in (so, ro, sel, wt)]):
            assert np.array_equal(a, b), f"replay {rep} differs from the eager call"
        dsmoe.forward_noalloc(cfg, w, C.make_x(case, T=T, step=rep + 1, device=gpu), torch.empty_like(so),
                              torch.empty_like(ro), torch.empty_like(sel), torch.empty_like(wt))
        torch.cuda.synchronize()
    del g
