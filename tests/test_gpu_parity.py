"""GPU parity: every HIP entry point against the CPU oracle on the same
seeded inputs, through the C ABI.

Integer and index work (routing, Q8_K/Q8_0 codes, dispatch) must match
bit for bit.  Float outputs are required to agree within relative L2 1e-3
(the north-star tolerance at f32 accumulation); because the kernels sum in
the reference's order with the same f32 operations, they are also expected
to be bit-identical, and the tests report the exact-match fraction."""
import os
import sys

import numpy as np
import pytest

import dsmoe
from dsmoe import configs as C
import oracle_ref as O

pytestmark = pytest.mark.gpu
NT = min(16, os.cpu_count() or 1)
REL_L2 = 1e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    n = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (n if n > 0 else 1.0))


def assert_close(got, want, what):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, what
    r = rel_l2(got, want)
    exact = float(np.mean(got.view(np.uint32) == want.view(np.uint32)))
    say(f"  {what}: rel_l2={r:.3e} exact={exact:.4f}")
    assert np.isfinite(got).all() == np.isfinite(want).all()
    assert r <= REL_L2, (what, r)
    return exact


def bits_equal(a, b):
    return np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


def np_(t):
    return t.detach().cpu().numpy()


# ------------------------------------------------------------------ synth
def test_synth_device_equals_host(gpu):
    import torch
    say("synth device vs host")
    for fmt, rows, cols, rr, cr in [(dsmoe.FMT_IQ2_XXS, 24, 1024, 20, 1024), (dsmoe.FMT_Q2_K, 16, 512, 16, 400),
                                    (dsmoe.FMT_Q8_0, 8, 256, 8, 256), (dsmoe.FMT_F16, 4, 512, 4, 512),
                                    (dsmoe.FMT_F32, 3, 300, 3, 300)]:
        h = dsmoe.synth(fmt, 5, 11, 2, rows, cols, rr, cr, sigma=0.02, device="cpu")
        d = dsmoe.synth(fmt, 5, 11, 2, rows, cols, rr, cr, sigma=0.02, device=gpu)
        torch.cuda.synchronize()
        assert bits_equal(np_(d), h.numpy()), fmt


# ------------------------------------------------------------------ router
@pytest.mark.parametrize("E,d,T", [(256, 7168, 5), (64, 2048, 1), (256, 7168, 33), (20, 2048, 50), (24, 1280, 17), (22, 1280, 3),
                                   (256, 7168, 300), (30, 2048, 1030)])
def test_router_logits_bitexact(gpu, E, d, T):
    import torch
    say(f"router_logits E={E} d={d} T={T}")
    w = dsmoe.synth(dsmoe.FMT_F16, 1, 1, 1, E, d, sigma=0.02, device=gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 1, 2, 1, T, d, sigma=1.0, device=gpu)
    out = torch.empty(T, E, device=gpu)
    dsmoe.router_logits(w, x, out, d, E, T)
    want = O.router_logits(np_(w).view(np.uint16).copy(), np_(x), d, E, T, NT)
    assert bits_equal(np_(out), want)


@pytest.mark.parametrize("T", [3, 40, 1030])
def test_router_logits_special_weights_bitexact(gpu, T):
    """Router weights over the whole finite f16 range with many subnormals
    (flushed to signed zeros by the reference's conversion) and signed zeros,
    per-row (T <= 8) and tiled (T > 8) kernels."""
    import torch
    E, d = 24, 2048
    say(f"router_logits special weights T={T}")
    rng = np.random.default_rng(11)
    h = rng.integers(0, 0x7C00, size=(E, d), dtype=np.uint16)
    u = rng.random((E, d))
    h[u < 0.25] = rng.integers(1, 0x0400, size=int((u < 0.25).sum()), dtype=np.uint16)  # subnormal
    h[(u >= 0.25) & (u < 0.3)] = 0
    h |= (rng.random((E, d)) < 0.5).astype(np.uint16) << 15
    w = torch.from_numpy(h.view(np.int16).copy()).to(gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 1, 2, 1, T, d, sigma=1.0, device=gpu)
    out = torch.empty(T, E, device=gpu)
    dsmoe.router_logits(w, x, out, d, E, T)
    want = O.router_logits(h.reshape(-1).copy(), np_(x), d, E, T, NT)
    assert bits_equal(np_(out), want)


@pytest.mark.parametrize("T", [24, 256])
def test_router_logits_every_finite_f16_weight(gpu, T):
    """Every finite f16 bit pattern once as a router weight (E = d = 256: the
    65,536 patterns, Inf and NaN replaced by zeros), so every subnormal, both
    zeros and every normal value pass through the tiled kernels' widening;
    T = 24 runs the small tiles, T = 256 the large ones."""
    import torch
    E = d = 256
    say(f"router_logits every f16 weight T={T}")
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h[(h & 0x7C00) == 0x7C00] = 0
    h = h.reshape(E, d)
    w = torch.from_numpy(h.view(np.int16).copy()).to(gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 1, 3, 1, T, d, sigma=1.0, device=gpu)
    out = torch.empty(T, E, device=gpu)
    dsmoe.router_logits(w, x, out, d, E, T)
    want = O.router_logits(h.reshape(-1).copy(), np_(x), d, E, T, NT)
    assert bits_equal(np_(out), want)


@pytest.mark.parametrize("E,k,ng,tg,bias,scale", [(256, 6, 1, 1, False, 1.5), (64, 6, 1, 1, True, 1.5),
                                                  (256, 8, 8, 4, True, 2.5), (256, 8, 8, 4, False, 2.5),
                                                  (16, 3, 4, 2, True, 1.0)])
def test_router_select_bitexact(gpu, E, k, ng, tg, bias, scale):
    import torch
    say(f"router_select E={E} k={k} groups={ng}/{tg} bias={bias}")
    rng = np.random.default_rng(E + k)
    T = 300
    logits = rng.normal(0, 2, (T, E)).astype(np.float32)
    logits[0] = 0.5
    logits[1, ::3] = 1.25
    logits[2, 5] = np.nan
    logits[3] = -40.0
    b = rng.normal(0, 0.01, E).astype(np.float32) if bias else None
    cfg = dsmoe.MoeConfig(d_model=512, d_ff=256, n_expert=E, top_k=k, n_group=ng, topk_group=tg,
                          route_scale=scale, has_bias=bias, shared_fmt=-1)
    dl = torch.from_numpy(logits).to(gpu)
    db = torch.from_numpy(b).to(gpu) if bias else None
    probs = torch.empty(T, E, device=gpu)
    sel = torch.empty(T, k, dtype=torch.int32, device=gpu)
    w = torch.empty(T, k, device=gpu)
    dsmoe.router_select(cfg, dl, db, T, probs, sel, w)
    p0, s0, w0 = O.router_select(cfg, logits, b, T)
    assert np.array_equal(np_(sel), s0)
    assert bits_equal(np_(w), w0)
    assert bits_equal(np_(probs)[~np.isnan(p0)], p0[~np.isnan(p0)])


# ------------------------------------------------------------------ activation quantizers
def test_q8k_and_q8_0_bitexact(gpu):
    import torch
    say("q8k / q8_0 quantize")
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (37, 7168)).astype(np.float32)
    x[1, :256] = 0
    x[2, :256] = -0.0
    x[3, 1], x[3, 2] = -5.0, 5.0
    x[4, :] = 1e-30
    dx = torch.from_numpy(x).to(gpu)
    out = torch.empty(37 * 28 * 292, dtype=torch.uint8, device=gpu)
    dsmoe.q8k_quantize(dx, out, 7168, 37)
    assert bits_equal(np_(out), O.q8k_quantize(x, 7168, 37))
    xq = torch.empty(37 * 7168, dtype=torch.int8, device=gpu)
    xs = torch.empty(37 * 224, device=gpu)
    dsmoe.q8_0_quantize(dx, xq, xs, 7168, 37)
    q0, s0 = O.q8_0_quantize(x, 7168, 37)
    assert np.array_equal(np_(xq), q0) and bits_equal(np_(xs), s0)


# ------------------------------------------------------------------ expert kernels
def _routing(rng, T, k, E):
    sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    sel[0, -1] = -1  # unfilled slot -> expert 0 (moe.rs:640-643)
    w = rng.uniform(0.1, 0.5, (T, k)).astype(np.float32)
    return sel, w


@pytest.mark.parametrize("d,I,E,T,k", [(2048, 1536, 8, 2, 3), (7168, 2048, 4, 1, 3), (1024, 512, 3, 5, 2),
                                       (1536, 512, 12, 2, 10)])
def test_gate_up_down_bitexact(gpu, d, I, E, T, k):
    import torch
    say(f"gate_up/down d={d} I={I} E={E} T={T} k={k}")
    gate = dsmoe.synth(dsmoe.FMT_IQ2_XXS, 2, 1, E, I, d, sigma=0.02, device=gpu)
    up = dsmoe.synth(dsmoe.FMT_IQ2_XXS, 2, 2, E, I, d, sigma=0.02, device=gpu)
    dn = dsmoe.synth(dsmoe.FMT_Q2_K, 2, 3, E, d, I, sigma=0.02, device=gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 2, 4, 1, T, d, sigma=1.0, device=gpu)
    rng = np.random.default_rng(d + T)
    sel, w = _routing(rng, T, k, E)
    dsel = torch.from_numpy(sel.reshape(-1)).to(gpu)
    dw = torch.from_numpy(w.reshape(-1)).to(gpu)
    xq = torch.empty(T * (d // 256) * 292, dtype=torch.uint8, device=gpu)
    dsmoe.q8k_quantize(x, xq, d, T)
    P_ = T * k
    g = torch.empty(P_, I, device=gpu)
    u = torch.empty(P_, I, device=gpu)
    m = torch.empty(P_, I, device=gpu)
    dsmoe.gate_up_mid(gate, up, xq, dsel, dw, g, u, m, d, I, T, k, E, 10.0)
    mq = torch.empty(P_ * (I // 256) * 292, dtype=torch.uint8, device=gpu)
    dsmoe.q8k_quantize(m, mq, I, P_)
    dd = torch.empty(P_, d, device=gpu)
    ro = torch.empty(T, d, device=gpu)
    dsmoe.down(dn, mq, dsel, dd, ro, d, I, T, k, E)
    ro2 = torch.empty(T, d, device=gpu)
    dsmoe.moe_sum(dd, ro2, d, k, T)
    torch.cuda.synchronize()

    L = O.load()
    xq_h = np_(xq)
    g0, u0, m0 = (np.zeros(P_ * I, np.float32) for _ in range(3))
    gate_h, up_h, dn_h = np_(gate), np_(up), np_(dn)
    L.or_gate_up_mid(O.P(gate_h), O.P(up_h), O.P(xq_h), O.P(sel.reshape(-1).copy()), O.P(w.reshape(-1).copy()),
                     O.P(g0), O.P(u0), O.P(m0), d, I, T, k, 10.0, NT)
    assert bits_equal(xq_h, O.q8k_quantize(np_(x), d, T))
    assert_close(np_(g).reshape(-1), g0, "gate")
    assert_close(np_(u).reshape(-1), u0, "up")
    assert_close(np_(m).reshape(-1), m0, "mid")
    mq_h = np_(mq)
    assert bits_equal(mq_h, O.q8k_quantize(np_(m), I, P_))
    d0 = np.zeros(P_ * d, np.float32)
    L.or_down(O.P(dn_h), O.P(mq_h), O.P(sel.reshape(-1).copy()), O.P(d0), d, I, T, k, NT)
    assert_close(np_(dd).reshape(-1), d0, "down per pair")
    s0 = np.zeros(T * d, np.float32)
    L.or_moe_sum(O.P(d0), O.P(s0), d, k, T)
    assert_close(np_(ro).reshape(-1), s0, "down slot sum")
    assert bits_equal(np_(ro2), np_(ro))


@pytest.mark.parametrize("d,I,E,T,k", [(7168, 2048, 8, 3, 8), (2048, 1024, 6, 2, 4), (1024, 4096, 12, 1, 10)])
def test_expert_ids_outside_range_read_expert_0(gpu, d, I, E, T, k):
    """gate_up_mid / down with ids -1, E, E + 5 and 2^31 - 1 in `selected`:
    those slots read expert 0 (the weights hold exactly E experts, so an
    unclamped id would read past the allocation) and give the bits of the
    same call with 0 in their place."""
    import torch
    say(f"ids outside [0,E) d={d} I={I} E={E} T={T} k={k}")
    gate = dsmoe.synth(dsmoe.FMT_IQ2_XXS, 3, 1, E, I, d, sigma=0.02, device=gpu)
    up = dsmoe.synth(dsmoe.FMT_IQ2_XXS, 3, 2, E, I, d, sigma=0.02, device=gpu)
    dn = dsmoe.synth(dsmoe.FMT_Q2_K, 3, 3, E, d, I, sigma=0.02, device=gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 3, 4, 1, T, d, sigma=1.0, device=gpu)
    rng = np.random.default_rng(E * 7 + T)
    sel = rng.integers(0, E, size=(T, k)).astype(np.int32)
    bad = np.array([-1, E, E + 5, 2**31 - 1], np.int32)
    pos = rng.choice(T * k, size=min(T * k, 6), replace=False)
    sel.reshape(-1)[pos] = bad[np.arange(len(pos)) % 4]
    fixed = np.where((sel < 0) | (sel >= E), 0, sel).astype(np.int32)
    w = rng.random((T, k), dtype=np.float32)
    xq = torch.empty(T * (d // 256) * 292, dtype=torch.uint8, device=gpu)
    dsmoe.q8k_quantize(x, xq, d, T)
    dw = torch.from_numpy(w.reshape(-1)).to(gpu)
    outs = []
    for s in (sel, fixed):
        dsel = torch.from_numpy(s.reshape(-1).copy()).to(gpu)
        m = torch.empty(T * k, I, device=gpu)
        dsmoe.gate_up_mid(gate, up, xq, dsel, dw, None, None, m, d, I, T, k, E, 10.0)
        mq = torch.empty(T * k * (I // 256) * 292, dtype=torch.uint8, device=gpu)
        dsmoe.q8k_quantize(m, mq, I, T * k)
        dd = torch.empty(T * k, d, device=gpu)
        ro = torch.empty(T, d, device=gpu)
        dsmoe.down(dn, mq, dsel, dd, ro, d, I, T, k, E)
        torch.cuda.synchronize()
        outs.append([np_(m), np_(dd), np_(ro)])
    for a, b in zip(*outs):
        assert bits_equal(a, b)


def _iq2_big_blocks(rng, n_blocks):
    """IQ2_XXS blocks with random codes and every sub-block scale at its
    maximum (ls = 31): superblock sums beyond the f32-exact range (2^24) of
    the grouped MFMA accumulation."""
    b = rng.integers(0, 256, size=(n_blocks, 66), dtype=np.uint8)
    b[:, 0], b[:, 1] = 0x00, 0x2C  # d = 0.0625
    for j in range(8):
        b[:, 2 + 8 * j + 7] |= 0xF0
    return b.reshape(-1)


@pytest.mark.parametrize("d,I,E,T,k,skew,big", [(7168, 2048, 16, 200, 8, True, False),
                                                (2048, 1536, 8, 70, 6, False, False),
                                                (1024, 512, 3, 33, 2, True, True),
                                                (2048, 512, 5, 40, 3, False, True)])
def test_gate_up_sorted_matches_per_pair(gpu, d, I, E, T, k, skew, big):
    """The grouped MFMA gate/up (pairs sorted by expert, tiles of 64) against
    the per-pair kernel, which the oracle pins bit for bit.  Its superblock
    sums are the reference's integers, but it adds the superblocks of a row
    in order 0, 1, 2, ... where the reference adds per-lane partials and a
    butterfly: the two differ by f32 rounding of that order, bounded here at
    rel-L2 1e-5 and 1e-4 of the row scale per element (north_star allows
    1e-3).  The grouped down the same way against the per-pair down."""
    import torch
    say(f"gate_up sorted d={d} I={I} E={E} T={T} k={k} skew={skew} big={big}")
    rng = np.random.default_rng(d + I + T)
    if big:
        gate = torch.from_numpy(_iq2_big_blocks(rng, E * I * (d // 256))).to(gpu)
        up = torch.from_numpy(_iq2_big_blocks(rng, E * I * (d // 256))).to(gpu)
    else:
        gate = dsmoe.synth(dsmoe.FMT_IQ2_XXS, 3, 1, E, I, d, sigma=0.02, device=gpu)
        up = dsmoe.synth(dsmoe.FMT_IQ2_XXS, 3, 2, E, I, d, sigma=0.02, device=gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 3, 4, 1, T, d, sigma=1.0, device=gpu)
    if skew:  # a few hot experts with several tiles, some experts unused
        p = np.array([0.5 ** i for i in range(E)])
        p /= p.sum()
        sel = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    else:
        sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.1, 0.5, (T, k)).astype(np.float32)
    P_ = T * k
    dsel = torch.from_numpy(sel.reshape(-1)).to(gpu)
    dw = torch.from_numpy(w.reshape(-1)).to(gpu)
    xq = torch.empty(T * (d // 256) * 292, dtype=torch.uint8, device=gpu)
    xh = torch.empty(T, d, dtype=torch.int16, device=gpu)
    dsmoe.q8k_quantize_h(x, xq, xh, d, T)
    m_ref = torch.empty(P_, I, device=gpu)
    g_ = torch.empty(P_, I, device=gpu)
    u_ = torch.empty(P_, I, device=gpu)
    dsmoe.gate_up_mid(gate, up, xq, dsel, dw, g_, u_, m_ref, d, I, T, k, E, 10.0)
    u32 = dict(dtype=torch.int32, device=gpu)
    counts, offsets = torch.empty(E, **u32), torch.empty(E + 1, **u32)
    sp = torch.empty(P_, **u32)
    max_tiles = P_ // dsmoe.GROUPED_TILE_M + min(E, P_)
    toff, texp, tst = torch.empty(E + 1, **u32), torch.empty(max_tiles, **u32), torch.empty(max_tiles, **u32)
    dsmoe.dispatch(dsel, P_, E, dsmoe.GROUPED_TILE_M, counts, offsets, sp, toff, texp, tst)
    m = torch.full((P_, I), float("nan"), device=gpu)
    dsmoe.gate_up_mid_sorted(gate, up, xh, xq, sp, offsets, toff, texp, tst, dw, m, d, I, k, E, P_, 10.0)
    torch.cuda.synchronize()
    xh_h = np_(xh).view(np.float16).astype(np.float32)
    q_h = O.q8k_quantize(np_(x), d, T).reshape(T, d // 256, 292)[:, :, 4:260].view(np.int8).reshape(T, d)
    assert np.array_equal(xh_h, q_h.astype(np.float32))
    say(f"  tiles={int(np_(toff)[-1])} max_count={int(np_(counts).max())}")
    # tiles of at most 32 pairs run their own loop copy (no products for pairs 32-63)
    fills = [min(64, int(c) - 64 * i) for c in np_(counts) for i in range((int(c) + 63) // 64)]
    say(f"  tiles with <= 32 pairs: {sum(f <= 32 for f in fills)}, with more: {sum(f > 32 for f in fills)}")
    if skew and not big:
        assert any(f <= 32 for f in fills) and any(f > 32 for f in fills)
    got, want = np_(m).astype(np.float64), np_(m_ref).astype(np.float64)
    assert np.isfinite(got).all()
    r = rel_l2(got, want)
    elem = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    say(f"  mid sorted vs per-pair: rel_l2={r:.3e} max_abs/row_scale={elem:.3e}")
    assert r <= 1e-5 and elem <= 1e-4, (r, elem)
    # down on the same pairs: grouped MFMA vs the per-pair kernel
    dn = dsmoe.synth(dsmoe.FMT_Q2_K, 3, 3, E, d, I, sigma=0.02, device=gpu)
    mq = torch.empty(P_ * (I // 256) * 292, dtype=torch.uint8, device=gpu)
    m8 = torch.empty(P_, I, dtype=torch.int8, device=gpu)
    bsh = torch.empty(P_, I // 16, dtype=torch.int16, device=gpu)
    dsmoe.q8k_quantize_i8(m_ref, mq, m8, bsh, I, P_)
    dd_ref = torch.empty(P_, d, device=gpu)
    ro = torch.empty(T, d, device=gpu)
    dsmoe.down(dn, mq, dsel, dd_ref, ro, d, I, T, k, E)
    dd = torch.full((P_, d), float("nan"), device=gpu)
    dsmoe.down_sorted(dn, m8, bsh, mq, sp, offsets, toff, texp, tst, dd, d, I, E, P_)
    torch.cuda.synchronize()
    # the int8 codes and f16 group sums are the Q8_K block's qs and bsums
    blk = np_(mq).reshape(P_, I // 256, 292)
    assert np.array_equal(np_(m8).reshape(P_, I), blk[:, :, 4:260].copy().view(np.int8).reshape(P_, I))
    bs16 = blk[:, :, 260:292].copy().view(np.int16).reshape(P_, I // 16)
    assert np.array_equal(np_(bsh).view(np.float16).astype(np.float32), bs16.astype(np.float32))
    got, want = np_(dd).astype(np.float64), np_(dd_ref).astype(np.float64)
    assert np.isfinite(got).all()
    r = rel_l2(got, want)
    elem = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    say(f"  down sorted vs per-pair: rel_l2={r:.3e} max_abs/row_scale={elem:.3e}")
    assert r <= 1e-5 and elem <= 1e-4, (r, elem)


@pytest.mark.parametrize("d,I,E,T,k,skew,bm", [(7168, 2048, 16, 40, 8, True, 8), (7168, 2048, 256, 32, 8, False, 2),
                                                (7168, 2048, 64, 32, 8, True, 4), (2048, 1536, 8, 5, 3, False, 8),
                                                (1024, 512, 3, 9, 2, True, 3)])
def test_expert_major_matches_per_pair(gpu, d, I, E, T, k, skew, bm):
    """The expert-major gate/up and down (pairs dispatched in tiles of 8, each
    expert's rows streamed once per tile) must give the per-pair kernels'
    bits: hot experts with several tiles, cold ones with one pair."""
    import torch
    say(f"expert-major d={d} I={I} E={E} T={T} k={k} skew={skew} block_m={bm}")
    rng = np.random.default_rng(d + I + T + 1)
    gate = dsmoe.synth(dsmoe.FMT_IQ2_XXS, 4, 1, E, I, d, sigma=0.02, device=gpu)
    up = dsmoe.synth(dsmoe.FMT_IQ2_XXS, 4, 2, E, I, d, sigma=0.02, device=gpu)
    dn = dsmoe.synth(dsmoe.FMT_Q2_K, 4, 3, E, d, I, sigma=0.02, device=gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 4, 4, 1, T, d, sigma=1.0, device=gpu)
    if skew:
        p = np.array([0.5 ** i for i in range(E)])
        p /= p.sum()
        sel = np.stack([rng.choice(E, k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    else:
        sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.1, 0.5, (T, k)).astype(np.float32)
    P_ = T * k
    dsel = torch.from_numpy(sel.reshape(-1)).to(gpu)
    dw = torch.from_numpy(w.reshape(-1)).to(gpu)
    xq = torch.empty(T * (d // 256) * 292, dtype=torch.uint8, device=gpu)
    dsmoe.q8k_quantize(x, xq, d, T)
    m_ref = torch.empty(P_, I, device=gpu)
    dsmoe.gate_up_mid(gate, up, xq, dsel, dw, None, None, m_ref, d, I, T, k, E, 10.0)
    u32 = dict(dtype=torch.int32, device=gpu)
    counts, offsets = torch.empty(E, **u32), torch.empty(E + 1, **u32)
    sp = torch.empty(P_, **u32)
    max_tiles = P_ // bm + min(E, P_)
    toff, texp, tst = torch.empty(E + 1, **u32), torch.empty(max_tiles, **u32), torch.empty(max_tiles, **u32)
    dsmoe.dispatch(dsel, P_, E, bm, counts, offsets, sp, toff, texp, tst)
    m = torch.full((P_, I), float("nan"), device=gpu)
    dsmoe.gate_up_mid_em(gate, up, xq, sp, offsets, toff, texp, tst, dw, m, d, I, k, E, P_, 10.0, bm)
    torch.cuda.synchronize()
    say(f"  tiles={int(np_(toff)[-1])} max_count={int(np_(counts).max())}")
    assert_close(np_(m).reshape(-1), np_(m_ref).reshape(-1), "mid expert-major vs per-pair")
    assert bits_equal(np_(m), np_(m_ref))
    mq = torch.empty(P_ * (I // 256) * 292, dtype=torch.uint8, device=gpu)
    dsmoe.q8k_quantize(m_ref, mq, I, P_)
    dd_ref = torch.empty(P_, d, device=gpu)
    dsmoe.down(dn, mq, dsel, dd_ref, None, d, I, T, k, E)
    dd = torch.full((P_, d), float("nan"), device=gpu)
    dsmoe.down_em(dn, mq, sp, offsets, toff, texp, tst, dd, d, I, E, P_, bm)
    torch.cuda.synchronize()
    assert_close(np_(dd).reshape(-1), np_(dd_ref).reshape(-1), "down expert-major vs per-pair")
    assert bits_equal(np_(dd), np_(dd_ref))


@pytest.mark.parametrize("din,dout,T", [(7168, 2048, 130), (2048, 1408, 64), (1408, 2048, 9), (2048, 7168, 70),
                                         (4096, 1024, 33)])
def test_q8_0_gemm_matches_matvec(gpu, din, dout, T):
    """The batch GEMM of the shared expert (matrix cores) against the per-token
    Q8_0 matvec and SwiGLU, which the oracle pins: same bits."""
    import torch
    say(f"q8_0 gemm din={din} dout={dout} T={T}")
    w0 = dsmoe.synth(dsmoe.FMT_Q8_0, 5, 1, 1, dout, din, sigma=0.02, device=gpu)
    w1 = dsmoe.synth(dsmoe.FMT_Q8_0, 5, 2, 1, dout, din, sigma=0.02, device=gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 5, 3, 1, T, din, sigma=1.0, device=gpu)
    xq = torch.empty(T * din, dtype=torch.int8, device=gpu)
    xs = torch.empty(T * (din // 32), device=gpu)
    xh = torch.empty(T, din, dtype=torch.int16, device=gpu)
    dsmoe.q8_0_quantize_h(x, xq, xs, xh, din, T)
    g = torch.empty(T, dout, device=gpu)
    u = torch.empty(T, dout, device=gpu)
    dsmoe.q8_0_matvec(w0, xq, xs, g, din, dout, T)
    dsmoe.q8_0_matvec(w1, xq, xs, u, din, dout, T)
    mid_ref = torch.empty(T, dout, device=gpu)
    dsmoe.swiglu(g, u, mid_ref, T * dout, 10.0, 1.0)
    out1 = torch.full((T, dout), float("nan"), device=gpu)
    mid = torch.full((T, dout), float("nan"), device=gpu)
    if dout % 64 == 0:
        dsmoe.q8_0_gemm(w0, None, xh, xs, out1, din, dout, T)
    dsmoe.q8_0_gemm(w0, w1, xh, xs, mid, din, dout, T, 10.0)
    torch.cuda.synchronize()
    q_ref = np_(xq).astype(np.float32)
    assert np.array_equal(np_(xh).view(np.float16).astype(np.float32).reshape(-1), q_ref)
    if dout % 64 == 0:
        assert_close(np_(out1).reshape(-1), np_(g).reshape(-1), "q8_0 gemm vs matvec")
        assert bits_equal(np_(out1), np_(g))
    assert_close(np_(mid).reshape(-1), np_(mid_ref).reshape(-1), "q8_0 gemm swiglu vs matvec + swiglu")
    assert bits_equal(np_(mid), np_(mid_ref))


@pytest.mark.parametrize("din,dout,T", [(7168, 2048, 1100), (2048, 7168, 1030), (2048, 1408, 300),
                                         (4096, 1024, 257), (1408, 2048, 3)])
def test_q8_0_gemm_unpacked(gpu, din, dout, T):
    """The unpacked layout against a numpy restatement (same bits), and the
    unpacked GEMM (blocks added in order) against dsmoe_q8_0_gemm, the
    reference's sum order, which the matvec test above pins: 1e-5 relative
    L2 and 1e-4 of the largest magnitude per element."""
    import torch
    say(f"q8_0 gemm unpacked din={din} dout={dout} T={T}")
    nb = din // 32
    w0 = dsmoe.synth(dsmoe.FMT_Q8_0, 6, 1, 1, dout, din, sigma=0.02, device=gpu)
    w1 = dsmoe.synth(dsmoe.FMT_Q8_0, 6, 2, 1, dout, din, sigma=0.02, device=gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 6, 3, 1, T, din, sigma=1.0, device=gpu)
    xq = torch.empty(T * din, dtype=torch.int8, device=gpu)
    xs = torch.empty(T * nb, device=gpu)
    xh = torch.empty(T, din, dtype=torch.int16, device=gpu)
    dsmoe.q8_0_quantize_h(x, xq, xs, xh, din, T)
    hs = [torch.empty(dout * din, dtype=torch.int16, device=gpu) for _ in range(2)]
    ss = [torch.empty(dout * nb, device=gpu) for _ in range(2)]
    dsmoe.q8_0_unpack(w0, dout, din, hs[0], ss[0])
    dsmoe.q8_0_unpack(w1, dout, din, hs[1], ss[1])
    mid = torch.full((T, dout), float("nan"), device=gpu)
    mid_ref = torch.full((T, dout), float("nan"), device=gpu)
    dsmoe.q8_0_gemm_unpacked(hs[0], ss[0], hs[1], ss[1], xh, xs, mid, din, dout, T, 10.0)
    dsmoe.q8_0_gemm(w0, w1, xh, xs, mid_ref, din, dout, T, 10.0)
    one = dout % 128 == 0
    if one:
        out = torch.full((T, dout), float("nan"), device=gpu)
        out_ref = torch.full((T, dout), float("nan"), device=gpu)
        dsmoe.q8_0_gemm_unpacked(hs[0], ss[0], None, None, xh, xs, out, din, dout, T)
        dsmoe.q8_0_gemm(w0, None, xh, xs, out_ref, din, dout, T)
    torch.cuda.synchronize()
    # layout: codes [rows / 16][nb][lane 16 q + r][8] = row 16 R + r, codes 8 q .. +7 of the block
    raw = np_(w0).reshape(dout, nb, 34)
    codes = raw[:, :, 2:].copy().view(np.int8).astype(np.float16)
    want = codes.reshape(dout // 16, 16, nb, 4, 8).transpose(0, 2, 3, 1, 4).reshape(-1)
    assert bits_equal(np_(hs[0]).view(np.float16), want)
    sc = raw[:, :, :2].copy().view(np.float16).reshape(dout, nb).astype(np.float32)
    # the reference's f16 conversion flushes subnormal scales to zero (sign kept)
    sc = np.where(np.abs(sc) < 2.0 ** -14, np.copysign(np.float32(0.0), sc), sc).astype(np.float32)
    assert bits_equal(np_(ss[0]), sc.reshape(dout // 16, 16, nb).transpose(0, 2, 1).reshape(-1))

    def close(got, ref, what):
        r = rel_l2(got, ref)
        err = float(np.abs(got - ref).max() / np.abs(ref).max())
        say(f"  {what}: rel_l2={r:.3e} max_err/max={err:.3e}")
        assert r <= 1e-5 and err <= 1e-4, (what, r, err)
    close(np_(mid), np_(mid_ref), "swiglu(gate, up)")
    if one:
        close(np_(out), np_(out_ref), "one matrix")


def test_q8_0_matvec_and_swiglu_bitexact(gpu):
    import torch
    say("q8_0 matvec + swiglu")
    d, Is, T = 7168, 1408, 3
    w = dsmoe.synth(dsmoe.FMT_Q8_0, 4, 1, 1, Is, d, sigma=0.02, device=gpu)
    x = dsmoe.synth(dsmoe.FMT_F32, 4, 2, 1, T, d, sigma=1.0, device=gpu)
    xq = torch.empty(T * d, dtype=torch.int8, device=gpu)
    xs = torch.empty(T * (d // 32), device=gpu)
    dsmoe.q8_0_quantize(x, xq, xs, d, T)
    out = torch.empty(T, Is, device=gpu)
    dsmoe.q8_0_matvec(w, xq, xs, out, d, Is, T)
    o0 = np.zeros(T * Is, np.float32)
    O.load().or_q8_0_matvec(O.P(np_(w)), O.P(np_(xq)), O.P(np_(xs)), O.P(o0), d, Is, T, NT)
    assert_close(np_(out).reshape(-1), o0, "q8_0 matvec")
    rng = np.random.default_rng(9)
    gg = rng.normal(0, 8, 5000).astype(np.float32)
    uu = rng.normal(0, 8, 5000).astype(np.float32)
    res = torch.empty(5000, device=gpu)
    dsmoe.swiglu(torch.from_numpy(gg).to(gpu), torch.from_numpy(uu).to(gpu), res, 5000, 10.0, 0.7)
    r0 = np.zeros(5000, np.float32)
    O.load().or_swiglu(O.P(gg), O.P(uu), O.P(r0), 5000, 10.0, 0.7)
    assert bits_equal(np_(res), r0)


# ------------------------------------------------------------------ dispatch
@pytest.mark.parametrize("E,pairs,bm", [(256, 8, 16), (256, 16384, 32), (64, 777, 8), (256, 1024, 64), (16, 0, 4)])
def test_dispatch_bitexact(gpu, E, pairs, bm):
    import torch
    say(f"dispatch E={E} pairs={pairs} bm={bm}")
    rng = np.random.default_rng(pairs + E)
    sel = rng.integers(-1, E, pairs).astype(np.int32)
    if pairs > 100:
        sel[: pairs // 2] = 7  # a hot expert
    ds = torch.from_numpy(sel).to(gpu) if pairs else torch.zeros(1, dtype=torch.int32, device=gpu)
    cnt = torch.empty(E, dtype=torch.int32, device=gpu)
    off = torch.empty(E + 1, dtype=torch.int32, device=gpu)
    sp = torch.empty(max(pairs, 1), dtype=torch.int32, device=gpu)
    nt = pairs // bm + E + 1
    to = torch.empty(E + 1, dtype=torch.int32, device=gpu)
    te = torch.empty(nt, dtype=torch.int32, device=gpu)
    ts = torch.empty(nt, dtype=torch.int32, device=gpu)
    dsmoe.dispatch(ds, pairs, E, bm, cnt, off, sp, to, te, ts)
    c0, o0, s0, to0, te0, ts0 = O.dispatch(sel, E, bm)
    assert np.array_equal(np_(cnt).view(np.uint32), c0)
    assert np.array_equal(np_(off).view(np.uint32), o0)
    assert np.array_equal(np_(sp).view(np.uint32)[:pairs], s0)
    assert np.array_equal(np_(to).view(np.uint32), to0)
    n = int(to0[E])
    assert np.array_equal(np_(te).view(np.uint32)[:n], te0)
    assert np.array_equal(np_(ts).view(np.uint32)[:n], ts0)


# ------------------------------------------------------------------ whole layer
def _host_weights(w):
    f = lambda t: None if t is None else np_(t).reshape(-1).copy()
    return {"router": np_(w.router_f16).view(np.uint16).reshape(-1).copy(), "bias": f(w.bias), "gate": f(w.gate),
            "up": f(w.up), "down": f(w.down), "sh_gate": f(w.sh_gate), "sh_up": f(w.sh_up), "sh_down": f(w.sh_down)}


def _run_layer(case, T, gpu, sample=None):
    """`sample`: rows checked against the oracle (None = all), or a function
    of the GPU's routing [T][k] that picks them."""
    import torch
    say(f"layer {case.name} T={T}")
    w = C.make_weights(case, device=gpu)
    x = C.make_x(case, T=T, device=gpu)
    d, k = case.cfg.d_model, case.cfg.top_k
    layer = dsmoe.MoeLayer(case.cfg, T)
    so = torch.empty(T, d, device=gpu)
    ro = torch.empty(T, d, device=gpu)
    sel = torch.empty(T, k, dtype=torch.int32, device=gpu)
    wt = torch.empty(T, k, device=gpu)
    layer.forward(w, x, so, ro, sel, wt)
    torch.cuda.synchronize()
    hw = _host_weights(w)
    rows = np.arange(T) if sample is None else sample(np_(sel)) if callable(sample) else sample
    say(f"  oracle rows: {len(rows)}")
    xs = np_(x)[rows].copy()
    so0, ro0, sel0, wt0 = O.moe_forward(case.cfg, hw, xs, len(rows), NT)
    assert np.array_equal(np_(sel)[rows], sel0), "routing differs"
    assert bits_equal(np_(wt)[rows], wt0)
    e1 = assert_close(np_(ro)[rows], ro0, f"{case.name} routed_out")
    e2 = assert_close(np_(so)[rows], so0, f"{case.name} shared_out")
    # the same context again: the in-launch counters (mid quantization, slot
    # sum) must have reset themselves
    for rep in range(2):
        ro2 = torch.full((T, d), float("nan"), device=gpu)
        so2 = torch.full((T, d), float("nan"), device=gpu)
        layer.forward(w, x, so2, ro2, sel, wt)
        torch.cuda.synchronize()
        assert bits_equal(np_(ro2), np_(ro)) and bits_equal(np_(so2), np_(so)), f"call {rep + 2} differs"
    layer.close()
    return np_(sel), e1, e2


def test_layer_c1_small(gpu):
    _run_layer(C.CASES["c1"], 1, gpu)
    _run_layer(C.CASES["c1"], 7, gpu)


def test_layer_c2_full_decode(gpu):
    _run_layer(C.CASES["c2"], 1, gpu)


def test_layer_c3_batch32(gpu):
    sel, _, _ = _run_layer(C.CASES["c3"], 32, gpu)
    say(f"  distinct experts at T=32: {len(np.unique(sel))}")


def test_layer_c4_tie_routing(gpu):
    case = C.CASES["c4tie"]
    sel, _, _ = _run_layer(case, 128, gpu, sample=np.arange(0, 128, 9))
    # identical router rows: every token picks the same experts (bias decides)
    assert (sel == sel[0]).all()


def test_layer_c4_binomial(gpu):
    """128 tokens with N(0, 0.02) routers, so expert loads
    are roughly Binomial(128, 8/256); every second row against the oracle."""
    sel, _, _ = _run_layer(C.CASES["c4"], 128, gpu, sample=np.arange(0, 128, 2))
    counts = np.bincount(sel.reshape(-1), minlength=256)
    say(f"  c4 expert loads: max {counts.max()}, experts used {np.count_nonzero(counts)}")
    assert np.count_nonzero(counts) > 64


@pytest.mark.parametrize("T", [1, 128])
def test_layer_reference_config(gpu, T):
    """The reference's own layer shape and routing (d=4096, E=256, top-6, no
    groups, scale 1.5, no bias) at decode and at a 128-token batch."""
    _run_layer(C.with_tokens(C.CASES["ref"], T), T, gpu)


def _hot_and_cold_rows(sel, n=256, seed=5):
    """Rows holding the 16 coldest used experts and the hottest expert,
    topped up with random rows to n."""
    T = sel.shape[0]
    counts = np.bincount(sel.reshape(-1), minlength=256)
    used = np.flatnonzero(counts)
    cold = used[np.argsort(counts[used], kind="stable")[:16]]
    hot = int(np.argmax(counts))
    rows = set(np.flatnonzero(np.isin(sel, cold).any(1)).tolist())
    rows |= set(np.flatnonzero((sel == hot).any(1))[:64].tolist())
    rest = np.random.default_rng(seed).permutation(T)
    for r in rest:
        if len(rows) >= n:
            break
        rows.add(int(r))
    return np.array(sorted(rows))


def test_layer_c5_zipf_sampled(gpu):
    case = C.CASES["c5"]
    sel, _, _ = _run_layer(case, 2048, gpu, sample=_hot_and_cold_rows)
    counts = np.bincount(sel.reshape(-1), minlength=256)
    top10 = np.sort(counts)[::-1][:10].sum() / counts.sum()
    say(f"  top-10 expert share at T=2048 Zipf: {top10:.3f}")
    assert top10 > 0.5


def test_layer_c5logit_sampled(gpu):
    """c5 with the Zipf prior added to the router logits (BASELINE.json's
    wording) rather than the selection bias: flatter loads over most of the
    experts, so many partial MFMA tiles; sampled rows against the oracle."""
    case = C.CASES["c5logit"]
    sel, _, _ = _run_layer(case, 2048, gpu, sample=_hot_and_cold_rows)
    counts = np.bincount(sel.reshape(-1), minlength=256)
    say(f"  c5logit: experts used {np.count_nonzero(counts)}, top-10 share "
        f"{np.sort(counts)[::-1][:10].sum() / counts.sum():.3f}")
    assert np.count_nonzero(counts) > 64


@pytest.mark.parametrize("name,T", [("ref", 1100), ("c1", 1030)])
def test_layer_shared_expert_wide_gemm(gpu, name, T):
    """Batches of 1024 tokens and more run the shared expert through the
    unpacked wide GEMM (blocks added in order, not in the reference's lane
    tree): the layer's shared output against the oracle on rows of the full
    256-token tiles and of the partial last one, and the same result on a
    second call."""
    import torch
    case = C.with_tokens(C.CASES[name], T)
    say(f"shared wide gemm {name} T={T}")
    w = C.make_weights(case, device=gpu)
    x = C.make_x(case, T=T, device=gpu)
    d, k = case.cfg.d_model, case.cfg.top_k
    layer = dsmoe.MoeLayer(case.cfg, T)
    so = torch.empty(T, d, device=gpu)
    ro = torch.empty(T, d, device=gpu)
    sel = torch.empty(T, k, dtype=torch.int32, device=gpu)
    wt = torch.empty(T, k, device=gpu)
    layer.forward(w, x, so, ro, sel, wt)
    so2 = torch.full((T, d), float("nan"), device=gpu)
    layer.forward(w, x, so2, ro, sel, wt)
    # the same weights with the shared expert unpacked once (dsmoe_weights.sh_codes)
    so3 = torch.full((T, d), float("nan"), device=gpu)
    ro3 = torch.full((T, d), float("nan"), device=gpu)
    w.unpack_shared(case.cfg)
    layer.forward(w, x, so3, ro3, sel, wt)
    torch.cuda.synchronize()
    layer.close()
    assert bits_equal(np_(so2), np_(so)), "second call differs"
    assert bits_equal(np_(so3), np_(so)) and bits_equal(np_(ro3), np_(ro)), "pre-unpacked shared expert differs"
    rows = np.array(sorted(set(range(0, T, 37)) | {255, 256, 1023, 1024, T - 1}))
    so0, _, _, _ = O.moe_forward(case.cfg, _host_weights(w), np_(x)[rows].copy(), len(rows), NT)
    got = np_(so)[rows]
    r = rel_l2(got, so0)
    per_row = np.linalg.norm(got - so0, axis=1) / np.linalg.norm(so0, axis=1)
    say(f"  shared_out rows={len(rows)} rel_l2={r:.3e} median row {np.median(per_row):.3e} max row {per_row.max():.3e}")
    # the shared mid is quantized again (Q8_0) before the down matrix: where
    # f32 rounding moves a block's largest element across a rounding step the
    # block's codes change, so single rows differ by up to about one
    # quantization step; the rest agree to f32 rounding
    assert r <= REL_L2, r
    assert np.median(per_row) <= 1e-5, np.median(per_row)


def test_layer_shared_expert_side_stream_same_bits(gpu):
    """Batches on the wide path run the quantization of x and the shared
    expert on a second stream of the context, forked before the router and
    joined into the caller's stream at the end; with stage profiling on, the
    same forward runs every stage on the caller's stream.  Both orders give
    the same bits, on a non-default caller stream and on two calls in a row
    (the second one also checks the join: its outputs are read on the caller's
    stream right after the call)."""
    import torch
    T = 1280
    case = C.with_tokens(C.CASES["c5"], T)
    say(f"side stream c5 T={T}")
    w = C.make_weights(case, device=gpu)
    x = C.make_x(case, T=T, device=gpu)
    d, k = case.cfg.d_model, case.cfg.top_k
    layer = dsmoe.MoeLayer(case.cfg, T)
    s = torch.cuda.Stream()
    outs = []
    for profiling in (False, True, False):
        layer.set_profiling(profiling)
        so = torch.full((T, d), float("nan"), device=gpu)
        ro = torch.full((T, d), float("nan"), device=gpu)
        sel = torch.empty(T, k, dtype=torch.int32, device=gpu)
        wt = torch.empty(T, k, device=gpu)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            layer.forward(w, x, so, ro, sel, wt, stream=s)
            # read on the caller's stream: the join must order it after the shared chain
            got = (so.clone(), ro.clone(), sel.clone())
        s.synchronize()
        if profiling:
            layer.profile_read(reset=True)
        outs.append([np_(t) for t in got])
    layer.set_profiling(False)
    layer.close()
    assert not np.isnan(outs[0][0]).any() and not np.isnan(outs[0][1]).any()
    for o in outs[1:]:
        assert np.array_equal(o[2], outs[0][2]), "routing differs"
        assert bits_equal(o[0], outs[0][0]), "shared_out differs between the forked and the serial order"
        assert bits_equal(o[1], outs[0][1]), "routed_out differs between the forked and the serial order"


def test_layer_many_experts_batch_on_the_row_path(gpu):
    """n_expert above the dispatch limit (576 > 512, 9 groups of 64): a
    context for 12 tokens has no grouped buffers, so the batch runs the
    row-streaming launches with T > 8 (no in-launch counters, selection in
    every routed workgroup); routing and outputs against the oracle, twice
    on the same context."""
    import dataclasses
    base = C.CASES["c1"]
    cfg = dataclasses.replace(base.cfg, d_model=1024, d_ff=512, n_expert=576, top_k=6, n_group=9, topk_group=4,
                              d_ff_shared=512)
    case = dataclasses.replace(base, name="e576", cfg=cfg, T=12, d_ff_real=512, d_ff_shared_real=512)
    _run_layer(case, 12, gpu)


@pytest.mark.parametrize("name,Ts", [("c1", [1, 3, 8, 5]), ("c2", [1, 2, 8])])
def test_decode_calls_in_a_row(gpu, name, Ts):
    """One context, decode calls of varying T in a row: every call matches the
    oracle (the completion counters of the selection and of the mid
    quantization reset themselves between launches)."""
    import torch
    case = C.CASES[name]
    w = C.make_weights(case, device=gpu)
    hw = _host_weights(w)
    d, k = case.cfg.d_model, case.cfg.top_k
    lay = dsmoe.MoeLayer(case.cfg, 8)
    for rep, T in enumerate(Ts * 2):
        say(f"decode calls {name} T={T} rep={rep}")
        x = C.make_x(case, T=T, step=rep, device=gpu)
        so = torch.full((T, d), float("nan"), device=gpu)
        ro = torch.full((T, d), float("nan"), device=gpu)
        sel = torch.full((T, k), -7, dtype=torch.int32, device=gpu)
        wt = torch.full((T, k), float("nan"), device=gpu)
        lay.forward(w, x, so, ro, sel, wt)
        torch.cuda.synchronize()
        so0, ro0, sel0, wt0 = O.moe_forward(case.cfg, hw, np_(x), T, NT)
        assert np.array_equal(np_(sel), sel0)
        assert bits_equal(np_(wt), wt0)
        assert bits_equal(np_(ro), ro0) and bits_equal(np_(so), so0), f"call {rep} differs from the oracle"
    lay.close()


@pytest.mark.parametrize("name", ["ref", "c2"])
def test_token_by_token_equals_one_batch(gpu, name):
    """64 calls with T = 1 (the matvec launches) against one call with
    T = 64 (the expert-major batch path: at most two pairs per expert on
    average) on the same context: the same routing bits and the same
    outputs, so a caller may split a prefill into chunks of any size up to
    that load (session.rs:795-895 runs the layer once per chunk); above it
    the grouped GEMMs add superblocks in their own order (f32 rounding)."""
    import torch
    case = C.with_tokens(C.CASES[name], 64)
    T, d, k = 64, case.cfg.d_model, case.cfg.top_k
    say(f"token by token vs batch {name} T={T}")
    w = C.make_weights(case, device=gpu)
    x = C.make_x(case, T=T, device=gpu)
    lay = dsmoe.MoeLayer(case.cfg, T)
    outs = []
    for mode in ("batch", "tokens"):
        so = torch.full((T, d), float("nan"), device=gpu)
        ro = torch.full((T, d), float("nan"), device=gpu)
        sel = torch.full((T, k), -7, dtype=torch.int32, device=gpu)
        wt = torch.full((T, k), float("nan"), device=gpu)
        if mode == "batch":
            lay.forward(w, x, so, ro, sel, wt)
        else:
            for t in range(T):
                lay.forward(w, x[t:t + 1], so[t:t + 1], ro[t:t + 1], sel[t:t + 1], wt[t:t + 1])
        torch.cuda.synchronize()
        outs.append([np_(v) for v in (so, ro, sel, wt)])
    (sb, rb, selb, wb), (st, rt, selt, wtt) = outs
    assert np.array_equal(selb, selt) and bits_equal(wb, wtt)
    e1 = assert_close(rt, rb, f"{name} routed_out tokens vs batch")
    e2 = assert_close(st, sb, f"{name} shared_out tokens vs batch")
    assert e1 == 1.0 and e2 == 1.0, "chunked and batched outputs differ in bits"
    lay.close()


@pytest.mark.parametrize("n,n_hc,T,has_add,mix,offset", [(4096, 4, 1, 1, 24, 0), (4096, 4, 5, 0, 24, 0),
                                                          (1000, 3, 2, 1, 15, 0), (4096, 4, 3, 1, 24, 1),
                                                          (7168, 2, 9, 1, 8, 0)])
def test_hc_expand_bitexact(gpu, n, n_hc, T, has_add, mix, offset):
    """hc_expand against the oracle, bit for bit: the vector form (n % 4 == 0,
    16-byte aligned), the scalar form (n = 1000, or buffers one float off
    16-byte alignment), has_add 0 and 1."""
    import torch
    say(f"hc_expand n={n} n_hc={n_hc} T={T} has_add={has_add} mix={mix} offset={offset}")
    rng = np.random.default_rng(n + T)
    bo = rng.normal(0, 1, (T, n)).astype(np.float32)
    ba = rng.normal(0, 1, (T, n)).astype(np.float32)
    res = rng.normal(0, 1, (T, n_hc, n)).astype(np.float32)
    split = rng.normal(0, 1, (T, mix)).astype(np.float32)

    def dev(a):  # a device copy starting `offset` floats into its allocation
        buf = torch.empty(a.size + offset, dtype=torch.float32, device=gpu)
        v = buf[offset:]
        v.copy_(torch.from_numpy(a.reshape(-1)))
        return v

    out = torch.full((T * n_hc * n + offset,), float("nan"), device=gpu)[offset:]
    dsmoe.hc_expand(dev(bo), dev(ba) if has_add else None, dev(res), dev(split), out, n, n_hc, T, mix, has_add)
    torch.cuda.synchronize()
    want = O.hc_expand(bo, ba if has_add else None, res, split, n, n_hc, T, mix, has_add)
    assert bits_equal(np_(out).reshape(T, n_hc, n), want)


@pytest.mark.parametrize("name", ["c2", "c1"])
def test_decode_layer_in_a_hip_graph(gpu, name):
    """The three decode launches captured in one HIP graph (no memset or
    allocation inside dsmoe_forward) and replayed with eager layer calls and
    synchronizations between the replays: every replay equals the eager call
    on the same input, bit for bit."""
    import torch
    case = C.CASES[name]
    cfg = case.cfg
    d, k = cfg.d_model, cfg.top_k
    say(f"hip graph decode {name}")
    w = C.make_weights(case, device=gpu)
    xs = [C.make_x(case, T=1, step=s, device=gpu) for s in range(4)]
    lay, ref = dsmoe.MoeLayer(cfg, 1), dsmoe.MoeLayer(cfg, 1)
    x = xs[0].clone()
    so, ro = torch.empty(1, d, device=gpu), torch.empty(1, d, device=gpu)
    sel, wt = torch.empty(1, k, dtype=torch.int32, device=gpu), torch.empty(1, k, device=gpu)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lay.forward(w, x, so, ro, sel, wt)  # warm (code objects loaded before the capture)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        lay.forward(w, x, so, ro, sel, wt)
    for rep in range(6):
        x.copy_(xs[rep % 4])
        g.replay()
        so2, ro2 = torch.empty(1, d, device=gpu), torch.empty(1, d, device=gpu)
        sel2, wt2 = torch.empty(1, k, dtype=torch.int32, device=gpu), torch.empty(1, k, device=gpu)
        ref.forward(w, xs[rep % 4], so2, ro2, sel2, wt2)
        torch.cuda.synchronize()
        for a_, b_ in ((so, so2), (ro, ro2), (sel, sel2), (wt, wt2)):
            assert bits_equal(np_(a_), np_(b_)), f"replay {rep} differs from the eager call"
    lay.close()
    ref.close()


def test_layer_from_gguf_file(gpu, tmp_path):
    """A layer written to a GGUF file, mapped by dsmoe_gguf_open and uploaded:
    dsmoe_forward on it gives the bits of the same layer from memory."""
    import torch
    from dsmoe import gguf as G
    case = C.CASES["c1"]
    cfg = case.cfg
    say("layer from gguf c1")
    w = C.make_weights(case, device=gpu)
    p = tmp_path / "c1.gguf"
    G.write(p, G.moe_layer_tensors(cfg, w, layer=0))
    with G.GgufFile(p) as g:
        w2 = G.layer_weights(g, 0, cfg, device=gpu)
    x = C.make_x(case, T=3, device=gpu)
    outs = []
    for ww in (w, w2):
        lay = dsmoe.MoeLayer(cfg, 3)
        so, ro = torch.empty(3, cfg.d_model, device=gpu), torch.empty(3, cfg.d_model, device=gpu)
        lay.forward(ww, x, so, ro)
        torch.cuda.synchronize()
        outs.append((np_(so), np_(ro)))
        lay.close()
    assert bits_equal(outs[0][0], outs[1][0]) and bits_equal(outs[0][1], outs[1][1])


def test_router_select_hash_bitexact(gpu):
    """Hash routing on the GPU against the oracle, bit for bit: tokens
    outside the table, negative tokens, table ids outside [0, E), the scalar
    token when no token array is given."""
    import torch
    say("router_select_hash")
    rng = np.random.default_rng(12)
    E, k, rows, T = 256, 6, 129, 40
    cfg = dsmoe.MoeConfig(d_model=512, d_ff=256, n_expert=E, top_k=k, route_scale=1.5, shared_fmt=-1)
    logits = rng.normal(0, 2, (T, E)).astype(np.float32)
    table = rng.integers(0, E, (rows, k)).astype(np.int32)
    table[5, 0], table[6, 5] = -1, E
    tokens = rng.integers(-3, rows + 3, T).astype(np.int32)
    tokens[:3] = [5, 6, 2**31 - 1]
    dl = torch.from_numpy(logits).to(gpu)
    dt = torch.from_numpy(table).to(gpu)
    for tok_arr in (tokens, None):
        probs = torch.empty(T, E, device=gpu)
        sel = torch.empty(T, k, dtype=torch.int32, device=gpu)
        w = torch.empty(T, k, device=gpu)
        dtok = None if tok_arr is None else torch.from_numpy(tok_arr).to(gpu)
        dsmoe.router_select_hash(cfg, dl, dt, rows, dtok, 17, T, probs, sel, w)
        p0, s0, w0 = O.router_select_hash(cfg, logits, table, rows, tok_arr, 17, T)
        torch.cuda.synchronize()
        assert np.array_equal(np_(sel), s0)
        assert bits_equal(np_(w), w0) and bits_equal(np_(probs), p0)


@pytest.mark.parametrize("T", [1, 5])
def test_layer_with_hash_routing(gpu, T):
    """dsmoe_forward with hash routing set: the selection equals
    dsmoe_router_select_hash on the layer's logits, and the routed output
    equals the per-kernel entry points on that selection."""
    import torch
    case = C.CASES["c1"]
    cfg = case.cfg
    d, I, E, k = cfg.d_model, cfg.d_ff, cfg.n_expert, cfg.top_k
    say(f"layer with hash routing T={T}")
    w = C.make_weights(case, device=gpu)
    x = C.make_x(case, T=T, device=gpu)
    rng = np.random.default_rng(13 + T)
    rows = 50
    table = torch.from_numpy(rng.integers(0, E, (rows, k)).astype(np.int32)).to(gpu)
    tokens = torch.from_numpy(rng.integers(0, rows, T).astype(np.int32)).to(gpu)
    lay = dsmoe.MoeLayer(cfg, T)
    lay.set_hash_routing(table, rows, tokens)
    so, ro = torch.empty(T, d, device=gpu), torch.empty(T, d, device=gpu)
    sel, wt = torch.empty(T, k, dtype=torch.int32, device=gpu), torch.empty(T, k, device=gpu)
    lay.forward(w, x, so, ro, sel, wt)
    logits = torch.empty(T, E, device=gpu)
    dsmoe.router_logits(w.router_f16, x, logits, d, E, T)
    s2, w2 = torch.empty(T, k, dtype=torch.int32, device=gpu), torch.empty(T, k, device=gpu)
    dsmoe.router_select_hash(cfg, logits, table, rows, tokens, 0, T, None, s2, w2)
    xq = torch.empty(T * (d // 256) * 292, dtype=torch.uint8, device=gpu)
    dsmoe.q8k_quantize(x, xq, d, T)
    m = torch.empty(T * k, I, device=gpu)
    dsmoe.gate_up_mid(w.gate, w.up, xq, s2, w2, None, None, m, d, I, T, k, E, cfg.swiglu_clamp)
    mq = torch.empty(T * k * (I // 256) * 292, dtype=torch.uint8, device=gpu)
    dsmoe.q8k_quantize(m, mq, I, T * k)
    ro2 = torch.empty(T, d, device=gpu)
    dsmoe.down(w.down, mq, s2, None, ro2, d, I, T, k, E)
    torch.cuda.synchronize()
    assert np.array_equal(np_(sel), np_(s2)) and bits_equal(np_(wt), np_(w2))
    assert bits_equal(np_(ro), np_(ro2))
    lay.set_hash_routing(None)
    lay.forward(w, x, so, ro, sel, wt)  # back to top-k
    torch.cuda.synchronize()
    lay.close()


# ---------------------------------------------------------------- HC FFN pre-norm
@pytest.mark.parametrize("n,rows,eps", [(256, 1, 1e-5), (128, 1, 1e-5), (16384, 3, 1e-6), (1000, 2, 1e-6)])
def test_rms_norm_plain_bitexact(gpu, n, rows, eps):
    """rms_norm_plain (norm.rs:14-63) against the oracle bit for bit, with
    the reference's own checks (kernels_smoke.rs:306-392) on all-equal rows."""
    import torch
    say(f"rms_norm_plain n={n} rows={rows}")
    rng = np.random.default_rng(n)
    x = rng.normal(0, 2, (rows, n)).astype(np.float32)
    out = torch.full((rows, n), float("nan"), device=gpu)
    dsmoe.rms_norm_plain(torch.from_numpy(x).to(gpu), out, n, rows, eps)
    torch.cuda.synchronize()
    assert bits_equal(np_(out), O.rms_norm_plain(x, n, rows, eps))
    if n in (128, 256):
        one = torch.full((1, n), 2.0, device=gpu)
        three = torch.full((1, n), 3.0, device=gpu)
        o1, o3 = torch.empty_like(one), torch.empty_like(three)
        dsmoe.rms_norm_plain(one, o1, n, 1, eps)
        dsmoe.rms_norm_plain(three, o3, n, 1, eps)
        torch.cuda.synchronize()
        assert abs(float(o1.pow(2).mean().sqrt()) - 1.0) < 1e-3 and bool((o1 == o1[0, 0]).all())
        assert abs(float(o1[0, 0]) - float(o3[0, 0])) < 1e-4


@pytest.mark.parametrize("n,T,iters", [(4096, 1, 20), (4096, 5, 20), (1000, 2, 1), (7168, 3, 3)])
def test_hc_split_norm_bitexact(gpu, n, T, iters):
    """hc_split_weighted_sum_norm_fused (hc.rs:313-398): split, ffn_cur and
    ffn_norm against the oracle bit for bit."""
    import torch
    say(f"hc_split_norm n={n} T={T} iters={iters}")
    rng = np.random.default_rng(n + T)
    mix = rng.normal(0, 1, (T, 24)).astype(np.float32)
    scale = np.array([0.5, 1.0, 1.5], np.float32)
    base = rng.normal(0, 0.3, 24).astype(np.float32)
    res = rng.normal(0, 1, (T, 4, n)).astype(np.float32)
    nw = rng.normal(1, 0.1, n).astype(np.float32)
    d = lambda a: torch.from_numpy(a).to(gpu)
    split = torch.full((T, 24), float("nan"), device=gpu)
    cur, norm = (torch.full((T, n), float("nan"), device=gpu) for _ in range(2))
    dsmoe.hc_split_norm(d(mix), d(scale), d(base), d(res), d(nw), split, cur, norm, n, T, iters, 1e-6, 1e-6)
    torch.cuda.synchronize()
    ws, wc, wn = O.hc_split_norm(mix, scale, base, res, nw, n, T, iters, 1e-6, 1e-6)
    assert bits_equal(np_(split), ws)
    assert bits_equal(np_(cur), wc)
    assert bits_equal(np_(norm), wn)


def test_hc_ffn_prenorm_chain(gpu):
    """The FFN pre-norm of session.rs:1830-1892 at the reference's shape
    (n_embd 4096, HC_DIM 16384, 24 mix values): rms_norm_plain ->
    router_logits (matmul_f16, d = 16384 on the wide-row path) ->
    hc_split_norm, each stage bit-equal to the oracle on the previous stage's
    oracle output, and the layer input `norm` bit-equal end to end."""
    import torch
    n, T = 4096, 2
    say(f"hc_ffn_prenorm n={n} T={T}")
    rng = np.random.default_rng(11)
    hc = rng.normal(0, 1, (T, 4, n)).astype(np.float32)
    wfn = (rng.normal(0, 0.02, (24, 4 * n)).astype(np.float16)).view(np.uint16)
    scale = np.array([0.5, 1.0, 1.5], np.float32)
    base = rng.normal(0, 0.3, 24).astype(np.float32)
    nw = rng.normal(1, 0.1, n).astype(np.float32)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    flat = torch.empty(T, 4 * n, device=gpu)
    mix = torch.empty(T, 24, device=gpu)
    split = torch.empty(T, 24, device=gpu)
    cur, norm = torch.empty(T, n, device=gpu), torch.empty(T, n, device=gpu)
    wdev = torch.from_numpy(wfn.view(np.int16)).to(gpu)
    dsmoe.hc_ffn_prenorm(d(hc), wdev, d(scale), d(base), d(nw), flat, mix, split, cur, norm, n, T)
    torch.cuda.synchronize()
    f = O.rms_norm_plain(hc.reshape(T, 4 * n), 4 * n, T, 1e-6)
    assert bits_equal(np_(flat), f)
    m = O.router_logits(wfn, f, 4 * n, 24, T)
    assert bits_equal(np_(mix), m)
    ws, wc, wn = O.hc_split_norm(m, scale, base, hc, nw, n, T, 20, 1e-6, 1e-6)
    assert bits_equal(np_(split), ws) and bits_equal(np_(cur), wc) and bits_equal(np_(norm), wn)


def test_forward_empty_and_oversized_batches(gpu):
    """T = 0 is a no-op that returns success and writes nothing; a batch
    larger than the context's max_tokens is refused before any launch, on
    the decode and the batch context alike."""
    import torch
    case = C.CASES["c1"]
    w = C.make_weights(case, device=gpu)
    d, k = case.cfg.d_model, case.cfg.top_k
    for max_t in (8, 64):
        say(f"empty / oversized batch, max_tokens={max_t}")
        lay = dsmoe.MoeLayer(case.cfg, max_t)
        x = C.make_x(case, T=max_t + 1, device=gpu)
        so = torch.full((max_t + 1, d), float("nan"), device=gpu)
        ro = torch.full((max_t + 1, d), float("nan"), device=gpu)
        sel = torch.full((max_t + 1, k), -7, dtype=torch.int32, device=gpu)
        lay.forward(w, x[:0], so[:0], ro[:0], sel[:0])
        torch.cuda.synchronize()
        assert torch.isnan(so).all() and torch.isnan(ro).all() and (sel == -7).all()
        with pytest.raises(dsmoe.DsmoeError):
            lay.forward(w, x, so, ro, sel)
        torch.cuda.synchronize()
        assert torch.isnan(ro).all() and (sel == -7).all()
        lay.close()
