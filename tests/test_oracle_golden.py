"""Pins the CPU oracle before it is trusted as the GPU checker.

Each check is one of: a known answer held by the reference's own tests
(engine/tests/quant_cpu.rs, kernels_smoke.rs), the reference's data tables
(tests/golden/reference_tables.json), a brute force over exact integer
codes, a closed form, or float64 mathematics.  None restates the oracle's
own formula."""
import ctypes
import math
import os
import re

import numpy as np
import pytest

import oracle_ref
from oracle_ref import P
import quant_ref as Q

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KA = Q.GOLDEN["known_answers"]
F16_ONE = 0x3C00


def f32(x):
    return np.float32(x)


# ---------------------------------------------------------------- tables
def test_grid_table_matches_reference_tables(oracle):
    ours = [oracle.or_iq2_grid(i) for i in range(256)]
    assert ours == [int(h, 16) for h in Q.GOLDEN["iq2xxs_grid_hex"]]
    import hashlib
    h = hashlib.sha256(b"".join(v.to_bytes(8, "little") for v in ours)).hexdigest()
    assert h == Q.GOLDEN["iq2xxs_grid_sha256_le"]


def test_product_grid_table_matches_reference_tables():
    txt = open(os.path.join(ROOT, "deepseek-rs_amd", "csrc", "dsmoe_formats.h")).read()
    body = txt[txt.index("kIq2xxsGrid[256]"):]
    body = body[:body.index("};")]
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]+)ull", body)]
    assert vals == [int(h, 16) for h in Q.GOLDEN["iq2xxs_grid_hex"]]


@pytest.mark.skipif(not os.path.isdir("/root/reference"), reason="reference sources not mounted")
def test_golden_file_matches_reference_source():
    src = open("/root/reference/engine/src/kernels/quantize.rs").read()
    txt = re.search(r"IQ2_XXS_GRID: \[u64; 256\] = \[(.*?)\];", src, re.S).group(1)
    assert [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", txt)] == [int(h, 16) for h in Q.GOLDEN["iq2xxs_grid_hex"]]


def test_sign_table(oracle):
    assert [oracle.or_iq2_sign(i) for i in range(128)] == Q.GOLDEN["iq2_signs"]
    for s in Q.GOLDEN["iq2_signs"]:
        assert bin(s).count("1") % 2 == 0


# ---------------------------------------------------------------- f16
def test_f16_ftz_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([oracle.or_f16_to_f32(int(b)) for b in bits], np.float32)
    ref = bits.view(np.float16).astype(np.float32)
    sub = ((bits >> 10) & 0x1F) == 0
    ref = np.where(sub, np.copysign(np.float32(0), ref), ref)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# ---------------------------------------------------------------- math
def _ulps(a, b):
    a = np.float32(a)
    b64 = float(b)
    sp = np.spacing(np.float32(abs(b64))) if b64 != 0 else np.float32(1e-45)
    return abs(float(a) - b64) / float(sp)


def test_exp_log_softplus_silu_float64(oracle):
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-103, 88, 4000), rng.uniform(-2, 2, 2000), [0.0, 1.0, -1.0, 88.7, -87.0]])
    worst = 0.0
    for x in xs.astype(np.float32):
        worst = max(worst, _ulps(oracle.or_expf(float(x)), math.exp(float(x))))
    assert worst <= 3.0, worst
    ys = np.concatenate([rng.uniform(1e-30, 1e30, 2000), rng.uniform(0.5, 4.0, 2000), [1.0, 2.0, 0.75]])
    worst = 0.0
    for y in ys.astype(np.float32):
        if y == 1.0:
            assert oracle.or_logf(1.0) == 0.0
            continue
        worst = max(worst, _ulps(oracle.or_logf(float(y)), math.log(float(y))))
    assert worst <= 3.0, worst
    for x in rng.uniform(-30, 30, 3000).astype(np.float32):
        ref = float(x) if x > 20 else (math.exp(float(x)) if x < -20 else math.log1p(math.exp(float(x))))
        got = oracle.or_softplus(float(x))
        if -20 <= x <= 20:
            # ln(1 + e^x) in f32 (moe.rs:22) rounds 1 + e^x first: absolute error ~2^-24
            assert abs(got - ref) <= 1.2e-7 + 4 * float(np.spacing(np.float32(ref)))
        else:
            assert _ulps(got, ref) <= 4.0
        g = float(x)
        assert abs(oracle.or_silu(g) - g / (1 + math.exp(-g))) <= 4 * np.spacing(np.float32(abs(g) + 1e-30)) + 1e-37
    assert math.isinf(oracle.or_expf(89.0)) and oracle.or_expf(-104.0) == 0.0


def test_router_math_known_answers(oracle):
    assert abs(oracle.or_softplus(100.0) - KA["quant_cpu.rs:453-456 softplus(100)"]) < 0.01
    assert oracle.or_softplus(-100.0) < KA["quant_cpu.rs:458-461 softplus(-100) below"]
    assert abs(oracle.or_softplus(0.0) - KA["quant_cpu.rs:463-466 softplus(0)"]) < 1e-5
    assert abs(math.sqrt(oracle.or_softplus(0.0)) - KA["quant_cpu.rs:468-471 score(0)"]) < 1e-5
    v, tol = KA["quant_cpu.rs:492-501 score(3.8282)"]
    assert abs(np.sqrt(np.float32(oracle.or_softplus(3.8282))) - v) < tol


# ---------------------------------------------------------------- IQ2_XXS . Q8_K
def test_iq2_known_answers(oracle):
    ones = np.ones(256, np.int8)
    iq2 = Q.make_iq2_block(F16_ONE, 0, 0, 1)
    assert oracle.or_dot_iq2_xxs_q8k(P(iq2), P(Q.make_q8k_block(0.0, ones))) == KA["quant_cpu.rs:304-317 iq2 zero q8k scale"]
    assert oracle.or_dot_iq2_xxs_q8k(P(Q.make_iq2_block(0, 0, 0, 1)), P(Q.make_q8k_block(1.0, ones))) == 0.0
    r1 = oracle.or_dot_iq2_xxs_q8k(P(iq2), P(Q.make_q8k_block(1.0, ones)))
    assert abs(r1 - KA["quant_cpu.rs:320-334 iq2 grid0 sign0 ls1 ones"]) < 0.01
    r3 = oracle.or_dot_iq2_xxs_q8k(P(Q.make_iq2_block(F16_ONE, 0, 0, 3)), P(Q.make_q8k_block(1.0, ones)))
    assert abs(r3 - KA["quant_cpu.rs:337-349 iq2 ls3 over ls1"] * r1) < 0.01
    r2 = oracle.or_dot_iq2_xxs_q8k(P(iq2), P(Q.make_q8k_block(2.0, ones)))
    assert abs(r2 - KA["quant_cpu.rs:352-364 iq2 q8k d linearity"] * r1) < 0.01


def _rand_iq2(rng, n):
    b = rng.integers(0, 256, size=(n, 66), dtype=np.uint8)
    d = (rng.uniform(0.01, 2.0, n) * rng.choice([-1, 1], n)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    return b


def _rand_q8k(rng, n, qmax=127):
    out = np.zeros((n, 292), np.uint8)
    for i in range(n):
        out[i] = Q.make_q8k_block(rng.uniform(-1, 1), rng.integers(-qmax, qmax + 1, 256))
    return out


def test_iq2_bruteforce_integer_codes(oracle):
    rng = np.random.default_rng(1)
    blocks = _rand_iq2(rng, 200)
    q8 = _rand_q8k(rng, 200)
    d, codes = Q.iq2_codes(blocks)
    yd, qs, _ = Q.q8k_unpack(q8)
    for i in range(200):
        want = int((codes[i] * qs[i]).sum())
        assert oracle.or_iq2_xxs_bsum(P(blocks[i]), P(q8[i])) == want
        f = oracle.or_dot_iq2_xxs_q8k(P(blocks[i]), P(q8[i]))
        ref = np.float32(np.float32(np.float32(0.125) * d[i]) * yd[i]) * np.float32(want)
        assert np.float32(f).view(np.uint32) == ref.view(np.uint32)


def test_iq2_closed_form_single_subblock(oracle):
    # one non-zero 32-sub-block j: result = 0.125*d*yd*ls*sum(sign*g*q)
    rng = np.random.default_rng(2)
    for j in range(8):
        for _ in range(10):
            blk = np.zeros(66, np.uint8)
            blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
            gi = rng.integers(0, 256, 4)
            si = rng.integers(0, 128, 4)
            lcode = int(rng.integers(0, 16))
            aux0 = int(gi[0] | (gi[1] << 8) | (gi[2] << 16) | (gi[3] << 24))
            aux1 = int(si[0] | (si[1] << 7) | (si[2] << 14) | (si[3] << 21)) | (lcode << 28)
            blk[2 + 8 * j: 10 + 8 * j] = np.frombuffer(np.array([aux0, aux1], np.uint32).tobytes(), np.uint8)
            q = np.zeros(256, np.int8)
            q[32 * j: 32 * j + 32] = rng.integers(-127, 128, 32)
            s = 0
            for g in range(4):
                gb = [(int(Q.GOLDEN["iq2xxs_grid_hex"][gi[g]], 16) >> (8 * t)) & 0xFF for t in range(8)]
                sb = Q.GOLDEN["iq2_signs"][si[g]]
                for t in range(8):
                    s += (-gb[t] if (sb >> t) & 1 else gb[t]) * int(q[32 * j + 8 * g + t])
            ls = 2 * lcode + 1
            # blocks other than j hold grid index 0 with ls 1 but aux words 0 -> they decode to
            # +8 magnitudes; zero activations there make them contribute nothing
            got = oracle.or_dot_iq2_xxs_q8k(P(blk), P(Q.make_q8k_block(0.25, q)))
            assert got == pytest.approx(0.125 * 0.5 * 0.25 * ls * s, rel=1e-6, abs=1e-6)


# ---------------------------------------------------------------- Q2_K . Q8_K
def test_q2k_known_answers(oracle):
    ones = np.ones(256, np.int8)
    q8 = Q.make_q8k_block(1.0, ones)
    assert abs(oracle.or_dot_q2k_q8k(P(Q.make_q2k_block(1.0, 0.0, 1, 1, 0x00)), P(q8))) < 0.01
    assert abs(oracle.or_dot_q2k_q8k(P(Q.make_q2k_block(1.0, 0.0, 1, 1, 0x55)), P(q8)) - KA["quant_cpu.rs:401-414 q2k 0x55 sc1"]) < 0.5
    r0 = oracle.or_dot_q2k_q8k(P(Q.make_q2k_block(1.0, 0.0, 1, 0, 0x55)), P(q8))
    r1 = oracle.or_dot_q2k_q8k(P(Q.make_q2k_block(1.0, 1.0, 1, 0, 0x55)), P(q8))
    assert abs(r0 - r1) < 0.01


def test_q2k_bruteforce_integer_codes(oracle):
    rng = np.random.default_rng(3)
    n = 200
    blocks = rng.integers(0, 256, size=(n, 84), dtype=np.uint8)
    blocks[:, 80:82] = rng.uniform(0.01, 1, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    blocks[:, 82:84] = rng.uniform(0.01, 1, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    q8 = _rand_q8k(rng, n)
    d, dmin, q, lo, hi = Q.q2k_codes(blocks)
    yd, qs, bs = Q.q8k_unpack(q8)
    g = np.arange(256) // 16
    for i in range(n):
        isum = int((lo[i][g] * q[i] * qs[i]).sum())
        summs = int((bs[i] * hi[i]).sum())
        a, b = ctypes.c_int32(), ctypes.c_int32()
        oracle.or_q2k_isum_summs(P(blocks[i]), P(q8[i]), ctypes.byref(a), ctypes.byref(b))
        assert (a.value, b.value) == (isum, summs)
        dall = np.float32(yd[i] * d[i])
        dm = np.float32(yd[i] * dmin[i])
        ref = np.float32(np.float32(dall * np.float32(isum)) - np.float32(dm * np.float32(summs)))
        assert np.float32(oracle.or_dot_q2k_q8k(P(blocks[i]), P(q8[i]))).view(np.uint32) == ref.view(np.uint32)


# ---------------------------------------------------------------- Q8_K / Q8_0 activation quantizers
def test_q8k_invariants_and_tree_tiebreak(oracle):
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, (6, 512)).astype(np.float32)
    x[2, :256] = 0.0  # zero block
    out = oracle_ref.q8k_quantize(x, 512, 6)
    d, qs, bs = Q.q8k_unpack(out)
    assert np.array_equal(bs, qs.reshape(-1, 16, 16).sum(2))
    assert d[4] == 0 and not qs[4].any() and not bs[4].any()
    xb = x.reshape(-1, 256)
    for i in range(12):
        if i == 4:
            continue
        k = int(np.argmax(np.abs(xb[i])))
        assert qs[i][k] == -127
        assert np.all(np.abs(qs[i] * np.float64(d[i]) - xb[i]) <= 0.5 * abs(d[i]) * 1.0001 + 1e-12)
    # all ones: iscale = -127 -> q = -127, d = -1/127
    o = oracle_ref.q8k_quantize(np.ones(256, np.float32), 256, 1)
    d1, q1, _ = Q.q8k_unpack(o)
    assert (q1 == -127).all() and d1[0] == np.float32(1.0) / np.float32(-127.0)
    # equal |x| with opposite signs at 1 (-1) and 2 (+1): the reference's halving tree
    # (quantize.rs:338-350) keeps element 2 (node 0 takes node 2 at stride 2 and
    # keeps it against node 1 at stride 1), so +1 is the signed max.
    t = np.full(256, 0.5, np.float32)
    t[1], t[2] = -1.0, 1.0
    d2, q2, _ = Q.q8k_unpack(oracle_ref.q8k_quantize(t, 256, 1))
    assert q2[0][2] == -127 and q2[0][1] == 127 and d2[0] < 0


def test_q8_0_known_answers(oracle):
    xq, xs = oracle_ref.q8_0_quantize(np.ones(32, np.float32), 32, 1)
    assert (xq == KA["kernels_smoke.rs:518-548 q8_0 ones q"]).all()
    assert abs(xs[0] - KA["kernels_smoke.rs:518-548 q8_0 ones scale"]) < 1e-6
    x = ((np.arange(32) - 16) * 0.1).astype(np.float32)
    xq, xs = oracle_ref.q8_0_quantize(x, 32, 1)
    assert np.all(np.abs(xq * xs[0] - x) < xs[0] * KA["kernels_smoke.rs:550-610 q8_0 ramp roundtrip factor"])
    # matvec known answers (quant_cpu.rs:156-245, kernels_smoke.rs:166-302)
    def row(scale_bits, q):
        b = np.zeros(34, np.uint8)
        b[0], b[1] = scale_bits & 0xFF, scale_bits >> 8
        b[2:] = np.array(q, np.int8).view(np.uint8)
        return b
    def mv(w, xq, xs, in_dim):
        out = np.zeros(1, np.float32)
        oracle.or_q8_0_matvec(P(w), P(xq), P(xs), P(out), in_dim, 1, 1, 1)
        return out[0]
    one = np.ones(32, np.int8)
    s1 = np.ones(1, np.float32)
    assert mv(row(F16_ONE, [0] * 32), one, s1, 32) == 0.0
    assert mv(row(F16_ONE, [1] * 32), np.zeros(32, np.int8), s1, 32) == 0.0
    assert mv(row(F16_ONE, [1] * 32), one, s1, 32) == KA["kernels_smoke.rs:166-214 q8_0 matvec ones"]
    assert mv(row(F16_ONE, [-1] * 32), one, s1, 32) == KA["kernels_smoke.rs:216-255 q8_0 matvec minus ones"]
    assert mv(row(0x3800, [1] * 32), one, s1, 32) == KA["kernels_smoke.rs:257-302 q8_0 matvec scale 0.5"]
    two = np.concatenate([row(0x3800, [1] * 32), row(0x3800, [1] * 32)])
    assert mv(two, np.ones(64, np.int8), np.ones(2, np.float32), 64) == 32.0


def test_swiglu_known_answers(oracle):
    def sw(g, u, clamp, w):
        gg, uu, o = np.full(4, g, np.float32), np.full(4, u, np.float32), np.zeros(4, np.float32)
        oracle.or_swiglu(P(gg), P(uu), P(o), 4, clamp, w)
        return o[0]
    lo, hi = KA["kernels_smoke.rs:397-432 swiglu(10,2) range"]
    assert lo < sw(10.0, 2.0, 0.0, 1.0) < hi
    assert sw(0.0, 5.0, 0.0, 1.0) == 0.0
    assert sw(1.0, 1.0, 0.0, 2.0) == pytest.approx(2.0 * sw(1.0, 1.0, 0.0, 1.0), rel=1e-6)
    # clamp (utils.rs:149-159): gate capped above only, up both sides
    assert sw(20.0, 20.0, 10.0, 1.0) == pytest.approx(10.0 / (1 + math.exp(-10.0)) * 10.0, rel=1e-6)
    assert sw(-20.0, -20.0, 10.0, 1.0) == pytest.approx(-20.0 / (1 + math.exp(20.0)) * -10.0, rel=1e-5)


# ---------------------------------------------------------------- router
def test_router_logits_closed_forms(oracle):
    # kernels_smoke.rs:54-148: all-ones W and x -> in_dim; identity row picks x[0]
    d, E = 512, 4
    w = np.full(E * d, F16_ONE, np.uint16)
    assert (oracle_ref.router_logits(w, np.ones(d, np.float32), d, E, 1) == d).all()
    w = np.zeros(E * d, np.uint16)
    w[0] = F16_ONE
    x = np.arange(d, dtype=np.float32)
    out = oracle_ref.router_logits(w, x, d, E, 1)
    assert out[0, 0] == 0.0 and (out[0, 1:] == 0).all()
    w[0], w[5] = 0, F16_ONE
    assert oracle_ref.router_logits(w, x, d, E, 1)[0, 0] == 5.0
    # f16 subnormal weights flush to zero (utils.rs:16-29)
    w = np.full(E * d, 0x0001, np.uint16)
    assert (oracle_ref.router_logits(w, np.ones(d, np.float32), d, E, 1) == 0).all()
    # random: close to float64
    rng = np.random.default_rng(5)
    wf = rng.normal(0, 0.02, (E, 7168)).astype(np.float16)
    x = rng.normal(0, 1, 7168).astype(np.float32)
    out = oracle_ref.router_logits(wf.view(np.uint16).copy(), x, 7168, E, 1)
    ref = Q.f16_ftz(wf.view(np.uint16)).astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(out[0], ref, rtol=1e-4, atol=1e-4)


class _Cfg:
    def __init__(self, E, k, n_group=1, topk_group=1, scale=1.5, has_bias=0):
        self.d_model, self.d_ff, self.n_expert, self.top_k = 512, 256, E, k
        self.n_group, self.topk_group, self.route_scale, self.swiglu_clamp = n_group, topk_group, scale, 10.0
        self.has_bias, self.shared_fmt, self.d_ff_shared = has_bias, -1, 256


def _brute_select(probs, bias, k, scale, n_group=1, topk_group=1):
    E = probs.size
    score = (probs + bias).astype(np.float32) if bias is not None else probs
    eligible = np.ones(E, bool)
    if n_group > 1:
        gsz = E // n_group
        gs = []
        for g in range(n_group):
            v = np.sort(score[g * gsz:(g + 1) * gsz][~np.isnan(score[g * gsz:(g + 1) * gsz])])[::-1]
            v = list(v) + [-np.inf, -np.inf]
            gs.append(np.float32(v[0]) + np.float32(v[1]) if gsz >= 2 else np.float32(v[0]))
        order = sorted([g for g in range(n_group) if gs[g] > -np.inf], key=lambda g: (-gs[g], g))[:topk_group]
        eligible = np.zeros(E, bool)
        for g in order:
            eligible[g * gsz:(g + 1) * gsz] = True
    cand = [e for e in range(E) if eligible[e] and score[e] > -np.inf and not np.isnan(score[e])]
    cand.sort(key=lambda e: (-score[e], e))
    sel = cand[:k] + [-1] * (k - len(cand[:k]))
    w = np.array([probs[e] if e >= 0 else 0 for e in sel], np.float32)
    s = np.float32(0)
    for v in w:
        s = np.float32(s + v)
    s = max(s, np.float32(6.103515625e-5))
    return np.array(sel, np.int32), (w / np.float32(s / np.float32(scale))).astype(np.float32)


@pytest.mark.parametrize("E,k,ng,tg,bias", [(256, 6, 1, 1, False), (256, 6, 1, 1, True), (64, 6, 1, 1, True),
                                            (256, 8, 8, 4, True), (256, 8, 8, 4, False), (16, 3, 4, 2, True)])
def test_router_select_bruteforce(oracle, E, k, ng, tg, bias):
    rng = np.random.default_rng(E * 7 + k)
    T = 40
    logits = rng.normal(0, 2, (T, E)).astype(np.float32)
    logits[0, :] = 0.5                      # all tie
    logits[1, ::3] = 1.25                   # many ties
    logits[2, 5] = np.nan                   # NaN never selected
    b = rng.normal(0, 0.01, E).astype(np.float32) if bias else None
    cfg = _Cfg(E, k, ng, tg, 2.5 if ng > 1 else 1.5, int(bias))
    probs, sel, w = oracle_ref.router_select(cfg, logits, b, T)
    for t in range(T):
        es, ew = _brute_select(probs[t], b, k, cfg.route_scale, ng, tg)
        assert np.array_equal(sel[t], es), t
        assert np.array_equal(w[t].view(np.uint32), ew.view(np.uint32)), t
    assert 5 not in sel[2]
    ok = sel[:, -1] >= 0
    assert np.allclose(w[ok].sum(1), cfg.route_scale, rtol=1e-5)


def test_router_normalise_ratio(oracle):
    # quant_cpu.rs:473-489: normalised weights sum to 1.5 and keep ratios
    E = 256
    logits = np.full((1, E), -30.0, np.float32)
    logits[0, 10], logits[0, 20] = 8.0, 2.0
    cfg = _Cfg(E, 2)
    probs, sel, w = oracle_ref.router_select(cfg, logits, None, 1)
    assert list(sel[0]) == [10, 20]
    assert abs(w[0].sum() - KA["quant_cpu.rs:473-482 normalise sum"]) < 1e-5
    assert abs(w[0, 0] / w[0, 1] - probs[0, 10] / probs[0, 20]) < 1e-5


# ---------------------------------------------------------------- dispatch
def test_dispatch_matches_stable_argsort(oracle):
    rng = np.random.default_rng(6)
    for E, P_, bm in [(256, 1, 16), (256, 16384, 32), (64, 600, 8), (8, 0, 4)]:
        sel = rng.integers(-1, E, P_).astype(np.int32)
        counts, offsets, sp, to, te, ts = oracle_ref.dispatch(sel, E, bm)
        key = np.where(sel < 0, 0, sel)
        assert np.array_equal(counts, np.bincount(key, minlength=E))
        assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))
        assert np.array_equal(sp, np.argsort(key, kind="stable"))
        nt = (counts + bm - 1) // bm
        assert np.array_equal(to, np.concatenate([[0], np.cumsum(nt)]))
        assert np.array_equal(te, np.repeat(np.arange(E), nt))
        assert np.array_equal(ts, np.concatenate([np.arange(n) * bm for n in nt]) if nt.sum() else np.zeros(0))


# ---------------------------------------------------------------- whole layer vs float64
def test_layer_matches_float64_dequant_gemm(oracle):
    """Independent closed form: dequantise every weight to float64 and run
    the layer in float64.  The activations go through the same quantizers as
    the reference's (Q8_K of x and of the routed SwiGLU output, Q8_0 of x and
    of the shared SwiGLU output; each quantizer is pinned by its own known
    answers above), so what is left between the oracle and this is f32
    rounding.  The weights are large enough that the SwiGLU clamp (gate <= 10,
    |up| <= 10, session.rs:1934-1950) is active on a good share of the rows,
    so a dropped or misplaced clamp fails the comparison."""
    rng = np.random.default_rng(7)
    d, I, E, k, Is, T = 512, 256, 8, 2, 256, 3
    nb, nbi = d // 256, I // 256

    def iq2_tensor(rows, nblk, n):
        b = np.zeros((n * rows * nblk, 66), np.uint8)
        b[:, 2:] = rng.integers(0, 256, (n * rows * nblk, 64), dtype=np.uint8)
        b[:, 0:2] = rng.uniform(0.004, 0.012, n * rows * nblk).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return b

    def q2k_tensor(rows, nblk, n):
        b = rng.integers(0, 256, (n * rows * nblk, 84), dtype=np.uint8)
        b[:, 80:82] = rng.uniform(0.0005, 0.002, b.shape[0]).astype(np.float16).view(np.uint8).reshape(-1, 2)
        b[:, 82:84] = rng.uniform(0.0005, 0.002, b.shape[0]).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return b

    def q80_tensor(rows, cols, lo, hi):
        b = np.zeros((rows * cols // 32, 34), np.uint8)
        b[:, 2:] = rng.integers(-127, 128, (b.shape[0], 32)).astype(np.int8).view(np.uint8)
        b[:, 0:2] = rng.uniform(lo, hi, b.shape[0]).astype(np.float16).view(np.uint8).reshape(-1, 2)
        return b

    w = {
        "router": rng.normal(0, 0.05, (E, d)).astype(np.float16).view(np.uint16).copy(),
        "bias": rng.normal(0, 0.01, E).astype(np.float32),
        "gate": iq2_tensor(I, nb, E), "up": iq2_tensor(I, nb, E), "down": q2k_tensor(d, nbi, E),
        "sh_gate": q80_tensor(Is, d, 0.002, 0.006), "sh_up": q80_tensor(Is, d, 0.002, 0.006),
        "sh_down": q80_tensor(d, Is, 0.0001, 0.0003),
    }
    x = rng.normal(0, 1, (T, d)).astype(np.float32)
    cfg = _Cfg(E, k, has_bias=1)
    cfg.d_model, cfg.d_ff, cfg.shared_fmt, cfg.d_ff_shared = d, I, 0, Is
    so, ro, sel, wt = oracle_ref.moe_forward(cfg, {kk: v.reshape(-1) if v.ndim > 1 and v.dtype == np.uint8 else v for kk, v in w.items()}, x, T)

    Wg = Q.dequant_iq2(w["gate"]).reshape(E, I, d)
    Wu = Q.dequant_iq2(w["up"]).reshape(E, I, d)
    Wd = Q.dequant_q2k(w["down"]).reshape(E, d, I)
    Sg = Q.dequant_q8_0(w["sh_gate"]).reshape(Is, d)
    Su = Q.dequant_q8_0(w["sh_up"]).reshape(Is, d)
    Sd = Q.dequant_q8_0(w["sh_down"]).reshape(d, Is)

    def q8k_deq(v):
        n = v.shape[-1]
        dd, qs, _ = Q.q8k_unpack(oracle_ref.q8k_quantize(v.astype(np.float32).reshape(1, n), n, 1))
        return (dd.astype(np.float64)[:, None] * qs).reshape(n)

    def q80_deq(v):
        n = v.shape[-1]
        q, sc = oracle_ref.q8_0_quantize(v.astype(np.float32).reshape(1, n), n, 1)
        return (q.reshape(-1, 32).astype(np.float64) * sc.astype(np.float64)[:, None]).reshape(n)

    silu = lambda g: g / (1 + np.exp(-g))
    clamped = total = 0
    for t in range(T):
        xk = q8k_deq(x[t])
        ref = np.zeros(d)
        for j in range(k):
            e = sel[t, j]
            g0, u0 = Wg[e] @ xk, Wu[e] @ xk
            clamped += int(np.sum(g0 > 10.0) + np.sum(np.abs(u0) > 10.0))
            total += 2 * I
            mid = silu(np.minimum(g0, 10.0)) * np.clip(u0, -10, 10) * wt[t, j]
            ref += Wd[e] @ q8k_deq(mid)
        rel = np.linalg.norm(ro[t] - ref) / np.linalg.norm(ref)
        assert rel < 1e-3, (t, rel)
        x0 = q80_deq(x[t])
        g0, u0 = Sg @ x0, Su @ x0
        clamped += int(np.sum(g0 > 10.0) + np.sum(np.abs(u0) > 10.0))
        total += 2 * Is
        sref = Sd @ q80_deq(silu(np.minimum(g0, 10.0)) * np.clip(u0, -10, 10))
        rel = np.linalg.norm(so[t] - sref) / np.linalg.norm(sref)
        assert rel < 1e-3, (t, rel)
    # the clamp is active on a real share of the products, not a corner
    assert 0.05 < clamped / total < 0.95, clamped / total


def test_moe_sum_is_slot_ordered(oracle):
    """or_moe_sum adds the k slots of a row left to right in f32
    (moe.rs:983-1005): values where the order changes the f32 result."""
    d, k, T = 4, 3, 2
    down = np.zeros((T, k, d), np.float32)
    down[0, :, 0] = [1e8, 1.0, -1e8]     # (1e8 + 1) - 1e8 = 0 in f32; any other order gives 1 or 0
    down[0, :, 1] = [1.0, 1e8, -1e8]     # (1 + 1e8) - 1e8 = 0
    down[0, :, 2] = [-1e8, 1e8, 1.0]     # 1
    down[0, :, 3] = [0.1, 0.2, 0.3]
    down[1] = np.random.default_rng(2).normal(0, 1e4, (k, d)).astype(np.float32)
    out = np.zeros(T * d, np.float32)
    oracle.or_moe_sum(P(down.reshape(-1).copy()), P(out), d, k, T)
    want = np.zeros((T, d), np.float32)
    for t in range(T):
        for j in range(k):
            want[t] = (want[t] + down[t, j]).astype(np.float32)
    assert np.array_equal(out.reshape(T, d).view(np.uint32), want.view(np.uint32))
    assert out[0] == 0.0 and out[2] == 1.0


# ---------------------------------------------------------------- hc_expand
def _hc_inputs(rng, T, n_hc, n, mix, dyadic):
    if dyadic:  # multiples of 1/8 in [-4, 4]: every product and sum below is exact in f32
        g = lambda *s: (rng.integers(-32, 33, s) / 8.0).astype(np.float32)
    else:
        g = lambda *s: rng.normal(0, 1, s).astype(np.float32)
    return g(T, n), g(T, n), g(T, n_hc, n), g(T, mix)


@pytest.mark.parametrize("n_hc,has_add", [(4, 1), (4, 0), (3, 1), (1, 1)])
def test_hc_expand_closed_form(oracle, n_hc, has_add):
    """Exact in f32 on dyadic inputs, so the oracle must equal the float64
    formula of hc.rs:212-259 bit for bit; comb is not symmetric, so a
    transposed comb index (src + dst*n_hc) fails, as does a post/comb offset
    off by n_hc or a dropped block_add."""
    rng = np.random.default_rng(40 + n_hc)
    T, n = 3, 40
    mix = 2 * n_hc + n_hc * n_hc + 2  # the reference's row stride may exceed the split
    bo, ba, res, split = _hc_inputs(rng, T, n_hc, n, mix, True)
    got = oracle_ref.hc_expand(bo, ba, res, split, n, n_hc, T, mix, has_add)
    want = np.zeros((T, n_hc, n))
    for t in range(T):
        v = bo[t].astype(np.float64) + (ba[t] if has_add else 0)
        post = split[t, n_hc:2 * n_hc].astype(np.float64)
        comb = split[t, 2 * n_hc:2 * n_hc + n_hc * n_hc].astype(np.float64).reshape(n_hc, n_hc)  # [src][dst]
        for dst in range(n_hc):
            want[t, dst] = v * post[dst] + comb[:, dst] @ res[t].astype(np.float64)
    assert np.array_equal(got.astype(np.float64), want)
    if n_hc > 1:
        assert not np.allclose(comb, comb.T)


def test_hc_expand_float64_and_order(oracle):
    """Random normal inputs: within f32 rounding of the float64 formula, and
    bit-equal to a numpy f32 evaluation in the reference's order."""
    rng = np.random.default_rng(9)
    T, n_hc, n, mix = 2, 4, 4096, 24
    bo, ba, res, split = _hc_inputs(rng, T, n_hc, n, mix, False)
    got = oracle_ref.hc_expand(bo, ba, res, split, n, n_hc, T, mix, 1)
    f = np.float32
    want = np.zeros((T, n_hc, n), np.float32)
    for t in range(T):
        v = (bo[t] + ba[t]).astype(f)
        for dst in range(n_hc):
            acc = (v * split[t, n_hc + dst]).astype(f)
            for src in range(n_hc):
                acc = (acc + (split[t, 2 * n_hc + dst + src * n_hc] * res[t, src]).astype(f)).astype(f)
            want[t, dst] = acc
            w64 = (bo[t].astype(np.float64) + ba[t]) * split[t, n_hc + dst] + sum(
                float(split[t, 2 * n_hc + dst + s * n_hc]) * res[t, s].astype(np.float64) for s in range(n_hc))
            assert np.max(np.abs(got[t, dst] - w64)) < 1e-5 * (1 + np.max(np.abs(w64)))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- hash routing
def test_router_select_hash_restated(oracle):
    """or_router_select_hash against a plain restatement of moe.rs:92-109
    and the weight normalisation :143-159: tokens outside the table and
    negative tokens use row 0, ids outside [0, E) weigh 0, a token array of
    None uses the scalar token, and the weights sum to route_scale."""
    rng = np.random.default_rng(11)
    E, k, rows, T = 32, 4, 10, 9
    logits = rng.normal(0, 2, (T, E)).astype(np.float32)
    table = rng.integers(0, E, (rows, k)).astype(np.int32)
    table[3, 1] = -1
    table[4, 2] = E + 3
    tokens = np.array([0, 3, 4, 9, 10, -5, 2**31 - 1, 7, 4], np.int32)
    cfg = _Cfg(E, k, scale=2.5)
    probs, sel, w = oracle_ref.router_select_hash(cfg, logits, table, rows, tokens, 0, T)
    p_ref, _, _ = oracle_ref.router_select(cfg, logits, None, T)
    assert np.array_equal(probs.view(np.uint32), p_ref.view(np.uint32))
    for t in range(T):
        tok = tokens[t] if 0 <= tokens[t] < rows else 0
        assert list(sel[t]) == list(table[tok])
        v = [np.float32(probs[t, e]) if 0 <= e < E else np.float32(0) for e in table[tok]]
        s = np.float32(0)
        for x in v:
            s = np.float32(s + x)
        s = max(s, np.float32(6.103515625e-5))
        want = np.array([np.float32(x / np.float32(s / np.float32(2.5))) for x in v], np.float32)
        assert np.array_equal(w[t].view(np.uint32), want.view(np.uint32)), t
    assert w[1, 1] == 0 and w[2, 2] == 0
    ok = [t for t in range(T) if (sel[t] >= 0).all() and (sel[t] < E).all()]
    assert np.allclose(w[ok].sum(1), 2.5, rtol=1e-5)
    _, sel2, _ = oracle_ref.router_select_hash(cfg, logits, table, rows, None, 7, T)
    assert (sel2 == table[7]).all()


def test_router_select_hash_hand_computed(oracle):
    """Weights worked out by hand on a tiny table (moe.rs:92-159): logits
    above 20 are their own softplus, so logits 36, 64, 100 give
    probabilities exactly 6, 8, 10.  Token 1 picks experts (2, 5): sum 14,
    weights 6 / (14 / 2.5) and 8 / (14 / 2.5).  Token 2 is out of range and
    takes row 0 = (4, 1).  Row 3 holds an id of -1: it weighs 0 and the other
    id takes the whole route_scale.  A logit of -100 (exp branch) gives a
    probability of ~1e-22, far below the 2^-14 floor of the sum, so that row's
    weights are p / (2^-14 / 2.5)."""
    E, k, rows, T = 8, 2, 4, 4
    logits = np.zeros((T, E), np.float32)
    logits[:, 2], logits[:, 5], logits[:, 4], logits[:, 1] = 36.0, 64.0, 100.0, 0.0
    logits[:, 6], logits[:, 7] = -100.0, -100.0
    table = np.array([[4, 1], [2, 5], [6, 7], [-1, 4]], np.int32)
    tokens = np.array([1, 9, 3, 2], np.int32)
    probs, sel, w = oracle_ref.router_select_hash(_Cfg(E, k, scale=2.5), logits, table, rows, tokens, 0, T)
    assert sel.tolist() == [[2, 5], [4, 1], [-1, 4], [6, 7]]
    assert probs[0, 2] == 6.0 and probs[0, 5] == 8.0 and probs[0, 4] == 10.0
    assert abs(float(probs[0, 1]) - math.sqrt(math.log(2.0))) < 1e-6
    f = np.float32
    assert w[0].tolist() == [f(6) / (f(14) / f(2.5)), f(8) / (f(14) / f(2.5))]
    assert abs(w[0, 0] - 6 / 5.6) < 1e-6 and abs(w[0, 1] - 8 / 5.6) < 1e-6
    p1 = f(math.sqrt(math.log(2.0)))
    s = f(f(10) + probs[0, 1])
    assert np.allclose(w[1], [10 / (s / 2.5), p1 / (s / 2.5)], rtol=1e-6)
    assert w[2].tolist() == [0.0, 2.5]
    tiny = float(probs[0, 6])
    assert 0 < tiny < 1e-20
    floor = 2.0 ** -14
    assert np.allclose(w[3], [tiny / (floor / 2.5), float(probs[0, 7]) / (floor / 2.5)], rtol=1e-6)


def test_hc4_split_closed_forms(oracle):
    """hc4_split_one (hc.rs:17-99) on inputs whose result is known in closed
    form.  Pre/post: with mix = 1, base = 0 and scales (ln 3, -ln 3, .),
    pre = sigmoid(ln 3) + eps = 0.75 + eps and post = 2 sigmoid(-ln 3) = 0.5:
    each section takes its own scale.  Comb with uniform logits and eps = 0.5:
    every entry follows x <- x / (eps + 4 x), starting from the softmax entry
    plus eps, once for the initial column pass and twice per further round, so
    a misplaced eps or a wrong round count gives another number.  Comb with a
    permutation pattern (logit L at (r, pi(r)), 0 elsewhere) and eps = 0: the
    row softmax is already doubly stochastic, so every round leaves it as
    e^L / (e^L + 3) at (r, pi(r)) and 1 / (e^L + 3) elsewhere; pi is not an
    involution, so a transposed comb fails."""
    ln3 = math.log(3.0)
    mix = np.ones(24, np.float32)
    base = np.zeros(24, np.float32)
    scale = np.array([ln3, -ln3, 0.0], np.float32)
    for iters in (1, 2, 3, 7):
        eps = 0.5
        got = oracle_ref.hc4_split(mix, scale, base, iters, eps).astype(np.float64)
        assert np.allclose(got[:4], 0.75 + eps, atol=1e-6) and np.allclose(got[4:8], 0.5, atol=1e-6)
        x = 0.25 + eps
        x = x / (eps + 4 * x)
        for _ in range(iters - 1):
            x = x / (eps + 4 * x)
            x = x / (eps + 4 * x)
        assert np.allclose(got[8:], x, rtol=1e-6), (iters, got[8:], x)
    pi = [2, 0, 3, 1]
    L = 3.0
    m = np.zeros(24, np.float32)
    for r in range(4):
        m[8 + 4 * r + pi[r]] = L
    for iters in (1, 4, 20):
        got = oracle_ref.hc4_split(m, np.array([0, 0, 1], np.float32), base, iters, 0.0)
        assert np.array_equal(got[:8], np.array([0.5] * 4 + [1.0] * 4, np.float32))
        comb = got[8:].astype(np.float64).reshape(4, 4)
        want = np.full((4, 4), 1 / (math.exp(L) + 3))
        for r in range(4):
            want[r, pi[r]] = math.exp(L) / (math.exp(L) + 3)
        assert np.allclose(comb, want, rtol=2e-6), (iters, comb)
        assert not np.allclose(comb.T, want, rtol=1e-3)


# ---------------------------------------------------------------- HC FFN pre-norm
def test_rms_norm_plain_reference_tests(oracle):
    """engine/tests/kernels_smoke.rs:306-392: all-equal input gives
    all-equal output of RMS 1 (n = 256, eps 1e-5), and 1.0 and 3.0 inputs
    (n = 128) give the same output."""
    out = oracle_ref.rms_norm_plain(np.full(256, 2.0), 256, 1, 1e-5)[0]
    assert abs(math.sqrt(float(np.mean(out.astype(np.float64) ** 2))) - 1.0) < 1e-3
    assert np.all(out == out[0])
    a = oracle_ref.rms_norm_plain(np.full(128, 1.0), 128, 1, 1e-5)[0]
    b = oracle_ref.rms_norm_plain(np.full(128, 3.0), 128, 1, 1e-5)[0]
    assert abs(float(a[0]) - float(b[0])) < 1e-4


def test_rms_norm_plain_exact_and_float64(oracle):
    """eps = 0 and x = +-2 gives mean square 4, so every output is exactly
    +-1 (a dropped 1/n or a sqrt of the sum fails); random rows are within
    f32 rounding of the float64 formula, each row normalised by its own
    mean square (n = 1000 is not a multiple of 256)."""
    rng = np.random.default_rng(3)
    x = np.where(rng.random(512) < 0.5, -2.0, 2.0).astype(np.float32)
    assert np.array_equal(oracle_ref.rms_norm_plain(x, 512, 1, 0.0)[0], x / 2)
    for n in (1000, 16384):
        x = rng.normal(0, 3, (3, n)).astype(np.float32)
        x[1] *= 100
        got = oracle_ref.rms_norm_plain(x, n, 3, 1e-6).astype(np.float64)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 ** 2, axis=1, keepdims=True) + 1e-6)
        assert np.max(np.abs(got - want)) < 2e-6 * np.max(np.abs(want))


def _sinkhorn64(logits, iters, eps):
    """Float64 hc4_split_one comb (hc.rs:40-99): row softmax + eps, a
    column normalisation, then iters - 1 rounds of rows then columns, every
    normaliser starting at eps."""
    c = np.exp(logits - logits.max(axis=1, keepdims=True))
    c = c / c.sum(axis=1, keepdims=True) + eps
    c = c / (eps + c.sum(axis=0, keepdims=True))
    for _ in range(iters - 1):
        c = c / (eps + c.sum(axis=1, keepdims=True))
        c = c / (eps + c.sum(axis=0, keepdims=True))
    return c


@pytest.mark.parametrize("iters", [1, 2, 20])
def test_hc4_split_float64(oracle, iters):
    """pre = sigmoid + eps, post = 2 sigmoid and the Sinkhorn comb within
    f32 rounding of float64; after 20 iterations the comb is doubly
    stochastic to 1e-5; scale = 0 makes the split a function of base alone;
    swapping two rows of comb logits swaps the comb's rows."""
    rng = np.random.default_rng(iters)
    eps = 1e-6
    mix = rng.normal(0, 1, 24).astype(np.float32)
    scale = np.array([0.7, 1.3, 2.1], np.float32)
    base = rng.normal(0, 0.5, 24).astype(np.float32)
    got = oracle_ref.hc4_split(mix, scale, base, iters, eps).astype(np.float64)
    z = mix.astype(np.float64) * np.repeat(scale.astype(np.float64), [4, 4, 16]) + base
    sig = 1 / (1 + np.exp(-z[:8]))
    assert np.max(np.abs(got[:4] - (sig[:4] + eps))) < 1e-6
    assert np.max(np.abs(got[4:8] - 2 * sig[4:8])) < 2e-6
    comb = _sinkhorn64(z[8:].reshape(4, 4), iters, eps)
    assert np.max(np.abs(got[8:].reshape(4, 4) - comb)) < 1e-5 * iters
    if iters == 20:
        cm = got[8:].reshape(4, 4)
        assert np.max(np.abs(cm.sum(axis=0) - 1)) < 1e-5 and np.max(np.abs(cm.sum(axis=1) - 1)) < 1e-5
    a = oracle_ref.hc4_split(mix, np.zeros(3, np.float32), base, iters, eps)
    b = oracle_ref.hc4_split(rng.normal(0, 1, 24), np.zeros(3, np.float32), base, iters, eps)
    assert np.array_equal(a, b)
    sw = mix.copy()
    sw[8:12], sw[12:16] = mix[12:16], mix[8:12]
    bsw = base.copy()
    bsw[8:12], bsw[12:16] = base[12:16], base[8:12]
    c1 = oracle_ref.hc4_split(mix, scale, base, iters, eps)[8:].reshape(4, 4)
    c2 = oracle_ref.hc4_split(sw, scale, bsw, iters, eps)[8:].reshape(4, 4)
    assert np.max(np.abs(c1[[1, 0, 2, 3]] - c2)) < 1e-6


def test_hc_split_norm_float64(oracle):
    """hc_split_weighted_sum_norm_fused (hc.rs:313-398): split rows equal
    hc4_split of each mix row; ffn_cur = sum_h residual[h] * pre[h] within
    f32 rounding of float64 (weights pre, not post: the residual rows are
    scaled so that a swap changes the result); norm_out = ffn_cur times
    its rms scale times norm_w."""
    rng = np.random.default_rng(5)
    T, n = 3, 1000
    mix = rng.normal(0, 1, (T, 24)).astype(np.float32)
    scale = np.array([0.5, 1.0, 1.5], np.float32)
    base = rng.normal(0, 0.3, 24).astype(np.float32)
    res = (rng.normal(0, 1, (T, 4, n)) * np.array([1, 2, 3, 4])[None, :, None]).astype(np.float32)
    nw = rng.normal(1, 0.1, n).astype(np.float32)
    split, cur, nout = oracle_ref.hc_split_norm(mix, scale, base, res, nw, n, T, 20, 1e-6, 1e-6)
    for t in range(T):
        assert np.array_equal(split[t], oracle_ref.hc4_split(mix[t], scale, base, 20, 1e-6))
        c64 = np.einsum("h,hi->i", split[t, :4].astype(np.float64), res[t].astype(np.float64))
        assert np.max(np.abs(cur[t] - c64)) < 1e-5 * np.max(np.abs(c64))
        n64 = c64 / np.sqrt(np.mean(c64 ** 2) + 1e-6) * nw
        assert np.max(np.abs(nout[t] - n64)) < 2e-5 * np.max(np.abs(n64))
