"""The synthetic-weight encoders (host side): deterministic, valid codes,
and a quantisation error in the expected range for 2-bit / 8-bit formats."""
import numpy as np
import pytest

import dsmoe
import quant_ref as Q


def host(fmt, tid, n, rows, cols, **kw):
    return dsmoe.synth(fmt, 77, tid, n, rows, cols, device="cpu", **kw).numpy()


def test_normals_are_standard():
    x = host(dsmoe.FMT_F32, 1, 1, 64, 4096).reshape(-1)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    assert np.array_equal(x, host(dsmoe.FMT_F32, 1, 1, 64, 4096).reshape(-1))
    assert not np.array_equal(x, host(dsmoe.FMT_F32, 2, 1, 64, 4096).reshape(-1))


@pytest.mark.parametrize("fmt,dec,blk,lo,hi", [
    (dsmoe.FMT_IQ2_XXS, Q.dequant_iq2, 66, 0.2, 0.6),
    (dsmoe.FMT_Q2_K, Q.dequant_q2k, 84, 0.15, 0.5),
    (dsmoe.FMT_Q8_0, Q.dequant_q8_0, 34, 0.0, 0.02),
])
def test_encoders_round_trip(fmt, dec, blk, lo, hi):
    rows, cols = 32, 2048
    ref = host(dsmoe.FMT_F32, 9, 1, rows, cols).reshape(-1).astype(np.float64) * 0.02
    q = host(fmt, 9, 1, rows, cols, sigma=0.02)
    got = dec(q.reshape(-1, blk)).reshape(-1)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert lo <= rel <= hi, rel


def test_padding_is_zero():
    q = host(dsmoe.FMT_IQ2_XXS, 3, 2, 8, 512, rows_real=5, sigma=0.02).reshape(2, 8, 2, 66)
    vals = Q.dequant_iq2(q.reshape(-1, 66)).reshape(2, 8, 512)
    assert not vals[:, 5:].any() and vals[:, :5].any()
    # Q2_K groups are 16 wide; padding on a group boundary (1408 = 88 * 16 in C1) is exact zero
    d = host(dsmoe.FMT_Q2_K, 4, 1, 4, 512, cols_real=304, sigma=0.02)
    v = Q.dequant_q2k(d.reshape(-1, 84)).reshape(4, 512)
    assert not v[:, 304:].any() and v[:, :304].any()


def test_iq2_sign_parity_encodable():
    q = host(dsmoe.FMT_IQ2_XXS, 5, 1, 16, 1024, sigma=0.02)
    ref = host(dsmoe.FMT_F32, 5, 1, 16, 1024).reshape(-1)
    got = Q.dequant_iq2(q.reshape(-1, 66)).reshape(-1)
    # signs agree except where the parity fix flipped the smallest |x| of a group of 8
    bad = np.sign(got) != np.sign(ref)
    assert bad.reshape(-1, 8).sum(1).max() <= 1


def test_f16_to_f32_ftz_forms_agree(tmp_path):
    """The branch-free f16 -> f32 conversion of the batch router kernel
    against the branching one every other kernel uses, and both against
    numpy's exact widening with subnormals flushed: all 65536 inputs."""
    import os
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    inc = os.path.join(os.path.dirname(__file__), "..", "deepseek-rs_amd", "csrc")
    src = tmp_path / "ftz.cpp"
    src.write_text('#include <cstdio>\n#include "dsmoe_formats.h"\nusing namespace dsm;\n'
                   "int main() { for (unsigned h = 0; h < 65536; h++) { float a = f16_to_f32_ftz(h), "
                   "b = f16_to_f32_ftz_nb(h); unsigned ua, ub; __builtin_memcpy(&ua, &a, 4); "
                   '__builtin_memcpy(&ub, &b, 4); printf("%u %u\\n", ua, ub); } }\n')
    exe = tmp_path / "ftz"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", inc, str(src), "-o", str(exe)], check=True)
    out = np.array(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split(),
                   dtype=np.uint64).reshape(-1, 2).astype(np.uint32)
    assert np.array_equal(out[:, 0], out[:, 1])
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    sub = (h & 0x7C00) == 0
    want[sub] = np.where((h[sub] & 0x8000) != 0, np.float32(-0.0), np.float32(0.0))
    fin = (h & 0x7C00) != 0x7C00
    assert np.array_equal(out[fin, 0], want.view(np.uint32)[fin])
    # Inf / NaN: all-ones exponent, mantissa moved up 13 bits, payload kept
    nan = ~fin
    exp_bits = ((h[nan].astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | ((h[nan].astype(np.uint32) & 0x3FF) << 13)
    assert np.array_equal(out[nan, 0], exp_bits)


def test_c5logit_prior_enters_the_router_logits():
    """c5logit adds the Zipf prior to the logits themselves: router column 0
    holds f16(-s ln rank) and x[:, 0] = 1, so each expert's logit is its prior
    plus the product over the other columns; the correction bias carries no
    prior (c5 puts it there instead)."""
    from dataclasses import replace
    import oracle_ref as O
    from dsmoe import configs as C
    small = replace(C.C2_CFG, d_model=512, d_ff=256, n_expert=32, n_group=4, topk_group=2, d_ff_shared=256)
    base = C.CASES["c5logit"]
    case = replace(base, cfg=small, T=16, d_ff_real=256, d_ff_shared_real=256)
    w = C.make_weights(case, device="cpu")
    x = C.make_x(case, device="cpu").numpy()
    E, d = small.n_expert, small.d_model
    prior = C.zipf_bias(E, base.zipf, base.seed).astype(np.float16)
    router = w.router_f16.numpy().view(np.uint16).reshape(E, d)
    assert np.array_equal(router[:, 0], prior.view(np.uint16))
    assert (x[:, 0] == 1.0).all()
    plain = replace(case, zipf=0.0, zipf_logit=False)
    wp = C.make_weights(plain, device="cpu")
    assert np.array_equal(w.bias.numpy(), wp.bias.numpy())  # the bias is the plain N(0, 0.01) one
    lg = O.router_logits(router.reshape(-1).copy(), x, d, E, case.T, 1)
    x0 = x.copy()
    x0[:, 0] = 0.0
    lg0 = O.router_logits(router.reshape(-1).copy(), x0, d, E, case.T, 1)
    diff = (lg - lg0).reshape(case.T, E)
    assert np.allclose(diff, prior.astype(np.float32)[None, :], atol=1e-5)
    # the bias variant keeps the router and moves the prior into the bias
    wb = C.make_weights(replace(case, zipf_logit=False), device="cpu")
    assert np.allclose(wb.bias.numpy() - wp.bias.numpy(), C.zipf_bias(E, base.zipf, base.seed), atol=1e-6)
