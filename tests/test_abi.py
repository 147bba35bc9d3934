"""CPU checks of the shipped C-ABI library: it loads, exports every entry
point include/dsmoe.h declares, and rejects bad shapes before launching
anything (the reference's anyhow errors, session.rs / engine.rs)."""
import ctypes
import os
import re

import pytest

import dsmoe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "dsmoe.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(dsmoe_[a-z0-9_]+)\s*\(", txt)))


def test_header_and_library_agree():
    L = dsmoe.lib()
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(L, s), s
    assert set(syms) == set(dsmoe.EXPORTED)


def test_code_object_built():
    assert os.path.getsize(dsmoe.CODE_OBJECT_PATH) > 10000
    blob = open(dsmoe.CODE_OBJECT_PATH, "rb").read()
    assert b"gfx950" in blob
    for k in ("dsmoe_prep", "dsmoe_up", "dsmoe_dn", "dsmoe_up_rows", "dsmoe_dn_rows", "dsmoe_midq",
              "dsmoe_router_select", "dsmoe_dispatch", "dsmoe_moe_sum", "dsmoe_swiglu", "dsmoe_synth"):
        assert k.encode() in blob
    gemm = os.path.join(os.path.dirname(dsmoe.CODE_OBJECT_PATH), "dsmoe_gemm.hsaco")
    blob = open(gemm, "rb").read()
    assert b"gfx950" in blob
    for k in ("dsmoe_gu_grouped", "dsmoe_dn_grouped", "dsmoe_q80_gemm", "dsmoe_q80_gemm_swiglu", "dsmoe_router_tile",
              "dsmoe_q80_gemm_j7", "dsmoe_q80_gemm_swiglu_j7", "dsmoe_q80_gemm_j2", "dsmoe_q80_gemm_swiglu_j2"):
        assert k.encode() in blob


def _cfg(**kw):
    c = dict(d_model=7168, d_ff=2048, n_expert=256, top_k=8, n_group=8, topk_group=4, route_scale=2.5,
             swiglu_clamp=10.0, has_bias=True, shared_fmt=0, d_ff_shared=2048)
    c.update(kw)
    return dsmoe.MoeConfig(**c)


@pytest.mark.parametrize("kw,code", [
    (dict(d_model=7000), 2), (dict(d_ff=1000), 1), (dict(top_k=0), 1), (dict(top_k=300), 1),
    (dict(n_group=7), 1), (dict(topk_group=9), 1), (dict(n_expert=2000, top_k=8, n_group=1), 2),
    (dict(shared_fmt=3), 1), (dict(d_ff_shared=100), 2), (dict(n_group=8, topk_group=1, top_k=33), 1),
])
def test_create_rejects_bad_config(kw, code):
    L = dsmoe.lib()
    ctx = ctypes.c_void_p()
    c = _cfg(**kw).c()
    assert L.dsmoe_create(ctypes.byref(c), 4, ctypes.byref(ctx)) == code
    assert L.dsmoe_last_error()
    assert not ctx.value


def test_stage_entry_points_validate_before_launch():
    L = dsmoe.lib()
    nul = ctypes.c_void_p(0)
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    assert L.dsmoe_router_logits(nul, fake, fake, 7168, 256, 1, nul) == 1
    assert L.dsmoe_q8k_quantize(fake, fake, 300, 1, nul) == 1
    assert L.dsmoe_gate_up_mid(fake, fake, fake, fake, fake, nul, nul, fake, 7168 + 256, 2048, 1, 8, 256, 10.0, nul) == 2
    assert L.dsmoe_gate_up_mid(ctypes.c_void_p(0x1004), fake, fake, fake, fake, nul, nul, fake, 7168, 2048, 1, 8, 256, 10.0, nul) == 1
    assert L.dsmoe_down(fake, fake, fake, nul, nul, 7168, 2048, 1, 8, 256, nul) == 1
    assert L.dsmoe_down(fake, fake, fake, nul, fake, 7168, 2000, 1, 8, 256, nul) == 1
    assert L.dsmoe_down(fake, fake, fake, nul, fake, 7168, 2048, 1, 8, 0, nul) == 1  # E < 1
    assert L.dsmoe_dispatch(fake, 10, 600, 16, fake, fake, fake, nul, nul, nul, nul) == 2
    assert L.dsmoe_q8_0_matvec(fake, fake, fake, fake, 100, 10, 1, nul) == 2
    c = _cfg(n_expert=2000).c()
    assert L.dsmoe_router_select(ctypes.byref(c), fake, fake, 1, nul, fake, fake, nul) == 2
    assert L.dsmoe_forward(nul, None, nul, 1, nul, nul, nul, nul, nul) == 1
    assert L.dsmoe_synth_tensor(fake, 0, 1, 1, 1, 4, 300, 4, 300, 1.0, nul) == 1


def test_tensor_bytes():
    assert dsmoe.tensor_bytes(dsmoe.FMT_IQ2_XXS, 256, 2048, 7168) == 256 * 2048 * 28 * 66
    assert dsmoe.tensor_bytes(dsmoe.FMT_Q2_K, 256, 7168, 2048) == 256 * 7168 * 8 * 84
    assert dsmoe.tensor_bytes(dsmoe.FMT_Q8_0, 1, 2048, 7168) == 2048 * 224 * 34
    c = _cfg()
    assert c.bytes_per_expert() == 12386304
    assert c.bytes_shared() == 46792704 and c.bytes_router() == 3670016
