"""ctypes binding of the CPU oracle (oracle/liboracle.so) for the tests.

The oracle is the checker, never the thing under test: nothing in the
shipped package imports this module."""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB = os.path.join(ORACLE_DIR, "build", "liboracle.so")


class OrConfig(ctypes.Structure):
    _fields_ = [
        ("d_model", ctypes.c_int32), ("d_ff", ctypes.c_int32), ("n_expert", ctypes.c_int32),
        ("top_k", ctypes.c_int32), ("n_group", ctypes.c_int32), ("topk_group", ctypes.c_int32),
        ("route_scale", ctypes.c_float), ("swiglu_clamp", ctypes.c_float), ("has_bias", ctypes.c_int32),
        ("shared_fmt", ctypes.c_int32), ("d_ff_shared", ctypes.c_int32),
    ]


def cfg_of(m):
    return OrConfig(m.d_model, m.d_ff, m.n_expert, m.top_k, m.n_group, m.topk_group, m.route_scale,
                    m.swiglu_clamp, int(m.has_bias), m.shared_fmt, m.d_ff_shared)


def P(a):
    """numpy array -> void* (None passes NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)  # keeps a reference to the array


_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    src = [os.path.join(ORACLE_DIR, f) for f in ("dsmoe_oracle.c", "dsmoe_oracle.h", "iq2xxs_grid.inc")]
    if not os.path.exists(LIB) or any(os.path.getmtime(s) > os.path.getmtime(LIB) for s in src):
        subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)
    L = ctypes.CDLL(LIB)
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_float
    sig = {
        "or_f16_to_f32": ([ctypes.c_uint16], f32),
        "or_expf": ([f32], f32), "or_logf": ([f32], f32), "or_softplus": ([f32], f32), "or_silu": ([f32], f32),
        "or_iq2_sign": ([ctypes.c_uint32], ctypes.c_uint8), "or_iq2_grid": ([ctypes.c_uint32], ctypes.c_uint64),
        "or_dot_iq2_xxs_q8k": ([vp, vp], f32), "or_iq2_xxs_bsum": ([vp, vp], i32),
        "or_dot_q2k_q8k": ([vp, vp], f32), "or_q2k_isum_summs": ([vp, vp, vp, vp], None),
        "or_q8k_quantize": ([vp, vp, i32, i32], None), "or_q8_0_quantize": ([vp, vp, vp, i32, i32], None),
        "or_router_logits": ([vp, vp, vp, i32, i32, i32, i32], None),
        "or_router_select": ([ctypes.POINTER(OrConfig), vp, vp, i32, vp, vp, vp], None),
        "or_q8_0_matvec": ([vp, vp, vp, vp, i32, i32, i32, i32], None),
        "or_swiglu": ([vp, vp, vp, i32, f32, f32], None),
        "or_gate_up_mid": ([vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, f32, i32], None),
        "or_down": ([vp, vp, vp, vp, i32, i32, i32, i32, i32], None),
        "or_moe_sum": ([vp, vp, i32, i32, i32], None),
        "or_router_select_hash": ([vp, vp, vp, i32, vp, i32, i32, vp, vp, vp], None),
        "or_rms_norm_plain": ([vp, vp, i32, i32, f32], None),
        "or_hc4_split": ([vp, vp, vp, i32, f32, vp], None),
        "or_hc_split_norm": ([vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, f32, f32], None),
        "or_hc_expand": ([vp, vp, vp, vp, vp, i32, i32, i32, i32, i32], None),
        "or_dispatch": ([vp, i32, i32, i32, vp, vp, vp, vp, vp, vp], None),
        "or_moe_forward": ([ctypes.POINTER(OrConfig), vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, vp, vp, vp, i32], i32),
    }
    for n, (a, r) in sig.items():
        f = getattr(L, n)
        f.argtypes = a
        f.restype = r
    _lib = L
    return L


# ---- numpy-level helpers -------------------------------------------------
def q8k_quantize(x, in_dim, rows):
    out = np.zeros(rows * (in_dim // 256) * 292, np.uint8)
    load().or_q8k_quantize(P(np.ascontiguousarray(x, np.float32)), P(out), in_dim, rows)
    return out


def q8_0_quantize(x, in_dim, rows):
    nb = (in_dim + 31) // 32
    xq = np.zeros(rows * nb * 32, np.int8)
    xs = np.zeros(rows * nb, np.float32)
    load().or_q8_0_quantize(P(np.ascontiguousarray(x, np.float32)), P(xq), P(xs), in_dim, rows)
    return xq, xs


def router_logits(w16, x, d, E, T, nthreads=8):
    out = np.zeros(T * E, np.float32)
    load().or_router_logits(P(w16), P(np.ascontiguousarray(x, np.float32)), P(out), d, E, T, nthreads)
    return out.reshape(T, E)


def router_select(mcfg, logits, bias, T):
    E, K = mcfg.n_expert, mcfg.top_k
    probs = np.zeros(T * E, np.float32)
    sel = np.zeros(T * K, np.int32)
    w = np.zeros(T * K, np.float32)
    c = cfg_of(mcfg)
    load().or_router_select(ctypes.byref(c), P(np.ascontiguousarray(logits, np.float32)),
                            P(None if bias is None else np.ascontiguousarray(bias, np.float32)), T, P(probs), P(sel), P(w))
    return probs.reshape(T, E), sel.reshape(T, K), w.reshape(T, K)


def router_select_hash(mcfg, logits, hash_table, hash_rows, tokens, token_scalar, T):
    E, K = mcfg.n_expert, mcfg.top_k
    probs = np.zeros(T * E, np.float32)
    sel = np.zeros(T * K, np.int32)
    w = np.zeros(T * K, np.float32)
    c = cfg_of(mcfg)
    load().or_router_select_hash(ctypes.byref(c), P(np.ascontiguousarray(logits, np.float32)),
                                 P(np.ascontiguousarray(hash_table, np.int32)), hash_rows,
                                 P(None if tokens is None else np.ascontiguousarray(tokens, np.int32)), token_scalar,
                                 T, P(probs), P(sel), P(w))
    return probs.reshape(T, E), sel.reshape(T, K), w.reshape(T, K)


def dispatch(sel, E, block_m):
    pairs = sel.size
    counts = np.zeros(E, np.uint32)
    offsets = np.zeros(E + 1, np.uint32)
    sp = np.zeros(max(pairs, 1), np.uint32)
    ntile = pairs // block_m + E + 1
    to = np.zeros(E + 1, np.uint32)
    te = np.zeros(ntile, np.uint32)
    ts = np.zeros(ntile, np.uint32)
    load().or_dispatch(P(np.ascontiguousarray(sel, np.int32)), pairs, E, block_m, P(counts), P(offsets), P(sp),
                       P(to), P(te), P(ts))
    return counts, offsets, sp[:pairs], to, te[:to[E]], ts[:to[E]]


def rms_norm_plain(x, n, rows, eps):
    out = np.zeros(rows * n, np.float32)
    load().or_rms_norm_plain(P(np.ascontiguousarray(x, np.float32)), P(out), n, rows, eps)
    return out.reshape(rows, n)


def hc4_split(mix, scale, base, iters, eps):
    out = np.zeros(24, np.float32)
    f = lambda a: np.ascontiguousarray(a, np.float32)
    load().or_hc4_split(P(f(mix)), P(f(scale)), P(f(base)), iters, eps, P(out))
    return out


def hc_split_norm(mix, scale, base, residual_hc, norm_w, n_embd, n_rows, iters, eps, norm_eps):
    f = lambda a: np.ascontiguousarray(a, np.float32)
    split = np.zeros(n_rows * 24, np.float32)
    out = np.zeros(n_rows * n_embd, np.float32)
    nout = np.zeros(n_rows * n_embd, np.float32)
    load().or_hc_split_norm(P(f(mix)), P(f(scale)), P(f(base)), P(f(residual_hc)), P(f(norm_w)), P(split), P(out),
                            P(nout), n_embd, n_rows, iters, eps, norm_eps)
    return split.reshape(n_rows, 24), out.reshape(n_rows, n_embd), nout.reshape(n_rows, n_embd)


def hc_expand(block_out, block_add, residual_hc, split, n_embd, n_hc, T, mix_hc, has_add):
    out = np.zeros(T * n_hc * n_embd, np.float32)
    f = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
    load().or_hc_expand(P(f(block_out)), P(f(block_add)), P(f(residual_hc)), P(f(split)), P(out), n_embd, n_hc, T,
                        mix_hc, int(has_add))
    return out.reshape(T, n_hc, n_embd)


def moe_forward(mcfg, w, x, T, nthreads=8):
    """w: dict of numpy arrays router (uint16), bias (f32 or None), gate, up, down, sh_gate, sh_up, sh_down (uint8)."""
    d, K = mcfg.d_model, mcfg.top_k
    so = np.zeros(T * d, np.float32)
    ro = np.zeros(T * d, np.float32)
    sel = np.zeros(T * K, np.int32)
    wt = np.zeros(T * K, np.float32)
    c = cfg_of(mcfg)
    rc = load().or_moe_forward(ctypes.byref(c), P(w["router"]), P(w.get("bias")), P(w["gate"]), P(w["up"]),
                               P(w["down"]), P(w.get("sh_gate")), P(w.get("sh_up")), P(w.get("sh_down")),
                               P(np.ascontiguousarray(x, np.float32)), T, P(so), P(ro), P(sel), P(wt), nthreads)
    assert rc == 0
    return so.reshape(T, d), ro.reshape(T, d), sel.reshape(T, K), wt.reshape(T, K)
