"""Python host mirror of the dsmoe C ABI (include/dsmoe.h).

The reference drives its MoE layer from Rust (Session::decode_attn_out_and_ffn,
engine/src/session.rs:1894-2155) through per-kernel launchers.  This module
binds the same surface through ctypes so tests and the benchmark call the
shipped library exactly as a foreign host would.  torch is used only to own
device memory and streams; every computation runs in libdsmoe.so's HIP
kernels.  There is no CPU fallback: if the library or its code object is
missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG = os.path.dirname(_HERE)
LIB_DIR = os.path.join(_PKG, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libdsmoe.so")
CODE_OBJECT_PATH = os.path.join(LIB_DIR, "dsmoe_kernels.hsaco")

FMT_IQ2_XXS, FMT_Q2_K, FMT_Q8_0, FMT_F16, FMT_F32 = 0, 1, 2, 3, 4
IQ2XXS_BYTES, Q2K_BYTES, Q8K_BYTES, Q8_0_BYTES = 66, 84, 292, 34

EXPORTED = [
    "dsmoe_version", "dsmoe_last_error", "dsmoe_init", "dsmoe_create", "dsmoe_destroy",
    "dsmoe_scratch_bytes", "dsmoe_forward", "dsmoe_forward_noalloc", "dsmoe_hc_expand", "dsmoe_probe", "dsmoe_gate_up_mid_em", "dsmoe_down_em", "dsmoe_router_logits", "dsmoe_router_select",
    "dsmoe_q8k_quantize", "dsmoe_q8_0_quantize", "dsmoe_gate_up_mid", "dsmoe_down", "dsmoe_moe_sum",
    "dsmoe_q8_0_matvec", "dsmoe_swiglu", "dsmoe_dispatch", "dsmoe_tensor_bytes", "dsmoe_synth_tensor",
    "dsmoe_synth_tensor_host", "dsmoe_stage_name", "dsmoe_set_profiling", "dsmoe_profile_read",
    "dsmoe_q8k_quantize_h", "dsmoe_q8k_quantize_i8", "dsmoe_gate_up_mid_sorted", "dsmoe_down_sorted", "dsmoe_q8_0_quantize_h",
    "dsmoe_q8_0_gemm", "dsmoe_q8_0_unpack", "dsmoe_q8_0_gemm_unpacked",
    "dsmoe_gguf_open", "dsmoe_gguf_close", "dsmoe_gguf_tensor_count", "dsmoe_gguf_data_offset", "dsmoe_gguf_tensor_at",
    "dsmoe_gguf_find", "dsmoe_gguf_kv_u32", "dsmoe_gguf_kv_i32_array", "dsmoe_gguf_moe_layer",
    "dsmoe_router_select_hash", "dsmoe_set_hash_routing", "dsmoe_rms_norm_plain", "dsmoe_hc_split_norm",
]
GROUPED_TILE_M = 64  # DSMOE_GROUPED_TILE_M
STAGE_COUNT = 9


class DsmoeError(RuntimeError):
    pass


class Config(ctypes.Structure):
    _fields_ = [
        ("d_model", ctypes.c_int32), ("d_ff", ctypes.c_int32), ("n_expert", ctypes.c_int32),
        ("top_k", ctypes.c_int32), ("n_group", ctypes.c_int32), ("topk_group", ctypes.c_int32),
        ("route_scale", ctypes.c_float), ("swiglu_clamp", ctypes.c_float), ("has_bias", ctypes.c_int32),
        ("shared_fmt", ctypes.c_int32), ("d_ff_shared", ctypes.c_int32),
    ]


class Weights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("router_f16", "bias", "gate", "up", "down", "sh_gate", "sh_up", "sh_down")] + \
               [("sh_codes", ctypes.c_void_p * 3), ("sh_scales", ctypes.c_void_p * 3)]


_lib = None


def lib():
    """Load libdsmoe.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise DsmoeError(f"{LIB_PATH} not built; run `python deepseek-rs_amd/build.py`")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, f32, u64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_uint64
    sig = {
        "dsmoe_version": ([], ctypes.c_char_p),
        "dsmoe_last_error": ([], ctypes.c_char_p),
        "dsmoe_init": ([ctypes.c_char_p], i32),
        "dsmoe_create": ([ctypes.POINTER(Config), i32, ctypes.POINTER(vp)], i32),
        "dsmoe_destroy": ([vp], i32),
        "dsmoe_scratch_bytes": ([vp], ctypes.c_size_t),
        "dsmoe_forward": ([vp, ctypes.POINTER(Weights), vp, i32, vp, vp, vp, vp, vp], i32),
        "dsmoe_gate_up_mid_em": ([vp] * 10 + [i32, i32, i32, i32, i32, i32, f32, vp], i32),
        "dsmoe_down_em": ([vp] * 8 + [i32, i32, i32, i32, i32, vp], i32),
        "dsmoe_router_select_hash": ([ctypes.POINTER(Config), vp, vp, i32, vp, i32, i32, vp, vp, vp, vp], i32),
        "dsmoe_set_hash_routing": ([vp, vp, i32, vp], i32),
        "dsmoe_rms_norm_plain": ([vp, vp, i32, i32, f32, vp], i32),
        "dsmoe_hc_split_norm": ([vp] * 8 + [i32, i32, i32, i32, f32, f32, vp], i32),
        "dsmoe_probe": ([i32, vp, ctypes.c_size_t, ctypes.c_int64, vp, vp], i32),
        "dsmoe_hc_expand": ([vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp], i32),
        "dsmoe_forward_noalloc": ([ctypes.POINTER(Config), ctypes.POINTER(Weights), vp, i32, vp, vp, vp, vp, vp], i32),
        "dsmoe_router_logits": ([vp, vp, vp, i32, i32, i32, vp], i32),
        "dsmoe_router_select": ([ctypes.POINTER(Config), vp, vp, i32, vp, vp, vp, vp], i32),
        "dsmoe_q8k_quantize": ([vp, vp, i32, i32, vp], i32),
        "dsmoe_q8_0_quantize": ([vp, vp, vp, i32, i32, vp], i32),
        "dsmoe_q8k_quantize_h": ([vp, vp, vp, i32, i32, vp], i32),
        "dsmoe_gate_up_mid_sorted": ([vp] * 11 + [i32] * 5 + [f32, vp], i32),
        "dsmoe_down_sorted": ([vp] * 10 + [i32] * 4 + [vp], i32),
        "dsmoe_q8k_quantize_i8": ([vp, vp, vp, vp, i32, i32, vp], i32),
        "dsmoe_q8_0_quantize_h": ([vp, vp, vp, vp, i32, i32, vp], i32),
        "dsmoe_q8_0_gemm": ([vp, vp, vp, vp, vp, i32, i32, i32, f32, vp], i32),
        "dsmoe_q8_0_unpack": ([vp, i32, i32, vp, vp, vp], i32),
        "dsmoe_q8_0_gemm_unpacked": ([vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, f32, vp], i32),
        "dsmoe_gate_up_mid": ([vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, vp], i32),
        "dsmoe_down": ([vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp], i32),
        "dsmoe_moe_sum": ([vp, vp, i32, i32, i32, vp], i32),
        "dsmoe_q8_0_matvec": ([vp, vp, vp, vp, i32, i32, i32, vp], i32),
        "dsmoe_swiglu": ([vp, vp, vp, i32, f32, f32, vp], i32),
        "dsmoe_dispatch": ([vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp], i32),
        "dsmoe_tensor_bytes": ([i32, i64, i32, i32], ctypes.c_size_t),
        "dsmoe_stage_name": ([i32], ctypes.c_char_p),
        "dsmoe_set_profiling": ([vp, i32], i32),
        "dsmoe_profile_read": ([vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64), i32], i32),
        "dsmoe_synth_tensor": ([vp, i32, u64, u64, i64, i32, i32, i32, i32, f32, vp], i32),
        "dsmoe_synth_tensor_host": ([vp, i32, u64, u64, i64, i32, i32, i32, i32, f32, i32], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def check(rc):
    if rc != 0:
        raise DsmoeError(f"dsmoe error {rc}: {lib().dsmoe_last_error().decode()}")


def init():
    """Load the gfx950 code object on the current device."""
    check(lib().dsmoe_init(CODE_OBJECT_PATH.encode()))


# --------------------------------------------------------------------------
# configuration
# --------------------------------------------------------------------------
@dataclass
class MoeConfig:
    d_model: int
    d_ff: int
    n_expert: int
    top_k: int
    n_group: int = 1
    topk_group: int = 1
    route_scale: float = 1.5
    swiglu_clamp: float = 10.0
    has_bias: bool = False
    shared_fmt: int = 0  # 0 = Q8_0 (reference), 1 = IQ2_XXS/Q2_K, -1 = none
    d_ff_shared: int = 2048

    def c(self) -> Config:
        return Config(self.d_model, self.d_ff, self.n_expert, self.top_k, self.n_group, self.topk_group,
                      self.route_scale, self.swiglu_clamp, int(self.has_bias), self.shared_fmt, self.d_ff_shared)

    # GGUF byte sizes of one layer's tensors
    def bytes_gate(self):
        return self.n_expert * self.d_ff * (self.d_model // 256) * IQ2XXS_BYTES

    def bytes_down(self):
        return self.n_expert * self.d_model * (self.d_ff // 256) * Q2K_BYTES

    def bytes_per_expert(self):
        return (2 * self.d_ff * (self.d_model // 256) * IQ2XXS_BYTES
                + self.d_model * (self.d_ff // 256) * Q2K_BYTES)

    def bytes_shared(self):
        if self.shared_fmt == 0:
            return 3 * self.d_model * self.d_ff_shared // 32 * Q8_0_BYTES
        if self.shared_fmt == 1:
            return (2 * self.d_ff_shared * (self.d_model // 256) * IQ2XXS_BYTES
                    + self.d_model * (self.d_ff_shared // 256) * Q2K_BYTES)
        return 0

    def bytes_router(self):
        return self.n_expert * self.d_model * 2


def _p(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


# --------------------------------------------------------------------------
# synthetic tensors
# --------------------------------------------------------------------------
def tensor_bytes(fmt, n_mats, rows, cols):
    return int(lib().dsmoe_tensor_bytes(fmt, n_mats, rows, cols))


def synth(fmt, seed, tensor_id, n_mats, rows, cols, rows_real=None, cols_real=None, sigma=1.0, device="cuda"):
    """N(0, sigma) tensor [n_mats][rows][cols] quantized to `fmt` (uint8 bytes,
    or f16 bits as int16 / f32 for the plain formats)."""
    import torch
    rows_real = rows if rows_real is None else rows_real
    cols_real = cols if cols_real is None else cols_real
    nbytes = tensor_bytes(fmt, n_mats, rows, cols)
    if str(device).startswith("cpu"):
        out = torch.empty(nbytes, dtype=torch.uint8)
        check(lib().dsmoe_synth_tensor_host(_p(out), fmt, seed, tensor_id, n_mats, rows, cols, rows_real,
                                            cols_real, sigma, os.cpu_count() or 1))
    else:
        out = torch.empty(nbytes, dtype=torch.uint8, device=device)
        check(lib().dsmoe_synth_tensor(_p(out), fmt, seed, tensor_id, n_mats, rows, cols, rows_real,
                                       cols_real, sigma, _stream()))
    if fmt == FMT_F16:
        return out.view(torch.int16).view(n_mats, rows, cols) if n_mats > 1 else out.view(torch.int16).view(rows, cols)
    if fmt == FMT_F32:
        return out.view(torch.float32).view(n_mats, rows, cols) if n_mats > 1 else out.view(torch.float32).view(rows, cols)
    return out


# --------------------------------------------------------------------------
# per-kernel entry points (torch tensors in, results written in place)
# --------------------------------------------------------------------------
def router_logits(w_f16, x, out, d, E, T, stream=None):
    check(lib().dsmoe_router_logits(_p(w_f16), _p(x), _p(out), d, E, T, _stream(stream)))


def router_select(cfg: MoeConfig, logits, bias, T, probs, selected, weights, stream=None):
    c = cfg.c()
    check(lib().dsmoe_router_select(ctypes.byref(c), _p(logits), _p(bias), T, _p(probs), _p(selected),
                                    _p(weights), _stream(stream)))


def q8k_quantize(x, out, in_dim, rows, stream=None):
    check(lib().dsmoe_q8k_quantize(_p(x), _p(out), in_dim, rows, _stream(stream)))


def q8k_quantize_h(x, out, out_h, in_dim, rows, stream=None):
    check(lib().dsmoe_q8k_quantize_h(_p(x), _p(out), _p(out_h), in_dim, rows, _stream(stream)))


def gate_up_mid_sorted(gate, up, xh, xq, sorted_pairs, offsets, tile_offsets, tile_experts, tile_starts, weights,
                       mid_out, d, I, k, E, pairs, clamp, stream=None):
    check(lib().dsmoe_gate_up_mid_sorted(_p(gate), _p(up), _p(xh), _p(xq), _p(sorted_pairs), _p(offsets),
                                         _p(tile_offsets), _p(tile_experts), _p(tile_starts), _p(weights),
                                         _p(mid_out), d, I, k, E, pairs, clamp, _stream(stream)))


def q8k_quantize_i8(x, out, out_i8, bsum_h, in_dim, rows, stream=None):
    check(lib().dsmoe_q8k_quantize_i8(_p(x), _p(out), _p(out_i8), _p(bsum_h), in_dim, rows, _stream(stream)))


def down_sorted(w, m8, bsum_h, mq, sorted_pairs, offsets, tile_offsets, tile_experts, tile_starts, down_out, d, I,
                E, pairs, stream=None):
    check(lib().dsmoe_down_sorted(_p(w), _p(m8), _p(bsum_h), _p(mq), _p(sorted_pairs), _p(offsets),
                                  _p(tile_offsets), _p(tile_experts), _p(tile_starts), _p(down_out), d, I, E, pairs,
                                  _stream(stream)))


def q8_0_quantize_h(x, xq, xscale, out_h, in_dim, rows, stream=None):
    check(lib().dsmoe_q8_0_quantize_h(_p(x), _p(xq), _p(xscale), _p(out_h), in_dim, rows, _stream(stream)))


def q8_0_gemm(w0, w1, xh, xscale, out, in_dim, out_dim, T, clamp=0.0, stream=None):
    check(lib().dsmoe_q8_0_gemm(_p(w0), _p(w1), _p(xh), _p(xscale), _p(out), in_dim, out_dim, T, clamp,
                                _stream(stream)))


def q8_0_unpack(w, rows, in_dim, codes, scales, stream=None):
    """A Q8_0 matrix rewritten for q8_0_gemm_unpacked: codes f16 [rows * in_dim],
    scales f32 [rows * in_dim / 32]."""
    check(lib().dsmoe_q8_0_unpack(_p(w), rows, in_dim, _p(codes), _p(scales), _stream(stream)))


def q8_0_gemm_unpacked(w0h, w0s, w1h, w1s, xh, xscale, out, in_dim, out_dim, T, clamp=0.0, stream=None):
    """q8_0_gemm over unpacked matrices, blocks added in order (f32 rounding
    of the reference's sum order)."""
    check(lib().dsmoe_q8_0_gemm_unpacked(_p(w0h), _p(w0s), _p(w1h), _p(w1s), _p(xh), _p(xscale), _p(out), in_dim,
                                         out_dim, T, clamp, _stream(stream)))


def q8_0_quantize(x, xq, xscale, in_dim, rows, stream=None):
    check(lib().dsmoe_q8_0_quantize(_p(x), _p(xq), _p(xscale), in_dim, rows, _stream(stream)))


def gate_up_mid(gate, up, xq, selected, weights, gate_out, up_out, mid_out, d, I, T, k, E, clamp, stream=None):
    """moe_gate_up_mid_qwarp32 (moe.rs:622-715); E = experts in gate/up (ids outside [0, E) read expert 0)."""
    check(lib().dsmoe_gate_up_mid(_p(gate), _p(up), _p(xq), _p(selected), _p(weights), _p(gate_out),
                                  _p(up_out), _p(mid_out), d, I, T, k, E, clamp, _stream(stream)))


def down(w, midq, selected, down_out, out, d, I, T, k, E, stream=None):
    """moe_down_qwarp32 + moe_sum (moe.rs:821-866, 983-1005); E as for gate_up_mid."""
    check(lib().dsmoe_down(_p(w), _p(midq), _p(selected), _p(down_out), _p(out), d, I, T, k, E,
                           _stream(stream)))


def moe_sum(down_t, out, d, k, T, stream=None):
    check(lib().dsmoe_moe_sum(_p(down_t), _p(out), d, k, T, _stream(stream)))


def q8_0_matvec(w, xq, xscale, out, in_dim, out_dim, T, stream=None):
    check(lib().dsmoe_q8_0_matvec(_p(w), _p(xq), _p(xscale), _p(out), in_dim, out_dim, T, _stream(stream)))


def swiglu(gate, up, out, n, clamp, weight, stream=None):
    check(lib().dsmoe_swiglu(_p(gate), _p(up), _p(out), n, clamp, weight, _stream(stream)))


def dispatch(selected, pairs, E, block_m, counts, offsets, sorted_pairs, tile_offsets=None,
             tile_experts=None, tile_starts=None, stream=None):
    check(lib().dsmoe_dispatch(_p(selected), pairs, E, block_m, _p(counts), _p(offsets), _p(sorted_pairs),
                               _p(tile_offsets), _p(tile_experts), _p(tile_starts), _stream(stream)))


# --------------------------------------------------------------------------
# whole layer
# --------------------------------------------------------------------------
@dataclass
class LayerWeights:
    router_f16: object
    bias: object
    gate: object
    up: object
    down: object
    sh_gate: object = None
    sh_up: object = None
    sh_down: object = None
    sh_unpacked: object = None  # (codes gate, up, down; scales gate, up, down) from unpack_shared

    def c(self) -> Weights:
        w = Weights(*[(_p(getattr(self, n)).value or None) for n in
                      ("router_f16", "bias", "gate", "up", "down", "sh_gate", "sh_up", "sh_down")])
        if self.sh_unpacked is not None:
            for i in range(3):
                w.sh_codes[i] = _p(self.sh_unpacked[i]).value
                w.sh_scales[i] = _p(self.sh_unpacked[3 + i]).value
        return w

    def unpack_shared(self, cfg, stream=None):
        """Rewrite the Q8_0 shared expert once into the wide GEMM's operand
        layout (dsmoe_q8_0_unpack) and keep it with these weights: batches of
        1024 tokens and more then skip the per-call unpack.  The unpacked
        copies must be redone if the shared-expert bytes change."""
        import torch
        if cfg.shared_fmt != 0 or self.sh_gate is None:
            return self
        d, Is = cfg.d_model, cfg.d_ff_shared
        dev = self.sh_gate.device
        shapes = ((self.sh_gate, Is, d), (self.sh_up, Is, d), (self.sh_down, d, Is))
        codes = [torch.empty(r * c, dtype=torch.int16, device=dev) for _, r, c in shapes]
        scales = [torch.empty(r * c // 32, dtype=torch.float32, device=dev) for _, r, c in shapes]
        for (m, r, cdim), h, s in zip(shapes, codes, scales):
            check(lib().dsmoe_q8_0_unpack(_p(m), r, cdim, _p(h), _p(s), _stream(stream)))
        self.sh_unpacked = tuple(codes) + tuple(scales)
        return self


def hc_expand(block_out, block_add, residual_hc, split, out_hc, n_embd, n_hc, T, mix_hc, has_add, stream=None):
    """hc_expand (hc.rs:212-259): the residual merge after the layer."""
    check(lib().dsmoe_hc_expand(_p(block_out), _p(block_add), _p(residual_hc), _p(split), _p(out_hc), n_embd, n_hc, T,
                                mix_hc, int(has_add), _stream(stream)))


EM_TILE_M = 8


def gate_up_mid_em(gate, up, xq, sorted_pairs, offsets, tile_offsets, tile_experts, tile_starts, weights, mid_out,
                   d, I, k, E, pairs, clamp, block_m=EM_TILE_M, stream=None):
    """Expert-major gate/up/SwiGLU over pairs dispatched with block_m <= EM_TILE_M (moe.rs:721-815)."""
    check(lib().dsmoe_gate_up_mid_em(_p(gate), _p(up), _p(xq), _p(sorted_pairs), _p(offsets), _p(tile_offsets),
                                     _p(tile_experts), _p(tile_starts), _p(weights), _p(mid_out), d, I, k, E, pairs,
                                     block_m, clamp, _stream(stream)))


def down_em(w, mq, sorted_pairs, offsets, tile_offsets, tile_experts, tile_starts, down_out, d, I, E, pairs,
            block_m=EM_TILE_M, stream=None):
    """Expert-major down over pairs dispatched with block_m <= EM_TILE_M (moe.rs:871-916)."""
    check(lib().dsmoe_down_em(_p(w), _p(mq), _p(sorted_pairs), _p(offsets), _p(tile_offsets), _p(tile_experts),
                              _p(tile_starts), _p(down_out), d, I, E, pairs, block_m, _stream(stream)))


def router_select_hash(cfg, logits, hash_table, hash_rows, tokens, token_scalar, T, probs, selected, weights,
                       stream=None):
    """router_select with hash_mode = 1 (moe.rs:92-109): experts from the token-id table."""
    c = cfg.c()
    check(lib().dsmoe_router_select_hash(ctypes.byref(c), _p(logits), _p(hash_table), hash_rows, _p(tokens),
                                         token_scalar, T, _p(probs), _p(selected), _p(weights), _stream(stream)))


def rms_norm_plain(x, out, n, rows, eps, stream=None):
    """rms_norm_plain (norm.rs:14-63)."""
    check(lib().dsmoe_rms_norm_plain(_p(x), _p(out), n, rows, eps, _stream(stream)))


def hc_split_norm(mix, scale, base, residual_hc, norm_w, split, out, norm_out, n_embd, n_rows, iters, eps, norm_eps,
                  stream=None):
    """hc_split_weighted_sum_norm_fused (hc.rs:313-398), n_hc = 4."""
    check(lib().dsmoe_hc_split_norm(_p(mix), _p(scale), _p(base), _p(residual_hc), _p(norm_w), _p(split), _p(out),
                                    _p(norm_out), n_embd, 4, n_rows, iters, eps, norm_eps, _stream(stream)))


def hc_ffn_prenorm(hc, w_fn_f16, scale, base, norm_w, flat, mix, split, cur, norm, n_embd, T, iters=20, eps=1e-6,
                   norm_eps=1e-6, stream=None):
    """The FFN pre-norm chain of session.rs:1830-1892 for T rows of HC
    residual streams hc [T][4][n_embd]: rms_norm_plain -> matmul_f16 (24
    mix values per row) -> hc_split_weighted_sum_norm_fused; `norm` is the
    layer input."""
    rms_norm_plain(hc, flat, 4 * n_embd, T, norm_eps, stream)
    router_logits(w_fn_f16, flat, mix, 4 * n_embd, 24, T, stream)
    hc_split_norm(mix, scale, base, hc, norm_w, split, cur, norm, n_embd, T, iters, eps, norm_eps, stream)


def probe(kind, src, nbytes, iters, sink, stream=None):
    """dsmoe_probe: kind 0 = dense f16 MFMA loop, 1 = HBM read of nbytes of src."""
    check(lib().dsmoe_probe(int(kind), _p(src), int(nbytes), int(iters), _p(sink), _stream(stream)))


def forward_noalloc(cfg, w, x, shared_out, routed_out, selected=None, weights=None, stream=None):
    """dsmoe_forward_noalloc: one decode call (T <= 8) on the static device
    scratch, with no context and no allocation; calls that overlap on one GPU race."""
    c, wc = cfg.c(), w.c()
    check(lib().dsmoe_forward_noalloc(ctypes.byref(c), ctypes.byref(wc), _p(x), x.shape[0], _p(shared_out),
                                      _p(routed_out), _p(selected), _p(weights), _stream(stream)))


class MoeLayer:
    """One MoE FFN layer bound to a dsmoe context (the Session's MoE scratch)."""

    def __init__(self, cfg: MoeConfig, max_tokens: int):
        self.cfg = cfg
        self.max_tokens = max_tokens
        self._ctx = ctypes.c_void_p()
        c = cfg.c()
        check(lib().dsmoe_create(ctypes.byref(c), max_tokens, ctypes.byref(self._ctx)))

    def close(self):
        if self._ctx:
            lib().dsmoe_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def scratch_bytes(self):
        return int(lib().dsmoe_scratch_bytes(self._ctx))

    def set_hash_routing(self, hash_table=None, hash_rows=0, tokens=None):
        """Route later forwards by token id (hash_table [hash_rows][k], tokens [T]); None returns to top-k."""
        self._hash_keep = (hash_table, tokens)  # the device buffers must outlive the forwards
        check(lib().dsmoe_set_hash_routing(self._ctx, _p(hash_table), hash_rows, _p(tokens)))

    def set_profiling(self, on: bool):
        check(lib().dsmoe_set_profiling(self._ctx, int(on)))

    def profile_read(self, reset=True):
        """{stage name: (total ms, launches)} accumulated since the last reset."""
        ms = (ctypes.c_double * STAGE_COUNT)()
        n = (ctypes.c_int64 * STAGE_COUNT)()
        check(lib().dsmoe_profile_read(self._ctx, ms, n, int(reset)))
        return {lib().dsmoe_stage_name(i).decode(): (ms[i], n[i]) for i in range(STAGE_COUNT) if n[i]}

    def forward(self, w: LayerWeights, x, shared_out, routed_out, selected=None, weights=None, stream=None):
        T = x.shape[0]
        wc = w.c()
        check(lib().dsmoe_forward(self._ctx, ctypes.byref(wc), _p(x), T, _p(shared_out), _p(routed_out),
                                  _p(selected), _p(weights), _stream(stream)))
