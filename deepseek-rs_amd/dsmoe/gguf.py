"""GGUF files for the MoE tensors: the library's reader (dsmoe_gguf_*, a
restatement of engine/src/gguf.rs) behind a small Python class, and a writer
for GGUF v3 files with the tensors this path uses (synthetic layers for tests
and benchmarks; the layout of engine/tests/gguf_parse.rs's builder: header,
metadata, tensor infos, data from the next 32-byte boundary)."""
import ctypes
import struct

import numpy as np

from . import check, lib

F32, F16, Q8_0, Q2_K, Q4_K, IQ2_XXS, I32 = 0, 1, 8, 10, 12, 16, 26
MOE_TENSORS = ("ffn_gate_inp.weight", "exp_probs_b.bias", "ffn_gate_exps.weight", "ffn_up_exps.weight",
               "ffn_down_exps.weight", "ffn_gate_shexp.weight", "ffn_up_shexp.weight", "ffn_down_shexp.weight",
               "ffn_gate_tid2eid.weight", "ffn_norm.weight")
ERR_NOT_FOUND = 6


class Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("dims", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64),
                ("data", ctypes.c_void_p)]

    def info(self):
        return {"name": self.name.decode(), "type": self.type, "dims": list(self.dims[:self.n_dims]),
                "offset": self.offset, "bytes": self.bytes}

    def array(self):
        """The tensor's bytes (a copy) as uint8."""
        if not self.bytes:
            return np.zeros(0, np.uint8)
        return np.ctypeslib.as_array((ctypes.c_uint8 * self.bytes).from_address(self.data)).copy()


_SIGS = {
    "dsmoe_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)], ctypes.c_int),
    "dsmoe_gguf_close": ([ctypes.c_void_p], ctypes.c_int),
    "dsmoe_gguf_tensor_count": ([ctypes.c_void_p], ctypes.c_int64),
    "dsmoe_gguf_data_offset": ([ctypes.c_void_p], ctypes.c_uint64),
    "dsmoe_gguf_tensor_at": ([ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(Tensor)], ctypes.c_int),
    "dsmoe_gguf_find": ([ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(Tensor)], ctypes.c_int),
    "dsmoe_gguf_kv_u32": ([ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)], ctypes.c_int),
    "dsmoe_gguf_kv_i32_array": ([ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int64,
                                 ctypes.POINTER(ctypes.c_int64)], ctypes.c_int),
    "dsmoe_gguf_moe_layer": ([ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32)],
                             ctypes.c_int),
}


def _lib():
    L = lib()
    for n, (a, r) in _SIGS.items():
        f = getattr(L, n)
        f.argtypes, f.restype = a, r
    return L


class GgufFile:
    """A memory-mapped GGUF file (GgufFile, gguf.rs:11-190)."""

    def __init__(self, path):
        self._h = ctypes.c_void_p()
        check(_lib().dsmoe_gguf_open(str(path).encode(), ctypes.byref(self._h)))

    def close(self):
        if self._h:
            _lib().dsmoe_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def data_offset(self):
        return int(_lib().dsmoe_gguf_data_offset(self._h))

    @property
    def tensors(self):
        out = []
        for i in range(_lib().dsmoe_gguf_tensor_count(self._h)):
            t = Tensor()
            check(_lib().dsmoe_gguf_tensor_at(self._h, i, ctypes.byref(t)))
            out.append(t)
        return out

    def find(self, name):
        t = Tensor()
        rc = _lib().dsmoe_gguf_find(self._h, name.encode(), ctypes.byref(t))
        if rc == ERR_NOT_FOUND:
            return None
        check(rc)
        return t

    def read_kv_u32(self, key):
        v = ctypes.c_uint32()
        rc = _lib().dsmoe_gguf_kv_u32(self._h, key.encode(), ctypes.byref(v))
        if rc == ERR_NOT_FOUND:
            return None
        check(rc)
        return int(v.value)

    def read_kv_i32_array(self, key):
        n = ctypes.c_int64()
        rc = _lib().dsmoe_gguf_kv_i32_array(self._h, key.encode(), None, 0, ctypes.byref(n))
        if rc == ERR_NOT_FOUND:
            return []
        check(rc)
        out = np.zeros(n.value, np.int32)
        check(_lib().dsmoe_gguf_kv_i32_array(self._h, key.encode(), out.ctypes.data_as(ctypes.c_void_p), n.value,
                                             ctypes.byref(n)))
        return out.tolist()

    def moe_layer(self, layer):
        """{name: Tensor} of the layer's MoE tensors that are present."""
        arr = (Tensor * len(MOE_TENSORS))()
        present = ctypes.c_int32()
        check(_lib().dsmoe_gguf_moe_layer(self._h, layer, ctypes.cast(arr, ctypes.c_void_p), ctypes.byref(present)))
        return {n: arr[i] for i, n in enumerate(MOE_TENSORS) if present.value >> i & 1}


# ---------------------------------------------------------------------- writer
def _kv(key, value):
    b = struct.pack("<Q", len(key)) + key.encode()
    if isinstance(value, bool):
        return b + struct.pack("<IB", 7, int(value))
    if isinstance(value, int):
        return b + struct.pack("<II", 4, value)
    if isinstance(value, float):
        return b + struct.pack("<If", 6, value)
    if isinstance(value, str):
        return b + struct.pack("<IQ", 8, len(value)) + value.encode()
    if isinstance(value, (list, tuple)):  # i32 array
        return b + struct.pack("<IIQ", 9, 5, len(value)) + struct.pack(f"<{len(value)}i", *value)
    raise TypeError(f"unsupported metadata value for {key!r}")


def write(path, tensors, kv=None):
    """Writes a GGUF v3 file.  tensors: list of (name, type, dims, bytes-like
    data); each tensor's data is placed at the next 32-byte offset."""
    kv = kv or {}
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kv)) + b"".join(_kv(k, v) for k, v in kv.items())
    infos, blobs, off = [], [], 0
    for name, ty, dims, data in tensors:
        data = bytes(memoryview(data).cast("B"))
        infos.append(struct.pack("<Q", len(name)) + name.encode() + struct.pack("<I", len(dims))
                     + struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", ty, off))
        blobs.append((off, data))
        off = (off + len(data) + 31) // 32 * 32
    meta = head + b"".join(infos)
    meta += b"\0" * ((-len(meta)) % 32)
    body = bytearray(off)
    for o, d in blobs:
        body[o:o + len(d)] = d
    with open(path, "wb") as f:
        f.write(meta)
        f.write(body)


def moe_layer_tensors(cfg, w, layer=0):
    """The GGUF tensor list of one layer's MoE weights (engine.rs:175-187
    names, dims fastest-varying first as llama.cpp writes them) from a
    LayerWeights (device or host torch tensors)."""
    host = lambda t: t.detach().cpu().contiguous().numpy().view(np.uint8).reshape(-1)
    d, I, E, Is = cfg.d_model, cfg.d_ff, cfg.n_expert, cfg.d_ff_shared
    p = f"blk.{layer}."
    out = [(p + "ffn_gate_inp.weight", F16, [d, E], host(w.router_f16)),
           (p + "ffn_gate_exps.weight", IQ2_XXS, [d, I, E], host(w.gate)),
           (p + "ffn_up_exps.weight", IQ2_XXS, [d, I, E], host(w.up)),
           (p + "ffn_down_exps.weight", Q2_K, [I, d, E], host(w.down))]
    if w.bias is not None:
        out.append((p + "exp_probs_b.bias", F32, [E], host(w.bias)))
    if cfg.shared_fmt == 0:
        out += [(p + "ffn_gate_shexp.weight", Q8_0, [d, Is], host(w.sh_gate)),
                (p + "ffn_up_shexp.weight", Q8_0, [d, Is], host(w.sh_up)),
                (p + "ffn_down_shexp.weight", Q8_0, [Is, d], host(w.sh_down))]
    elif cfg.shared_fmt == 1:
        out += [(p + "ffn_gate_shexp.weight", IQ2_XXS, [d, Is], host(w.sh_gate)),
                (p + "ffn_up_shexp.weight", IQ2_XXS, [d, Is], host(w.sh_up)),
                (p + "ffn_down_shexp.weight", Q2_K, [Is, d], host(w.sh_down))]
    return out


def moe_layout(cfg):
    """GGUF type and dims of each MoE tensor of a layer of shape `cfg` (the
    layout moe_layer_tensors writes); the bias only when cfg.has_bias."""
    d, I, E, Is = cfg.d_model, cfg.d_ff, cfg.n_expert, cfg.d_ff_shared
    out = {"ffn_gate_inp.weight": (F16, [d, E]), "ffn_gate_exps.weight": (IQ2_XXS, [d, I, E]),
           "ffn_up_exps.weight": (IQ2_XXS, [d, I, E]), "ffn_down_exps.weight": (Q2_K, [I, d, E])}
    if cfg.has_bias:
        out["exp_probs_b.bias"] = (F32, [E])
    if cfg.shared_fmt in (0, 1):
        a, b = (Q8_0, Q8_0) if cfg.shared_fmt == 0 else (IQ2_XXS, Q2_K)
        out.update({"ffn_gate_shexp.weight": (a, [d, Is]), "ffn_up_shexp.weight": (a, [d, Is]),
                    "ffn_down_shexp.weight": (b, [Is, d])})
    return out


def layer_weights(g, layer, cfg, device="cuda"):
    """LayerWeights on `device` from a GgufFile's MoE tensors of `layer`,
    after checking every tensor the layer of shape `cfg` needs: present,
    of the type and dims the kernels read (a mismatch raises ValueError
    rather than running the layer on bytes of another shape)."""
    import torch
    from . import LayerWeights
    t = g.moe_layer(layer)
    for name, (ty, dims) in moe_layout(cfg).items():
        if name not in t:
            raise ValueError(f"blk.{layer}.{name}: missing")
        got = t[name]
        gd = list(got.dims[:got.n_dims])
        if got.type != ty or gd != dims:
            raise ValueError(f"blk.{layer}.{name}: type {got.type} dims {gd}, the layer needs type {ty} dims {dims}")
    up = lambda n: None if n not in t else torch.from_numpy(t[n].array()).to(device)
    return LayerWeights(up("ffn_gate_inp.weight"), None if "exp_probs_b.bias" not in t else
                        torch.from_numpy(t["exp_probs_b.bias"].array().view(np.float32)).to(device),
                        up("ffn_gate_exps.weight"), up("ffn_up_exps.weight"), up("ffn_down_exps.weight"),
                        up("ffn_gate_shexp.weight"), up("ffn_up_shexp.weight"), up("ffn_down_shexp.weight"))
