"""ctypes binding of the CPU parity oracle (liblfm_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
oracle restates the reference's CPU path (engine/src/q6k.rs, engine/src/lfm.rs,
engine/src/main.rs:112-141, engine/tests/dequant_mirror.rs); see lfm_oracle.h.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblfm_oracle.so")
MAX_LAYERS = 64


class OracleHparams(C.Structure):
    _fields_ = [
        ("dim", C.c_uint32), ("heads", C.c_uint32), ("head_dim", C.c_uint32),
        ("n_layers", C.c_uint32), ("kv_heads", C.c_uint32 * MAX_LAYERS),
        ("vocab", C.c_uint32), ("eps", C.c_float), ("rope_theta", C.c_float),
        ("eos", C.c_uint32), ("n_expert", C.c_uint32), ("n_used", C.c_uint32),
        ("expert_ff", C.c_uint32), ("n_ff", C.c_uint32), ("dense_lead", C.c_uint32),
        ("conv_l_cache", C.c_uint32),
    ]


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    P, u32, sz, f32 = C.c_void_p, C.c_uint32, C.c_size_t, C.c_float
    pf, pu32, pu8, pu64 = (C.POINTER(C.c_float), C.POINTER(C.c_uint32), C.POINTER(C.c_uint8),
                           C.POINTER(C.c_uint64))
    sig = {
        "oracle_f16_to_f32": (f32, [C.c_uint16]), "oracle_f32_to_f16": (C.c_uint16, [f32]),
        "oracle_f16_round": (f32, [f32]),
        "oracle_f32_to_f16_array": (None, [pf, C.POINTER(C.c_uint16), sz]),
        "oracle_q6k_dequant_block": (None, [pu8, pf]),
        "oracle_q6k_mirror_elem": (f32, [pu8, u32]),
        "oracle_q6k_dequant_row": (None, [pu8, sz, pf]),
        "oracle_q6k_matvec": (None, [pu8, sz, sz, pf, pf]),
        "oracle_q6k_repack_aligned": (None, [pu8, sz, pu8]),
        "oracle_argmax": (u32, [pf, sz]), "oracle_argmax_scalar": (u32, [pf, sz]),
        "oracle_route": (None, [pf, pf, u32, u32, pu32, pf, pf]),
        "oracle_powi": (f32, [f32, C.c_int]),
        "oracle_set_threads": (None, [C.c_int]), "oracle_get_threads": (C.c_int, []),
        "oracle_engine_create": (P, [C.POINTER(OracleHparams), u32, C.c_int]),
        "oracle_engine_destroy": (None, [P]),
        "oracle_engine_set_tensor": (C.c_int, [P, C.c_char_p, u32, pu64, u32, P, sz]),
        "oracle_engine_finalize": (C.c_int, [P]),
        "oracle_forward": (C.c_int, [P, pu32, u32, C.c_int64, pf]),
        "oracle_run_mixer": (C.c_int, [P, u32, pf, u32, C.c_int64]),
        "oracle_run_ffn": (C.c_int, [P, u32, pf, u32]),
        "oracle_head": (C.c_int, [P, pf, pf]),
        "oracle_embed": (C.c_int, [P, u32, pf]),
        "oracle_state_bytes": (sz, [P, u32]),
        "oracle_snapshot": (C.c_int, [P, u32, pu8, sz]),
        "oracle_restore": (C.c_int, [P, u32, pu8, sz]),
        "oracle_reset": (None, [P]),
        "oracle_last_route": (C.c_int, [P, u32, pu32, pf, pf]),
        "oracle_route_layer": (C.c_int, [P, u32, pf, pu32, pf, pf, pf]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _f(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _u8(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint8))


def set_threads(n: int):
    lib().oracle_set_threads(int(n))


def f32_to_f16_bits(x: float) -> int:
    return int(lib().oracle_f32_to_f16(x))


def f16_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(h))


def f32_to_f16_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_f(x), out.ctypes.data_as(C.POINTER(C.c_uint16)), x.size)
    return out


def dequant_block(block: np.ndarray) -> np.ndarray:
    block = np.ascontiguousarray(block, dtype=np.uint8)
    out = np.empty(256, dtype=np.float32)
    lib().oracle_q6k_dequant_block(_u8(block), _f(out))
    return out


def mirror_elem(block: np.ndarray, k: int) -> float:
    block = np.ascontiguousarray(block, dtype=np.uint8)
    return float(np.float32(lib().oracle_q6k_mirror_elem(_u8(block), k)))


def dequant_rows(raw: np.ndarray, rows: int, in_dim: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(rows * in_dim, dtype=np.float32)
    lib().oracle_q6k_dequant_row(_u8(raw), rows * in_dim, _f(out))
    return out.reshape(rows, in_dim)


def q6k_matvec(raw: np.ndarray, in_dim: int, out_dim: int, x: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(out_dim, dtype=np.float32)
    lib().oracle_q6k_matvec(_u8(raw), in_dim, out_dim, _f(x), _f(y))
    return y


def repack_aligned(raw: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(raw.size // 210 * 212, dtype=np.uint8)
    lib().oracle_q6k_repack_aligned(_u8(raw), raw.size, _u8(out))
    return out


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib().oracle_argmax(_f(v), v.size))


def argmax_scalar(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib().oracle_argmax_scalar(_f(v), v.size))


def route(logits: np.ndarray, bias: np.ndarray, n_used: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    sel = np.zeros(8, dtype=np.uint32)
    w = np.zeros(8, dtype=np.float32)
    scores = np.zeros(logits.size, dtype=np.float32)
    lib().oracle_route(_f(logits), _f(bias), logits.size, n_used,
                       sel.ctypes.data_as(C.POINTER(C.c_uint32)), _f(w), _f(scores))
    return [int(s) for s in sel[:n_used]], w[:n_used].copy(), scores


def powi(a: float, b: int) -> float:
    return float(np.float32(lib().oracle_powi(a, b)))


def to_oracle_hparams(hp) -> OracleHparams:
    o = OracleHparams()
    for name, _ in OracleHparams._fields_:
        if name == "kv_heads":
            for i in range(MAX_LAYERS):
                o.kv_heads[i] = hp.kv_heads[i]
        else:
            setattr(o, name, getattr(hp, name))
    return o


class OracleEngine:
    """The reference's CPU Engine (engine/src/lfm.rs:67-745), KV rounded to binary16."""

    def __init__(self, hp, ctx: int = 4096, kv_f16: bool = True):
        self.hp = hp
        self.ctx = ctx
        self._ohp = to_oracle_hparams(hp)
        self._e = lib().oracle_engine_create(C.byref(self._ohp), ctx, 1 if kv_f16 else 0)
        if not self._e:
            raise ValueError("oracle_engine_create failed")

    def set_tensor(self, name: str, ggml_type: int, shape: Sequence[int], data: np.ndarray):
        data = np.ascontiguousarray(data)
        ne = (C.c_uint64 * 4)(*([int(s) for s in shape] + [1] * (4 - len(shape))))
        rc = lib().oracle_engine_set_tensor(self._e, name.encode(), ggml_type, ne, len(shape),
                                            data.ctypes.data, data.nbytes)
        if rc:
            raise ValueError(f"set_tensor {name}: {rc}")

    def finalize(self):
        rc = lib().oracle_engine_finalize(self._e)
        if rc:
            raise ValueError(f"finalize: {rc}")

    def forward(self, ids: Sequence[int], start_pos: int) -> np.ndarray:
        ids_a = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(self.hp.vocab, dtype=np.float32)
        rc = lib().oracle_forward(self._e, ids_a.ctypes.data_as(C.POINTER(C.c_uint32)), ids_a.size,
                                  start_pos, _f(out))
        if rc:
            raise ValueError(f"forward: {rc}")
        return out

    def run_mixer(self, layer: int, x: np.ndarray, start_pos: int, n: int = 1) -> np.ndarray:
        xa = np.array(x, dtype=np.float32, copy=True)
        rc = lib().oracle_run_mixer(self._e, layer, _f(xa), n, start_pos)
        if rc:
            raise ValueError(f"run_mixer: {rc}")
        return xa

    def run_ffn(self, layer: int, x: np.ndarray, n: int = 1) -> np.ndarray:
        xa = np.array(x, dtype=np.float32, copy=True)
        rc = lib().oracle_run_ffn(self._e, layer, _f(xa), n)
        if rc:
            raise ValueError(f"run_ffn: {rc}")
        return xa

    def head(self, x: np.ndarray) -> np.ndarray:
        xa = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(self.hp.vocab, dtype=np.float32)
        rc = lib().oracle_head(self._e, _f(xa), _f(out))
        if rc:
            raise ValueError(f"head: {rc}")
        return out

    def embed(self, token: int) -> np.ndarray:
        out = np.empty(self.hp.dim, dtype=np.float32)
        rc = lib().oracle_embed(self._e, token, _f(out))
        if rc:
            raise ValueError(f"embed: {rc}")
        return out

    def state_bytes(self, valid: int) -> int:
        return int(lib().oracle_state_bytes(self._e, valid))

    def snapshot(self, valid: int) -> bytes:
        n = self.state_bytes(valid)
        buf = np.empty(n, dtype=np.uint8)
        rc = lib().oracle_snapshot(self._e, valid, _u8(buf), n)
        if rc:
            raise ValueError(f"snapshot: {rc}")
        return buf.tobytes()

    def restore(self, valid: int, data: bytes):
        a = np.frombuffer(data, dtype=np.uint8).copy()
        rc = lib().oracle_restore(self._e, valid, _u8(a), a.size)
        if rc:
            raise ValueError(f"restore: {rc}")

    def reset(self):
        lib().oracle_reset(self._e)

    def last_route(self, layer: int):
        ids = np.zeros(8, dtype=np.uint32)
        w = np.zeros(8, dtype=np.float32)
        scores = np.zeros(self.hp.n_expert, dtype=np.float32)
        lib().oracle_last_route(self._e, layer, ids.ctypes.data_as(C.POINTER(C.c_uint32)), _f(w),
                                _f(scores))
        return [int(i) for i in ids[: self.hp.n_used]], w[: self.hp.n_used].copy(), scores

    def route_layer(self, layer: int, x: np.ndarray):
        """Routing of residual x at MoE layer `layer` (ids, weights, scores, logits)."""
        xa = np.ascontiguousarray(x, dtype=np.float32)
        ids = np.zeros(8, dtype=np.uint32)
        w = np.zeros(8, dtype=np.float32)
        scores = np.zeros(self.hp.n_expert, dtype=np.float32)
        logits = np.zeros(self.hp.n_expert, dtype=np.float32)
        rc = lib().oracle_route_layer(self._e, layer, _f(xa), ids.ctypes.data_as(C.POINTER(C.c_uint32)),
                                      _f(w), _f(scores), _f(logits))
        if rc:
            raise ValueError(f"route_layer: {rc}")
        n = self.hp.n_used
        return [int(i) for i in ids[:n]], w[:n].copy(), scores, logits

    def close(self):
        if self._e:
            lib().oracle_engine_destroy(self._e)
            self._e = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
