"""Python mirror of the reference engine interface over the C ABI (include/lfm_hip.h).

The reference's callers use ``GpuEngine`` (Amidwestnoob/lfm2-w9100-rust
engine/src/gpu_lfm.rs:23-245, engine/src/gpu_lfm/resident_graph.rs:89-602) and
``GpuOps`` (engine/src/ops.rs).  This module keeps those names, argument
meanings and error behaviour (precondition failures raise ``LfmError`` where the
reference returns ``anyhow`` errors) on top of ``liblfm_hip.so``, whose HIP
kernels do all the work.  There is no CPU fallback: if the library or its gfx950
code object is missing, every call raises.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import weakref
from typing import Iterable, List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblfm_hip.so")
CODE_OBJECT_PATH = os.path.join(_HERE, "lfm_kernels.hsaco")

LFM_OK, LFM_EINVAL, LFM_ERANGE, LFM_EDEVICE, LFM_ESTATE, LFM_EINTERNAL, LFM_ENOTFOUND = range(7)
GGML_TYPE_F32 = 0
GGML_TYPE_Q6_K = 14
MAX_LAYERS = 64
MAX_CTX = 4096
QK_K = 256
Q6_K_BYTES = 210


class LfmError(RuntimeError):
    """A non-zero status from the C ABI; ``code`` is one of the LFM_E* values."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class Hparams(C.Structure):
    """``lfm_hparams``; mirrors Hyperparams (engine/src/lfm.rs:31-49)."""

    _fields_ = [
        ("dim", C.c_uint32), ("heads", C.c_uint32), ("head_dim", C.c_uint32),
        ("n_layers", C.c_uint32), ("kv_heads", C.c_uint32 * MAX_LAYERS),
        ("vocab", C.c_uint32), ("eps", C.c_float), ("rope_theta", C.c_float),
        ("eos", C.c_uint32), ("n_expert", C.c_uint32), ("n_used", C.c_uint32),
        ("expert_ff", C.c_uint32), ("n_ff", C.c_uint32), ("dense_lead", C.c_uint32),
        ("conv_l_cache", C.c_uint32),
    ]

    def kv_list(self) -> List[int]:
        return [int(self.kv_heads[i]) for i in range(self.n_layers)]


class TensorDesc(C.Structure):
    _fields_ = [
        ("name", C.c_char * 96), ("ggml_type", C.c_uint32), ("n_dims", C.c_uint32),
        ("ne", C.c_uint64 * 4), ("kind", C.c_uint32), ("sigma", C.c_float),
    ]

    @property
    def shape(self):
        return tuple(int(self.ne[i]) for i in range(self.n_dims))


class SynthOpts(C.Structure):
    _fields_ = [
        ("seed", C.c_uint64), ("d_sigma", C.c_float), ("norm_sigma", C.c_float),
        ("router_sigma", C.c_float), ("bias_sigma", C.c_float), ("conv_sigma", C.c_float),
        ("full_scales", C.c_uint32),
    ]


(GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL, GGUF_STRING,
 GGUF_ARRAY, GGUF_U64, GGUF_I64, GGUF_F64) = range(13)
GGUF_MAX_DIMS = 8


class GgufTensorInfo(C.Structure):
    """``lfm_gguf_tensor``: parser::gguf::TensorInfo (gguf.rs:58-70) with the
    absolute offset of model_file::TensorInfo (model_file.rs:7-14)."""

    _fields_ = [
        ("name", C.c_char_p), ("ggml_type", C.c_uint32), ("n_dims", C.c_uint32),
        ("ne", C.c_uint64 * GGUF_MAX_DIMS), ("offset", C.c_uint64), ("file_offset", C.c_uint64),
        ("nbytes", C.c_uint64),
    ]

    @property
    def shape(self):
        return tuple(int(self.ne[i]) for i in range(self.n_dims))


class GgufValue(C.Structure):
    _fields_ = [
        ("type", C.c_uint32), ("elem_type", C.c_uint32), ("u64", C.c_uint64), ("i64", C.c_int64),
        ("f64", C.c_double), ("str", C.c_void_p), ("len", C.c_uint64),
    ]


# Attention layers of the synthetic LFM2.5-8B-A1B-shaped model (18 conv + 6 GQA).
LFM2_ATTENTION_LAYERS = (2, 6, 10, 14, 18, 21)


def make_hparams(dim=2048, heads=32, n_layers=24, attention_layers=LFM2_ATTENTION_LAYERS,
                 kv=8, vocab=65536, eps=1e-5, rope_theta=1e6, eos=124900, n_expert=32,
                 n_used=4, expert_ff=1792, n_ff=7168, dense_lead=2) -> Hparams:
    hp = Hparams()
    hp.dim, hp.heads, hp.head_dim, hp.n_layers = dim, heads, 64, n_layers
    for l in range(n_layers):
        hp.kv_heads[l] = kv if l in attention_layers else 0
    hp.vocab, hp.eps, hp.rope_theta, hp.eos = vocab, eps, rope_theta, eos
    hp.n_expert, hp.n_used, hp.expert_ff, hp.n_ff = n_expert, n_used, expert_ff, n_ff
    hp.dense_lead, hp.conv_l_cache = dense_lead, 3
    return hp


_lib = None


def lib():
    """Load liblfm_hip.so (raises if it or the gfx950 code object is missing)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH) or not os.path.exists(CODE_OBJECT_PATH):
        raise LfmError(LFM_EDEVICE, f"native library not built: {LIB_PATH} / {CODE_OBJECT_PATH}"
                       " (run __graft_entry__.build())")
    L = C.CDLL(LIB_PATH)
    P, u32, u64, i32, f32, sz = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int, C.c_float, C.c_size_t
    pu32, pf32, pu8 = C.POINTER(C.c_uint32), C.POINTER(C.c_float), C.POINTER(C.c_uint8)
    sig = {
        "lfm_last_error": (C.c_char_p, []), "lfm_version": (C.c_char_p, []),
        "lfm_device_count": (i32, [C.POINTER(i32)]),
        "lfm_engine_create": (i32, [C.POINTER(Hparams), i32, C.POINTER(P)]),
        "lfm_engine_upload_tensor": (i32, [P, C.c_char_p, u32, C.POINTER(u64), u32, P, sz]),
        "lfm_engine_finalize": (i32, [P]), "lfm_engine_set_ctx": (i32, [P, u32]),
        "lfm_engine_destroy": (None, [P]), "lfm_engine_hparams": (i32, [P, C.POINTER(Hparams)]),
        "lfm_forward_logits": (i32, [P, pu32, u32, u32, pf32, sz]),
        "lfm_forward_token": (i32, [P, pu32, u32, u32, pu32, pf32]),
        "lfm_decode_run": (i32, [P, u32, u32, u32, u32, pu32, pu32]),
        "lfm_reset_session": (i32, [P]),
        "lfm_snapshot_bytes": (i32, [P, u32, C.POINTER(sz)]),
        "lfm_snapshot_cache": (i32, [P, u32, pu8, sz, C.POINTER(sz)]),
        "lfm_restore_session": (i32, [P, u32, pu8, sz]),
        "lfm_snapshot_logits": (i32, [P, pf32, sz]),
        "lfm_dispatch_count": (u64, [P]), "lfm_device_name": (i32, [P, C.c_char_p, sz]),
        "lfm_engine_set_prefill_mode": (i32, [P, i32]), "lfm_engine_h16_bytes": (i32, [P, C.POINTER(u64)]),
        "lfm_copy_time": (i32, [u64, u32, pf32]),
        "lfm_engine_run_mixer": (i32, [P, u32, pf32, u32]),
        "lfm_engine_run_ffn": (i32, [P, u32, pf32]),
        "lfm_engine_last_route": (i32, [P, pu32, pf32, u32]),
        "lfm_engine_run_layer": (i32, [P, u32, pf32, u32, pf32]),
        "lfm_engine_fused_router": (i32, [P, u32, C.POINTER(C.c_int)]),
        "lfm_engine_route_records": (i32, [P, pu32, sz]),
        "lfm_engine_set_route_log": (i32, [P, i32]),
        "lfm_engine_prefill_routes": (i32, [P, u32, pu32, pu32, C.POINTER(C.c_int), pu32, pf32, pf32,
                                            sz]),
        "lfm_engine_time_moe_gateup": (i32, [P, u32, pf32, C.POINTER(u64)]),
        "lfm_engine_time_head": (i32, [P, u32, u32, pf32, C.POINTER(u64)]),
        "lfm_dev_alloc": (i32, [sz, C.POINTER(P)]), "lfm_dev_free": (i32, [P]),
        "lfm_memcpy_htod": (i32, [P, P, sz]), "lfm_memcpy_dtoh": (i32, [P, P, sz]),
        "lfm_dev_synchronize": (i32, []),
        "lfm_q6k_nbytes": (sz, [u64, u64]), "lfm_q6k_pack": (i32, [P, u64, u64, P]),
        "lfm_q6k_unpack": (i32, [P, u64, u64, P]),
        "lfm_q6k_dequant": (i32, [P, u64, u64, P, P]),
        "lfm_q6k_matvec": (i32, [P, u64, u64, P, P, P]),
        "lfm_q6k_matvec_time": (i32, [P, u32, u64, u64, P, P, u32, pf32]),
        "lfm_q6k_gemm": (i32, [P, u64, u64, P, u32, P, P]),
        "lfm_argmax": (i32, [P, u32, pu32, pf32]),
        "lfm_argmax_noalloc": (i32, [P, u32, pu32, pf32]),
        "lfm_synth_default_opts": (None, [C.POINTER(SynthOpts)]),
        "lfm_model_tensor_count": (i32, [C.POINTER(Hparams)]),
        "lfm_model_tensor_desc": (i32, [C.POINTER(Hparams), C.POINTER(SynthOpts), i32,
                                        C.POINTER(TensorDesc)]),
        "lfm_tensor_nbytes": (sz, [C.POINTER(TensorDesc)]),
        "lfm_synth_tensor": (i32, [C.POINTER(SynthOpts), C.POINTER(TensorDesc), P, sz, i32]),
        "lfm_synth_q6k_blocks": (i32, [u64, C.c_char_p, u64, f32, P, i32]),
        "lfm_synth_q6k_blocks_ex": (i32, [u64, C.c_char_p, u64, f32, i32, P, i32]),
        "lfm_synth_normal_f32": (i32, [u64, C.c_char_p, u64, f32, f32, P, i32]),
        "lfm_engine_load_synthetic": (i32, [P, C.POINTER(SynthOpts), i32]),
        "lfm_f32_to_f16": (C.c_uint16, [f32]), "lfm_f16_to_f32": (f32, [C.c_uint16]),
        "lfm_gguf_open": (i32, [C.c_char_p, C.POINTER(P)]),
        "lfm_gguf_parse_memory": (i32, [P, sz, C.POINTER(P)]),
        "lfm_gguf_close": (None, [P]),
        "lfm_gguf_header": (i32, [P, pu32, pu32, C.POINTER(u64), C.POINTER(u64), C.POINTER(u64)]),
        "lfm_gguf_meta_key": (i32, [P, u64, C.POINTER(C.c_char_p)]),
        "lfm_gguf_meta_get": (i32, [P, C.c_char_p, C.POINTER(GgufValue)]),
        "lfm_gguf_meta_array_get": (i32, [P, C.c_char_p, u64, C.POINTER(GgufValue)]),
        "lfm_gguf_meta_u32": (i32, [P, C.c_char_p, pu32]),
        "lfm_gguf_meta_f32": (i32, [P, C.c_char_p, pf32]),
        "lfm_gguf_meta_str": (i32, [P, C.c_char_p, C.c_char_p, sz, C.POINTER(sz)]),
        "lfm_gguf_meta_u32_array": (i32, [P, C.c_char_p, pu32, sz, C.POINTER(sz)]),
        "lfm_gguf_tensor_info": (i32, [P, u64, C.POINTER(GgufTensorInfo)]),
        "lfm_gguf_find_tensor": (i32, [P, C.c_char_p, C.POINTER(u64)]),
        "lfm_gguf_read_tensor": (i32, [P, C.c_char_p, P, sz]),
        "lfm_gguf_read_tensor_range": (i32, [P, C.c_char_p, u64, P, u64]),
        "lfm_gguf_hparams": (i32, [P, i32, C.POINTER(Hparams)]),
        "lfm_engine_load_gguf": (i32, [P, P]),
        "lfm_engine_open_gguf": (i32, [C.c_char_p, i32, u32, i32, C.POINTER(P)]),
        "lfm_gguf_writer_create": (i32, [C.POINTER(P)]),
        "lfm_gguf_writer_free": (None, [P]),
        "lfm_gguf_writer_set_scalar": (i32, [P, C.c_char_p, u32, P]),
        "lfm_gguf_writer_set_string": (i32, [P, C.c_char_p, C.c_char_p, u64]),
        "lfm_gguf_writer_set_array": (i32, [P, C.c_char_p, u32, P, u64]),
        "lfm_gguf_writer_set_string_array": (i32, [P, C.c_char_p, C.POINTER(C.c_char_p),
                                                   C.POINTER(u64), u64]),
        "lfm_gguf_writer_set_hparams": (i32, [P, C.POINTER(Hparams)]),
        "lfm_gguf_writer_add_tensor": (i32, [P, C.c_char_p, u32, u32, C.POINTER(u64),
                                             C.POINTER(u64)]),
        "lfm_gguf_writer_begin": (i32, [P, C.c_char_p]),
        "lfm_gguf_writer_write_tensor": (i32, [P, u64, P, u64]),
        "lfm_gguf_writer_finish": (i32, [P]),
        "lfm_gguf_write_synthetic": (i32, [C.c_char_p, C.POINTER(Hparams), C.POINTER(SynthOpts),
                                           i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int):
    if rc != LFM_OK:
        raise LfmError(rc, lib().lfm_last_error().decode(errors="replace"))


def _u32p(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def _f32p(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def device_count() -> int:
    n = C.c_int(0)
    _check(lib().lfm_device_count(C.byref(n)))
    return n.value


# ------------------------------------------------------------------ synthetic model
def synth_opts(seed: int = 0x9E3779B97F4A7C15, bias_sigma: float = 0.0, **kw) -> SynthOpts:
    o = SynthOpts()
    lib().lfm_synth_default_opts(C.byref(o))
    o.seed = seed
    o.bias_sigma = bias_sigma
    for k, v in kw.items():
        setattr(o, k, v)
    return o


def model_tensor_descs(hp: Hparams, opts: Optional[SynthOpts] = None) -> List[TensorDesc]:
    n = lib().lfm_model_tensor_count(C.byref(hp))
    if n < 0:
        raise LfmError(LFM_EINVAL, "bad hparams")
    out = []
    for i in range(n):
        d = TensorDesc()
        _check(lib().lfm_model_tensor_desc(C.byref(hp), C.byref(opts) if opts else None, i, C.byref(d)))
        out.append(d)
    return out


def synth_tensor(desc: TensorDesc, opts: Optional[SynthOpts] = None, threads: int = 8) -> np.ndarray:
    """Seeded tensor content: uint8 raw GGUF bytes (Q6_K) or float32 values."""
    nb = lib().lfm_tensor_nbytes(C.byref(desc))
    buf = np.empty(nb, dtype=np.uint8)
    _check(lib().lfm_synth_tensor(C.byref(opts) if opts else None, C.byref(desc),
                                  buf.ctypes.data, nb, threads))
    return buf if desc.ggml_type == GGML_TYPE_Q6_K else buf.view(np.float32)


def synth_q6k_blocks(seed: int, stream: str, nblocks: int, d_sigma: float = 1e-3,
                     threads: int = 8, full_scales: bool = False) -> np.ndarray:
    out = np.empty(nblocks * Q6_K_BYTES, dtype=np.uint8)
    _check(lib().lfm_synth_q6k_blocks_ex(seed, stream.encode(), nblocks, d_sigma, int(full_scales),
                                         out.ctypes.data, threads))
    return out


def synth_normal(seed: int, stream: str, n: int, mean: float = 0.0, sigma: float = 1.0,
                 threads: int = 8) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _check(lib().lfm_synth_normal_f32(seed, stream.encode(), n, mean, sigma, out.ctypes.data,
                                      threads))
    return out


def f32_to_f16_bits(x: float) -> int:
    return int(lib().lfm_f32_to_f16(x))


# ------------------------------------------------------------------ GGUF files
_GGUF_SCALAR = {GGUF_U8: np.uint8, GGUF_I8: np.int8, GGUF_U16: np.uint16, GGUF_I16: np.int16,
                GGUF_U32: np.uint32, GGUF_I32: np.int32, GGUF_F32: np.float32,
                GGUF_BOOL: np.uint8, GGUF_U64: np.uint64, GGUF_I64: np.int64,
                GGUF_F64: np.float64}
_GGUF_UNSIGNED = (GGUF_U8, GGUF_U16, GGUF_U32, GGUF_U64)
_GGUF_SIGNED = (GGUF_I8, GGUF_I16, GGUF_I32, GGUF_I64)


def _gguf_scalar(v: GgufValue):
    if v.type in _GGUF_UNSIGNED:
        return int(v.u64)
    if v.type in _GGUF_SIGNED:
        return int(v.i64)
    if v.type == GGUF_BOOL:
        return bool(v.u64)
    if v.type in (GGUF_F32, GGUF_F64):
        return float(v.f64)
    if v.type == GGUF_STRING:
        return C.string_at(v.str, v.len).decode()
    raise LfmError(LFM_EINTERNAL, f"unexpected GGUF value type {v.type}")


class GgufFile:
    """A parsed GGUF v3 file: the reference's ModelFile (engine/src/model_file.rs:30-186)
    over parser::gguf::parse (parser/src/gguf.rs:299-440), parsed by the C++ reader."""

    def __init__(self, handle: C.c_void_p):
        self._g = handle
        ver, al = C.c_uint32(), C.c_uint32()
        off, nkv, nt = C.c_uint64(), C.c_uint64(), C.c_uint64()
        _check(lib().lfm_gguf_header(self._g, C.byref(ver), C.byref(al), C.byref(off),
                                     C.byref(nkv), C.byref(nt)))
        self.version, self.alignment, self.data_offset = ver.value, al.value, off.value
        self.n_kv, self.n_tensors = nkv.value, nt.value

    @classmethod
    def open(cls, path: str) -> "GgufFile":
        g = C.c_void_p()
        _check(lib().lfm_gguf_open(os.fsencode(path), C.byref(g)))
        return cls(g)

    @classmethod
    def parse(cls, data: bytes) -> "GgufFile":
        g = C.c_void_p()
        buf = C.create_string_buffer(bytes(data), len(data)) if data else None
        _check(lib().lfm_gguf_parse_memory(buf, len(data), C.byref(g)))
        return cls(g)

    def keys(self) -> List[str]:
        k = C.c_char_p()
        out = []
        for i in range(self.n_kv):
            _check(lib().lfm_gguf_meta_key(self._g, i, C.byref(k)))
            out.append(k.value.decode())
        return out

    def value_type(self, key: str) -> int:
        v = GgufValue()
        _check(lib().lfm_gguf_meta_get(self._g, key.encode(), C.byref(v)))
        return int(v.type)

    def get(self, key: str):
        """A metadata value as Python: int, float, bool, str or a list of those."""
        v = GgufValue()
        _check(lib().lfm_gguf_meta_get(self._g, key.encode(), C.byref(v)))
        if v.type != GGUF_ARRAY:
            return _gguf_scalar(v)
        return [self._element(key, i) for i in range(v.len)]

    def _element(self, key: str, i: int):
        e = GgufValue()
        _check(lib().lfm_gguf_meta_array_get(self._g, key.encode(), i, C.byref(e)))
        if e.type == GGUF_ARRAY:
            raise LfmError(LFM_EINVAL, f"{key}[{i}]: nested arrays are read with the C API")
        return _gguf_scalar(e)

    @property
    def metadata(self) -> dict:
        return {k: self.get(k) for k in self.keys()}

    def meta_u32(self, key: str) -> int:
        out = C.c_uint32()
        _check(lib().lfm_gguf_meta_u32(self._g, key.encode(), C.byref(out)))
        return out.value

    def meta_f32(self, key: str) -> float:
        out = C.c_float()
        _check(lib().lfm_gguf_meta_f32(self._g, key.encode(), C.byref(out)))
        return out.value

    def meta_str(self, key: str) -> str:
        n = C.c_size_t()
        rc = lib().lfm_gguf_meta_str(self._g, key.encode(), None, 0, C.byref(n))
        if rc not in (LFM_OK, LFM_ERANGE):
            _check(rc)
        buf = C.create_string_buffer(n.value + 1)
        _check(lib().lfm_gguf_meta_str(self._g, key.encode(), buf, n.value + 1, C.byref(n)))
        return buf.raw[:n.value].decode()

    def meta_u32_array(self, key: str) -> List[int]:
        n = C.c_size_t()
        rc = lib().lfm_gguf_meta_u32_array(self._g, key.encode(), None, 0, C.byref(n))
        if rc not in (LFM_OK, LFM_ERANGE):
            _check(rc)
        out = np.zeros(max(n.value, 1), dtype=np.uint32)
        _check(lib().lfm_gguf_meta_u32_array(self._g, key.encode(), _u32p(out), n.value,
                                             C.byref(n)))
        return [int(x) for x in out[:n.value]]

    def tensor_info(self, index: int) -> GgufTensorInfo:
        t = GgufTensorInfo()
        _check(lib().lfm_gguf_tensor_info(self._g, index, C.byref(t)))
        return t

    @property
    def tensors(self) -> List[GgufTensorInfo]:
        return [self.tensor_info(i) for i in range(self.n_tensors)]

    def tensor(self, name: str) -> GgufTensorInfo:
        i = C.c_uint64()
        _check(lib().lfm_gguf_find_tensor(self._g, name.encode(), C.byref(i)))
        return self.tensor_info(i.value)

    def has_tensor(self, name: str) -> bool:
        i = C.c_uint64()
        return lib().lfm_gguf_find_tensor(self._g, name.encode(), C.byref(i)) == LFM_OK

    def read_tensor(self, name: str) -> np.ndarray:
        """The tensor's raw bytes (read_tensor_into)."""
        out = np.empty(self.tensor(name).nbytes, dtype=np.uint8)
        _check(lib().lfm_gguf_read_tensor(self._g, name.encode(), out.ctypes.data, out.nbytes))
        return out

    def read_tensor_range(self, name: str, byte_off: int, length: int) -> np.ndarray:
        out = np.empty(length, dtype=np.uint8)
        _check(lib().lfm_gguf_read_tensor_range(self._g, name.encode(), byte_off,
                                                out.ctypes.data, length))
        return out

    def hparams(self, strict: bool = True) -> Hparams:
        """load_hyperparams (engine/src/lfm.rs:102-145)."""
        hp = Hparams()
        _check(lib().lfm_gguf_hparams(self._g, int(strict), C.byref(hp)))
        return hp

    def close(self):
        if self._g:
            lib().lfm_gguf_close(self._g)
            self._g = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GgufWriter:
    """Streaming GGUF v3 writer: metadata and tensor table, then ``begin(path)``,
    each tensor's bytes, then ``finish()``."""

    def __init__(self):
        self._w = C.c_void_p()
        _check(lib().lfm_gguf_writer_create(C.byref(self._w)))

    def set_scalar(self, key: str, type_: int, value):
        a = np.array([value], dtype=_GGUF_SCALAR[type_])
        _check(lib().lfm_gguf_writer_set_scalar(self._w, key.encode(), type_, a.ctypes.data))

    def set_string(self, key: str, value: str):
        b = value.encode()
        _check(lib().lfm_gguf_writer_set_string(self._w, key.encode(), b, len(b)))

    def set_array(self, key: str, elem_type: int, values):
        if elem_type == GGUF_STRING:
            bs = [v.encode() for v in values]
            arr = (C.c_char_p * max(len(bs), 1))(*bs)
            lens = (C.c_uint64 * max(len(bs), 1))(*[len(b) for b in bs])
            _check(lib().lfm_gguf_writer_set_string_array(self._w, key.encode(), arr, lens,
                                                          len(bs)))
            return
        a = np.ascontiguousarray(np.array(values, dtype=_GGUF_SCALAR[elem_type]))
        _check(lib().lfm_gguf_writer_set_array(self._w, key.encode(), elem_type, a.ctypes.data,
                                               a.size))

    def set_hparams(self, hp: Hparams):
        _check(lib().lfm_gguf_writer_set_hparams(self._w, C.byref(hp)))

    def add_tensor(self, name: str, ggml_type: int, shape: Sequence[int]) -> int:
        ne = (C.c_uint64 * GGUF_MAX_DIMS)(*[int(x) for x in shape])
        idx = C.c_uint64()
        _check(lib().lfm_gguf_writer_add_tensor(self._w, name.encode(), ggml_type, len(shape), ne,
                                                C.byref(idx)))
        return idx.value

    def begin(self, path: str):
        _check(lib().lfm_gguf_writer_begin(self._w, os.fsencode(path)))

    def write_tensor(self, index: int, data: np.ndarray):
        data = np.ascontiguousarray(data)
        _check(lib().lfm_gguf_writer_write_tensor(self._w, index, data.ctypes.data, data.nbytes))

    def finish(self):
        _check(lib().lfm_gguf_writer_finish(self._w))

    def close(self):
        if self._w:
            lib().lfm_gguf_writer_free(self._w)
            self._w = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def write_synthetic_gguf(path: str, hp: Hparams, opts: Optional[SynthOpts] = None,
                         threads: int = 8):
    """The seeded synthetic model as a GGUF file."""
    _check(lib().lfm_gguf_write_synthetic(os.fsencode(path), C.byref(hp),
                                          C.byref(opts) if opts else None, threads))


# ------------------------------------------------------------------ device buffers
# Engines and device buffers still open.  They are released at interpreter exit
# (atexit runs before module teardown), while the HIP runtime and any tool
# attached to it are still up, rather than by __del__ during teardown.
_LIVE = weakref.WeakSet()


@atexit.register
def _close_live_engines():
    for e in list(_LIVE):
        try:
            e.close()
        except Exception:
            pass


class DeviceBuffer:
    """Device memory owned by the library's HIP runtime (hipMalloc)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(lib().lfm_dev_alloc(self.nbytes, C.byref(p)))
        self.ptr = p.value
        _LIVE.add(self)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        _check(lib().lfm_memcpy_htod(b.ptr, a.ctypes.data, a.nbytes))
        return b

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        _check(lib().lfm_memcpy_htod(self.ptr + offset, a.ctypes.data, a.nbytes))

    def download(self, dtype, count: Optional[int] = None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else count
        out = np.empty(n, dtype=dt)
        _check(lib().lfm_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            _check(lib().lfm_dev_free(self.ptr))
            self.ptr = None
        _LIVE.discard(self)

    close = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------------------------ Q6_K operator API
def q6k_nbytes(rows: int, in_dim: int) -> int:
    return rows * (in_dim // QK_K) * Q6_K_BYTES


def q6k_pack(raw: np.ndarray, rows: int, in_dim: int) -> np.ndarray:
    """Raw GGUF Q6_K bytes -> the device plane layout (host to host)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    if raw.nbytes != q6k_nbytes(rows, in_dim):
        raise LfmError(LFM_EINVAL, "raw size does not match rows x in_dim")
    out = np.empty_like(raw)
    _check(lib().lfm_q6k_pack(raw.ctypes.data, rows, in_dim, out.ctypes.data))
    return out


def q6k_unpack(packed: np.ndarray, rows: int, in_dim: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty_like(packed)
    _check(lib().lfm_q6k_unpack(packed.ctypes.data, rows, in_dim, out.ctypes.data))
    return out


class Q6Weight:
    """A packed Q6_K tensor resident on the device (rows x in_dim)."""

    def __init__(self, raw: np.ndarray, rows: int, in_dim: int):
        self.rows, self.in_dim = rows, in_dim
        self.buf = DeviceBuffer.from_array(q6k_pack(raw, rows, in_dim))

    def dequant(self) -> np.ndarray:
        out = DeviceBuffer(self.rows * self.in_dim * 4)
        _check(lib().lfm_q6k_dequant(self.buf.ptr, self.rows, self.in_dim, out.ptr, None))
        return out.download(np.float32).reshape(self.rows, self.in_dim)

    def matvec(self, x: np.ndarray) -> np.ndarray:
        """GpuOps::q6k_matmul for one column (engine/src/ops.rs:340-374)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.shape != (self.in_dim,):
            raise LfmError(LFM_EINVAL, "x has the wrong length")
        xb = DeviceBuffer.from_array(x)
        yb = DeviceBuffer(self.rows * 4)
        _check(lib().lfm_q6k_matvec(self.buf.ptr, self.rows, self.in_dim, xb.ptr, yb.ptr, None))
        return yb.download(np.float32)


def q6k_gemm(w: "Q6Weight", x: np.ndarray) -> np.ndarray:
    """Prefill GEMM: y[t] = W x[t] for every row t of x [T][in_dim] (matrix cores)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    if x.ndim != 2 or x.shape[1] != w.in_dim:
        raise LfmError(LFM_EINVAL, "x must be [T][in_dim]")
    xb = DeviceBuffer.from_array(x)
    yb = DeviceBuffer(T * w.rows * 4)
    _check(lib().lfm_q6k_gemm(w.buf.ptr, w.rows, w.in_dim, xb.ptr, T, yb.ptr, None))
    return yb.download(np.float32).reshape(T, w.rows)


def q6k_matvec_time(weights: DeviceBuffer, ncopies: int, rows: int, in_dim: int,
                    x: DeviceBuffer, y: DeviceBuffer, iters: int) -> float:
    ms = C.c_float(0)
    _check(lib().lfm_q6k_matvec_time(weights.ptr, ncopies, rows, in_dim, x.ptr, y.ptr, iters,
                                     C.byref(ms)))
    return ms.value


def copy_time(nbytes: int, reps: int = 10) -> float:
    """Mean microseconds of a plain device copy of nbytes (read + write)."""
    us = C.c_float()
    _check(lib().lfm_copy_time(nbytes, reps, C.byref(us)))
    return us.value


def argmax(v: np.ndarray):
    """GPU greedy argmax (ties to the lowest id, NaN never wins) -> (index, value)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    b = DeviceBuffer.from_array(v)
    idx, val = C.c_uint32(0), C.c_float(0)
    _check(lib().lfm_argmax(b.ptr, v.size, C.byref(idx), C.byref(val)))
    return idx.value, val.value


def argmax_device(buf: "DeviceBuffer", n: int, noalloc: bool = False):
    """Argmax of n floats already on the device -> (index, value); noalloc uses
    the entry point that allocates nothing (lfm_argmax_noalloc)."""
    idx, val = C.c_uint32(0), C.c_float(0)
    fn = lib().lfm_argmax_noalloc if noalloc else lib().lfm_argmax
    _check(fn(buf.ptr, n, C.byref(idx), C.byref(val)))
    return idx.value, val.value


# ------------------------------------------------------------------ engine
class GpuEngine:
    """The reference's GpuEngine (engine/src/gpu_lfm.rs:23-245) on MI355X."""

    def __init__(self, hp: Hparams, device: int = 0, ctx: int = MAX_CTX):
        self._e = C.c_void_p()
        _check(lib().lfm_engine_create(C.byref(hp), device, C.byref(self._e)))
        _LIVE.add(self)
        self.hp = hp
        self.ctx = ctx
        _check(lib().lfm_engine_set_ctx(self._e, ctx))
        self._finalized = False

    # GpuEngine::load (gpu_lfm.rs:51-115), tensors supplied by the caller
    @classmethod
    def load(cls, hp: Hparams, tensors: Iterable, device: int = 0, ctx: int = MAX_CTX) -> "GpuEngine":
        e = cls(hp, device, ctx)
        for name, ggml_type, shape, data in tensors:
            e.upload_tensor(name, ggml_type, shape, data)
        e.finalize()
        return e

    @classmethod
    def load_synthetic(cls, hp: Hparams, opts: Optional[SynthOpts] = None, device: int = 0,
                       ctx: int = MAX_CTX, threads: int = 16) -> "GpuEngine":
        e = cls(hp, device, ctx)
        o = opts if opts is not None else synth_opts()
        _check(lib().lfm_engine_load_synthetic(e._e, C.byref(o), threads))
        e.finalize()
        return e

    @classmethod
    def from_gguf(cls, path: str, device: int = 0, ctx: int = MAX_CTX,
                  strict: bool = True) -> "GpuEngine":
        """ModelFile::open + GpuEngine::load (gpu_lfm.rs:51-120) in one call."""
        h = C.c_void_p()
        _check(lib().lfm_engine_open_gguf(os.fsencode(path), device, ctx, int(strict),
                                          C.byref(h)))
        e = cls.__new__(cls)
        e._e = h
        _LIVE.add(e)
        e.hp = Hparams()
        _check(lib().lfm_engine_hparams(h, C.byref(e.hp)))
        e.ctx = ctx
        e._finalized = True
        return e

    def load_gguf(self, f: GgufFile):
        """Upload every F32 and Q6_K tensor of an open file (before finalize)."""
        _check(lib().lfm_engine_load_gguf(self._e, f._g))

    def upload_tensor(self, name: str, ggml_type: int, shape: Sequence[int], data: np.ndarray):
        data = np.ascontiguousarray(data)
        ne = (C.c_uint64 * 4)(*([int(s) for s in shape] + [1] * (4 - len(shape))))
        _check(lib().lfm_engine_upload_tensor(self._e, name.encode(), ggml_type, ne, len(shape),
                                              data.ctypes.data, data.nbytes))

    def finalize(self):
        _check(lib().lfm_engine_finalize(self._e))
        self._finalized = True

    def set_ctx(self, ctx: int):
        _check(lib().lfm_engine_set_ctx(self._e, ctx))
        self.ctx = ctx

    def forward(self, ids: Sequence[int], start_pos: int) -> np.ndarray:
        ids_a = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(self.hp.vocab, dtype=np.float32)
        _check(lib().lfm_forward_logits(self._e, _u32p(ids_a), ids_a.size, start_pos, _f32p(out),
                                        out.size))
        return out

    def forward_token(self, ids: Sequence[int], position: int) -> int:
        ids_a = np.ascontiguousarray(ids, dtype=np.uint32)
        nxt, val = C.c_uint32(0), C.c_float(0)
        _check(lib().lfm_forward_token(self._e, _u32p(ids_a), ids_a.size, position, C.byref(nxt),
                                       C.byref(val)))
        self.last_max_logit = val.value
        return nxt.value

    def decode_run(self, first_token: int, start_pos: int, steps: int, eos: Optional[int] = None) -> List[int]:
        out = np.empty(max(steps, 1), dtype=np.uint32)
        n = C.c_uint32(0)
        e = self.hp.eos if eos is None else eos
        _check(lib().lfm_decode_run(self._e, first_token, start_pos, steps, e, _u32p(out), C.byref(n)))
        return [int(t) for t in out[: n.value]]

    def reset_session(self):
        _check(lib().lfm_reset_session(self._e))

    def snapshot_bytes(self, valid_tokens: int) -> int:
        n = C.c_size_t(0)
        _check(lib().lfm_snapshot_bytes(self._e, valid_tokens, C.byref(n)))
        return n.value

    def snapshot_resident_cache(self, valid_tokens: int) -> bytes:
        n = self.snapshot_bytes(valid_tokens)
        buf = np.empty(n, dtype=np.uint8)
        w = C.c_size_t(0)
        _check(lib().lfm_snapshot_cache(self._e, valid_tokens,
                                        buf.ctypes.data_as(C.POINTER(C.c_uint8)), n, C.byref(w)))
        return buf.tobytes()

    def restore_session(self, valid_tokens: int, data: bytes):
        a = np.frombuffer(data, dtype=np.uint8)
        _check(lib().lfm_restore_session(self._e, valid_tokens,
                                         a.ctypes.data_as(C.POINTER(C.c_uint8)), a.size))

    def snapshot_resident_logits(self) -> np.ndarray:
        out = np.empty(self.hp.vocab, dtype=np.float32)
        _check(lib().lfm_snapshot_logits(self._e, _f32p(out), out.size))
        return out

    def set_prefill_mode(self, stepwise: bool):
        """False: batched matrix-core prefill (default); True: one decode step per token."""
        _check(lib().lfm_engine_set_prefill_mode(self._e, 1 if stepwise else 0))

    def dispatch_count(self) -> int:
        return int(lib().lfm_dispatch_count(self._e))

    def h16_bytes(self) -> int:
        """lfm_engine_h16_bytes: device bytes of the binary16 GEMM weight copies."""
        n = C.c_uint64()
        _check(lib().lfm_engine_h16_bytes(self._e, C.byref(n)))
        return int(n.value)

    @property
    def device_name(self) -> str:
        buf = C.create_string_buffer(256)
        _check(lib().lfm_device_name(self._e, buf, 256))
        return buf.value.decode()

    # layer-level entry points (one decode-step half on a host residual vector)
    def run_mixer(self, layer: int, x: np.ndarray, pos: int) -> np.ndarray:
        xa = np.array(x, dtype=np.float32, copy=True)
        _check(lib().lfm_engine_run_mixer(self._e, layer, _f32p(xa), pos))
        return xa

    def run_ffn(self, layer: int, x: np.ndarray) -> np.ndarray:
        xa = np.array(x, dtype=np.float32, copy=True)
        _check(lib().lfm_engine_run_ffn(self._e, layer, _f32p(xa)))
        return xa

    def run_layer(self, layer: int, x: np.ndarray, pos: int):
        """One whole layer as the decode step runs it (fused router where the step
        fuses it): returns (x after the layer, x between mixer and FFN)."""
        xa = np.array(x, dtype=np.float32, copy=True)
        mid = np.empty_like(xa)
        _check(lib().lfm_engine_run_layer(self._e, layer, _f32p(xa), pos, _f32p(mid)))
        return xa, mid

    def fused_router(self, layer: int) -> bool:
        v = C.c_int(0)
        _check(lib().lfm_engine_fused_router(self._e, layer, C.byref(v)))
        return bool(v.value)

    def last_route(self):
        ids = np.zeros(8, dtype=np.uint32)
        w = np.zeros(8, dtype=np.float32)
        _check(lib().lfm_engine_last_route(self._e, _u32p(ids), _f32p(w), 8))
        return [int(i) for i in ids[: self.hp.n_used]], w[: self.hp.n_used].copy()

    ROUTE_REC_WORDS = 144

    def route_records(self):
        """The decode step's routing per layer: {layer: (ids, weights, logits,
        scores)} for the MoE layers, scores being the p + bias values the
        kernel ranked the experts by (lfm_engine_route_records)."""
        hp, W = self.hp, self.ROUTE_REC_WORDS
        words = np.zeros(hp.n_layers * W, dtype=np.uint32)
        _check(lib().lfm_engine_route_records(self._e, _u32p(words), words.size))
        out = {}
        for l in range(hp.dense_lead, hp.n_layers):
            r = words[l * W:(l + 1) * W]
            out[l] = ([int(i) for i in r[:hp.n_used]], r[8:8 + hp.n_used].view(np.float32).copy(),
                      r[16:16 + hp.n_expert].view(np.float32).copy(),
                      r[80:80 + hp.n_expert].view(np.float32).copy())
        return out

    def set_route_log(self, on: bool = True):
        """Keep the routing of later multi-token forwards (lfm_engine_set_route_log)."""
        _check(lib().lfm_engine_set_route_log(self._e, int(on)))

    def prefill_routes(self, layer: int):
        """Routing of layer `layer` in the last multi-token forward:
        (first row, ids [n][4], weights [n][4], logits [n][n_expert] or None)."""
        hp = self.hp
        first, n, has = C.c_uint32(0), C.c_uint32(0), C.c_int(0)
        cap = self.ctx
        ids = np.zeros(cap * 4, dtype=np.uint32)
        w = np.zeros(cap * 4, dtype=np.float32)
        lg = np.zeros(cap * hp.n_expert, dtype=np.float32)
        _check(lib().lfm_engine_prefill_routes(self._e, layer, C.byref(first), C.byref(n), C.byref(has),
                                               _u32p(ids), _f32p(w), _f32p(lg), cap))
        k = n.value
        return (first.value, ids[:k * 4].reshape(k, 4)[:, :hp.n_used].copy(),
                w[:k * 4].reshape(k, 4)[:, :hp.n_used].copy(),
                lg[:k * hp.n_expert].reshape(k, hp.n_expert).copy() if has.value else None)

    def time_moe_gateup(self, reps: int = 10):
        """(us per launch, algorithmic bytes per launch) of the routed gate/up kernel."""
        us, nb = C.c_float(0), C.c_uint64(0)
        _check(lib().lfm_engine_time_moe_gateup(self._e, reps, C.byref(us), C.byref(nb)))
        return us.value, nb.value


    def time_head(self, ncopies: int = 3, reps: int = 5):
        """Mean k_head duration (us) and its algorithmic bytes, over `ncopies`
        rotating copies of the embedding planes."""
        us, nb = C.c_float(0), C.c_uint64(0)
        _check(lib().lfm_engine_time_head(self._e, ncopies, reps, C.byref(us), C.byref(nb)))
        return us.value, nb.value
    def close(self):
        """lfm_engine_destroy: waits for the engine's stream, frees its buffers and graphs."""
        if self._e:
            lib().lfm_engine_destroy(self._e)
            self._e = None
        _LIVE.discard(self)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
