"""The C-ABI library loads and exports every symbol include/lfm_hip.h declares;
argument errors come back as status codes with messages (no GPU work here)."""
import ctypes as C
import os
import re

import numpy as np

from conftest import REPO


def declared_functions():
    text = open(os.path.join(REPO, "include", "lfm_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(lfm_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_every_declared_symbol_is_exported(lfm):
    L = lfm.lib()
    names = declared_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_code_object_present(lfm):
    assert os.path.getsize(lfm.CODE_OBJECT_PATH) > 1000
    with open(lfm.CODE_OBJECT_PATH, "rb") as f:
        head = f.read(24)
    assert head[:4] == b"\x7fELF" or head == b"__CLANG_OFFLOAD_BUNDLE__"


def test_argument_errors_are_status_codes(lfm):
    L = lfm.lib()
    assert L.lfm_q6k_pack(None, 1, 256, None) == lfm.LFM_EINVAL
    assert b"in_dim" in L.lfm_last_error()
    hp = lfm.make_hparams(dim=300)
    e = C.c_void_p()
    assert L.lfm_engine_create(C.byref(hp), 0, C.byref(e)) == lfm.LFM_EINVAL
    assert b"dim" in L.lfm_last_error()
    hp = lfm.make_hparams()
    hp.conv_l_cache = 4
    assert L.lfm_engine_create(C.byref(hp), 0, C.byref(e)) == lfm.LFM_EINVAL
    # 32-bit byte offsets into the binary16 activation copies bound T x in_dim; the
    # check comes before any device work (the pointers are never dereferenced)
    fake = C.c_void_p(256)
    assert L.lfm_q6k_gemm(fake, 64, 2048, fake, 1 << 20, fake, None) == lfm.LFM_EINVAL
    assert b"2 GiB" in L.lfm_last_error()
    hp = lfm.make_hparams()
    if lfm.device_count() == 0:
        assert L.lfm_engine_create(C.byref(hp), 0, C.byref(e)) == lfm.LFM_EDEVICE


def test_pack_unpack_roundtrip(lfm):
    raw = np.random.default_rng(0).integers(0, 256, size=7 * 210 * 3, dtype=np.uint8)
    packed = lfm.q6k_pack(raw, 3, 1792)
    assert not np.array_equal(packed, raw)
    assert np.array_equal(lfm.q6k_unpack(packed, 3, 1792), raw)
