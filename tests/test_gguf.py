"""GGUF v3 reader/writer (no GPU): the reference parser's own cases
(parser/src/gguf.rs:555-846), typed metadata access (engine/src/model_file.rs:131-182),
load_hyperparams (engine/src/lfm.rs:102-145) and writer round trips.

Files are built here byte by byte from the format (GGUF v3, little-endian), not
with the library's writer, so the reader and the writer are each checked against
an independent encoding."""
import os
import struct

import numpy as np
import pytest

import lfm_hip as L
from model_util import small_hparams

# ---------------------------------------------------------------- independent encoder
# value = (type id, python value); arrays are (9, (elem type id, [values]))
_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q",
        11: "<q", 12: "<d"}
_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
          9: (32, 36), 10: (256, 84), 11: (256, 112), 12: (256, 144), 13: (256, 176),
          14: (256, 210), 15: (256, 288)}


def enc_str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def enc_payload(t, v):
    if t == 8:
        return enc_str(v)
    if t == 9:
        et, vals = v
        return struct.pack("<IQ", et, len(vals)) + b"".join(enc_payload(et, x) for x in vals)
    return struct.pack(_FMT[t], v)


def nbytes_of(t, dims):
    be, bb = _BLOCK[t]
    n = 1
    for d in dims:
        n *= d
    return n // be * bb


def build(version=3, align=32, meta=(), tensors=(), tail=True):
    """meta: [(key, type, value)], tensors: [(name, dims, ggml_type, offset)].
    With tail=True the data section is zero-filled to cover every tensor."""
    b = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, t, v in meta:
        b += enc_str(k) + struct.pack("<I", t) + enc_payload(t, v)
    for name, dims, t, off in tensors:
        b += enc_str(name) + struct.pack("<I", len(dims))
        b += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", t, off)
    b += b"\0" * (-len(b) % align)
    if tail:
        end = max([off + nbytes_of(t, d) for _, d, t, off in tensors] + [0])
        b += b"\0" * end
    return b


def parse_err(data, match=None):
    with pytest.raises(L.LfmError) as ei:
        L.GgufFile.parse(data)
    assert ei.value.code == L.LFM_EINVAL
    if match:
        assert match in str(ei.value), str(ei.value)
    return str(ei.value)


def sparse_file(tmp_path, head, total, name="m.gguf"):
    """Header bytes followed by a hole up to `total` bytes (reads as zeros)."""
    p = str(tmp_path / name)
    with open(p, "wb") as f:
        f.write(head)
        f.truncate(total)
    return p


# ---------------------------------------------------------------- reference test cases
def test_tensor_sizes_known_answers(tmp_path):
    # test_compute_nbytes_{f32,f16,q6_k} (gguf.rs:596-624)
    cases = [("a", [2048], 0, 8192), ("b", [2048, 128000], 0, 1048576000), ("c", [0], 0, 0),
             ("d", [10, 0, 5], 0, 0), ("e", [2048], 1, 4096), ("f", [2048], 14, 1680),
             ("g", [2048, 128000], 14, 215040000)]
    tensors, off = [], 0
    for name, dims, t, _ in cases:
        tensors.append((name, dims, t, off))
        off += -(-nbytes_of(t, dims) // 32) * 32
    head = build(tensors=tensors, tail=False)
    p = sparse_file(tmp_path, head, len(head) + off)
    with L.GgufFile.open(p) as f:
        got = {t.name.decode(): int(t.nbytes) for t in f.tensors}
    assert got == {name: nb for name, _, _, nb in cases}


def test_block_table_is_the_reference_parsers(tmp_path):
    # ggml_type_block_info (gguf.rs:174-192): Q3_K takes 112 bytes and Q8_K 288 per
    # 256 elements there (ggml's structs: 110 and 292).  A drop-in reader sizes,
    # places and accepts tensors exactly as the reference does.
    tensors = [("q3", [512], 11, 0), ("q8", [256], 15, 224)]
    data = build(tensors=tensors)
    with L.GgufFile.parse(data) as f:
        assert f.tensor("q3").nbytes == 224 and f.tensor("q8").nbytes == 288
    # the same file one byte short of the reference's Q8_K size is out of bounds
    parse_err(data[:-1])


@pytest.mark.parametrize("dims,t", [([100], 14), ([10], 999), ([2**64 - 1, 2], 0)])
def test_tensor_size_errors(dims, t):
    # Q6_K element count not a multiple of 256, unknown type, overflowing dims
    parse_err(build(tensors=[("t", dims, t, 0)], tail=False))


def test_parse_minimal(tmp_path):
    # test_parse_minimal (gguf.rs:637-667): a 215 MB Q6_K tensor in a sparse file
    meta = [("general.architecture", 8, "test"), ("general.alignment", 4, 32)]
    tensors = [("tensor_a", [2048], 0, 0), ("tensor_b", [2048, 128000], 14, 8192)]
    head = build(meta=meta, tensors=tensors, tail=False)
    p = sparse_file(tmp_path, head, len(head) + 8192 + 215040000)
    with L.GgufFile.open(p) as f:
        assert (f.version, f.alignment, f.n_kv, f.n_tensors) == (3, 32, 2, 2)
        a, b = f.tensors
        assert (a.name, a.shape, a.ggml_type, a.nbytes) == (b"tensor_a", (2048,), 0, 8192)
        assert (b.name, b.shape, b.ggml_type, b.nbytes) == (b"tensor_b", (2048, 128000), 14,
                                                            215040000)
        assert b.file_offset == f.data_offset + 8192 and f.data_offset == len(head)
        assert f.data_offset % 32 == 0


def test_invalid_magic_and_version():
    parse_err(b"XXXX", "magic")
    parse_err(build(version=2), "version")


def test_invalid_alignment():
    parse_err(build(align=33, meta=[("general.alignment", 4, 33)]), "alignment")


def test_duplicates():
    parse_err(build(meta=[("key", 8, "a"), ("key", 8, "b")]), "duplicate metadata key")
    parse_err(build(tensors=[("t", [10], 0, 0), ("t", [20], 0, 64)]), "duplicate tensor")


def test_truncated_header():
    parse_err(b"GGUF\x03\x00\x00\x00", "truncated")
    full = build(meta=[("k", 8, "value")], tensors=[("t", [8], 0, 0)])
    for cut in range(len(full) - 32):
        parse_err(full[:cut])


def test_empty_tensor():
    with L.GgufFile.parse(build(tensors=[("empty", [0, 2048], 0, 0)])) as f:
        assert f.tensor("empty").nbytes == 0


@pytest.mark.parametrize("dims,t", [([0, 2048], 14), ([2048, 0], 14), ([0], 0)])
def test_empty_tensor_is_rejected_by_the_engine_loader(tmp_path, dims, t):
    # An empty tensor parses (test_empty_tensor) but the engine takes no zero
    # dimension: lfm_engine_open_gguf reports it before any device work (no
    # division by a zero row length, no device needed to see the error).
    meta = lfm_meta()
    p = str(tmp_path / "empty.gguf")
    with open(p, "wb") as fh:
        fh.write(build(meta=meta, tensors=[("blk.0.attn_norm.weight", [2048], 0, 0),
                                           ("token_embd.weight", dims, t, 8192)]))
    eng = L.C.c_void_p()
    rc = L.lib().lfm_engine_open_gguf(p.encode(), 0, 0, 1, L.C.byref(eng))
    assert rc == L.LFM_EINVAL, (rc, L.lib().lfm_last_error())
    assert b"dimension" in L.lib().lfm_last_error()
    assert not eng.value


def test_array_and_bool_metadata():
    meta = [("test.array", 9, (4, [1, 2, 3])), ("test.bool", 7, 1)]
    with L.GgufFile.parse(build(meta=meta)) as f:
        assert f.get("test.array") == [1, 2, 3]
        assert f.get("test.bool") is True
        assert f.value_type("test.bool") == L.GGUF_BOOL


def test_alignment_default_and_nondefault():
    with L.GgufFile.parse(build()) as f:
        assert f.alignment == 32
    with L.GgufFile.parse(build(align=64, meta=[("general.alignment", 4, 64)],
                                tensors=[("t", [3], 0, 0)])) as f:
        assert f.alignment == 64 and f.data_offset % 64 == 0
    # only a U32 value sets the alignment (gguf.rs:343-347)
    with L.GgufFile.parse(build(meta=[("general.alignment", 10, 64)])) as f:
        assert f.alignment == 32


def test_out_of_file_storage():
    # test_parse_out_of_file_storage (gguf.rs:783-804)
    parse_err(build(tensors=[("big", [1000000], 0, 0)], tail=False), "exceeds data size")
    # offset past the data section, and offset + nbytes overflowing
    parse_err(build(tensors=[("t", [4], 0, 4096)], tail=False), "exceeds data size")
    parse_err(build(tensors=[("t", [4], 0, 2**64 - 8)], tail=False))


def test_bad_metadata_values():
    parse_err(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + enc_str("k") + struct.pack("<I", 99),
              "unknown metadata value type")
    parse_err(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + enc_str("k") + struct.pack("<I", 7) +
              b"\x02", "BOOL")
    parse_err(build(meta=[("k", 8, b"\xff\xfe")]), "UTF-8")
    parse_err(build(meta=[("k", 8, b"\xc0\x80")]), "UTF-8")          # overlong NUL
    parse_err(build(meta=[("k", 8, b"\xed\xa0\x80")]), "UTF-8")      # surrogate
    parse_err(build(tensors=[("t", [1] * 9, 0, 0)]), "dimensions")
    parse_err(build(meta=[("a\0b", 4, 1)]), "NUL")
    parse_err(build(tensors=[("t\0", [4], 0, 0)]), "NUL")
    big_str = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", (1 << 30) + 1)
    parse_err(big_str, "1 GiB")
    big_arr = (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + enc_str("k") +
               struct.pack("<IIQ", 9, 4, 10_000_001))
    parse_err(big_arr, "10 M")
    parse_err(b"GGUF" + struct.pack("<IQQ", 3, 100_001, 0), "tensor count")
    parse_err(b"GGUF" + struct.pack("<IQQ", 3, 0, 100_001), "KV count")


def test_every_value_type_and_key_order():
    meta = [("z.u8", 0, 255), ("y.i8", 1, -128), ("x.u16", 2, 65535), ("w.i16", 3, -32768),
            ("v.u32", 4, 2**32 - 1), ("u.i32", 5, -2**31), ("t.f32", 6, 1.5),
            ("s.bool", 7, 0), ("r.str", 8, "héllo ✓"), ("q.u64", 10, 2**64 - 1),
            ("p.i64", 11, -2**63), ("o.f64", 12, -0.1),
            ("n.strs", 9, (8, ["a", "", "ü"])), ("m.nest", 9, (9, [(4, [1]), (4, [2, 3])])),
            ("B.upper", 4, 7)]
    with L.GgufFile.parse(build(meta=meta)) as f:
        assert f.keys() == sorted(k for k, _, _ in meta)          # byte order: "B" < "m"
        for k, t, v in meta:
            assert f.value_type(k) == t
            if t == 9 and v[0] == 9:
                continue
            got = f.get(k)
            want = v[1] if t == 9 else v
            assert got == (bool(want) if t == 7 else want), k
        assert f.get("o.f64") == -0.1                              # exact f64


def test_typed_accessors():
    # model_file.rs:131-182 conversions
    meta = [("a", 4, 7), ("b", 10, 2**32 + 5), ("c", 5, -1), ("d", 11, -2), ("e", 0, 9),
            ("f", 2, 3), ("g", 6, 0.25), ("h", 12, 0.1), ("s", 8, "txt"),
            ("ai", 9, (1, [-1, 2])), ("au", 9, (2, [7, 8])), ("af", 9, (6, [1.0]))]
    with L.GgufFile.parse(build(meta=meta)) as f:
        assert [f.meta_u32(k) for k in "abcde"] == [7, 5, 2**32 - 1, 2**32 - 2, 9]
        with pytest.raises(L.LfmError, match="not a u32"):
            f.meta_u32("f")                                        # U16 is not accepted
        assert f.meta_f32("g") == 0.25
        assert f.meta_f32("h") == np.float32(0.1)
        with pytest.raises(L.LfmError):
            f.meta_f32("a")
        assert f.meta_str("s") == "txt"
        assert f.meta_u32_array("ai") == [2**32 - 1, 2] and f.meta_u32_array("au") == [7, 8]
        with pytest.raises(L.LfmError, match="not int"):
            f.meta_u32_array("af")
        with pytest.raises(L.LfmError) as ei:
            f.meta_u32("missing")
        assert ei.value.code == L.LFM_ENOTFOUND


def test_tensor_reads(tmp_path):
    rng = np.random.default_rng(3)
    a = rng.standard_normal(40).astype(np.float32)
    q = rng.integers(0, 256, 2 * 210, dtype=np.uint8)
    head = build(tensors=[("a", [40], 0, 0), ("q", [512], 14, 160)], tail=False)
    body = a.tobytes() + b"\0" * 0 + bytes(160 - a.nbytes) + q.tobytes()
    p = str(tmp_path / "r.gguf")
    with open(p, "wb") as fh:
        fh.write(head + body)
    with L.GgufFile.open(p) as f:
        assert np.array_equal(f.read_tensor("a").view(np.float32), a)
        assert np.array_equal(f.read_tensor("q"), q)
        assert np.array_equal(f.read_tensor_range("q", 200, 20), q[200:220])
        with pytest.raises(L.LfmError, match="range exceeds"):
            f.read_tensor_range("q", 400, 21)
        with pytest.raises(L.LfmError) as ei:
            f.read_tensor("nope")
        assert ei.value.code == L.LFM_ENOTFOUND and not f.has_tensor("nope")


# ---------------------------------------------------------------- hyper-parameters
def lfm_meta(**over):
    m = {"lfm2moe.block_count": (4, 24), "lfm2moe.embedding_length": (4, 2048),
         "lfm2moe.attention.head_count": (4, 32),
         "lfm2moe.attention.head_count_kv": (9, (5, [8 if l in L.LFM2_ATTENTION_LAYERS else 0
                                                     for l in range(24)])),
         "lfm2moe.vocab_size": (4, 128000), "lfm2moe.expert_count": (4, 32),
         "lfm2moe.expert_used_count": (4, 4), "lfm2moe.expert_feed_forward_length": (4, 1792),
         "lfm2moe.feed_forward_length": (4, 7168),
         "lfm2moe.attention.layer_norm_rms_epsilon": (6, 1e-5),
         "lfm2moe.rope.freq_base": (6, 1e6)}
    m.update(over)
    return [(k, t, v) for k, (t, v) in m.items() if t is not None]


def test_hparams_real_geometry():
    with L.GgufFile.parse(build(meta=lfm_meta())) as f:
        hp = f.hparams(strict=True)
    assert (hp.dim, hp.heads, hp.head_dim, hp.n_layers, hp.vocab) == (2048, 32, 64, 24, 128000)
    assert hp.kv_list() == [8 if l in L.LFM2_ATTENTION_LAYERS else 0 for l in range(24)]
    assert (hp.n_expert, hp.n_used, hp.expert_ff, hp.n_ff) == (32, 4, 1792, 7168)
    # defaults (lfm.rs:112-113, 140): dense lead 2, l_cache 3, eos 124900
    assert (hp.dense_lead, hp.conv_l_cache, hp.eos) == (2, 3, 124900)
    assert hp.eps == np.float32(1e-5) and hp.rope_theta == 1e6


def test_hparams_defaults_and_errors():
    # meta_u32_default falls back on any failure, including a value of another type
    with L.GgufFile.parse(build(meta=lfm_meta(**{
            "lfm2moe.leading_dense_block_count": (8, "x"), "lfm2moe.shortconv.l_cache": (4, 5),
            "tokenizer.ggml.eos_token_id": (4, 7)}))) as f:
        hp = f.hparams()
        assert (hp.dense_lead, hp.conv_l_cache, hp.eos) == (2, 5, 7)
    for key, bad in [("lfm2moe.vocab_size", 65536), ("lfm2moe.expert_count", 16),
                     ("lfm2moe.embedding_length", 1024)]:
        with L.GgufFile.parse(build(meta=lfm_meta(**{key: (4, bad)}))) as f:
            with pytest.raises(L.LfmError, match="unsupported geometry"):
                f.hparams(strict=True)
    with L.GgufFile.parse(build(meta=lfm_meta(**{"lfm2moe.vocab_size": (4, 65536)}))) as f:
        assert f.hparams(strict=False).vocab == 65536
    with L.GgufFile.parse(build(meta=lfm_meta(**{"lfm2moe.rope.freq_base": (None, 0)}))) as f:
        with pytest.raises(L.LfmError) as ei:
            f.hparams()
        assert ei.value.code == L.LFM_ENOTFOUND
    with L.GgufFile.parse(build(meta=lfm_meta(**{
            "lfm2moe.attention.head_count_kv": (9, (5, [0] * 23))}))) as f:
        with pytest.raises(L.LfmError, match="entries"):
            f.hparams()


# ---------------------------------------------------------------- writer
def test_writer_matches_independent_encoding(tmp_path):
    meta = [("general.architecture", 8, "test"), ("general.alignment", 4, 64),
            ("n.arr", 9, (5, [3, -4])), ("f", 12, 2.5), ("s", 9, (8, ["x", "yz"]))]
    tensors = [("a", [40], 0, 0), ("q", [512], 14, 192)]
    want = bytearray(build(align=64, meta=meta, tensors=tensors))
    want += b"\0" * (-len(want) % 64)
    rng = np.random.default_rng(5)
    a = rng.standard_normal(40).astype(np.float32)
    q = rng.integers(0, 256, 420, dtype=np.uint8)
    data_off = len(build(align=64, meta=meta, tensors=tensors, tail=False))
    want[data_off:data_off + 160] = a.tobytes()
    want[data_off + 192:data_off + 192 + 420] = q.tobytes()

    w = L.GgufWriter()
    w.set_string("general.architecture", "test")
    w.set_scalar("general.alignment", L.GGUF_U32, 64)
    w.set_array("n.arr", L.GGUF_I32, [3, -4])
    w.set_scalar("f", L.GGUF_F64, 2.5)
    w.set_array("s", L.GGUF_STRING, ["x", "yz"])
    ia = w.add_tensor("a", 0, [40])
    iq = w.add_tensor("q", 14, [512])
    p = str(tmp_path / "w.gguf")
    w.begin(p)
    w.write_tensor(iq, q)
    w.write_tensor(ia, a)
    w.finish()
    w.close()
    assert open(p, "rb").read() == bytes(want)


def test_writer_errors(tmp_path):
    w = L.GgufWriter()
    with pytest.raises(L.LfmError, match="BOOL"):
        w.set_scalar("b", L.GGUF_BOOL, 2)
    with pytest.raises(L.LfmError):
        w.add_tensor("q", 14, [100])
    w.add_tensor("t", 0, [4])
    with pytest.raises(L.LfmError, match="duplicate"):
        w.add_tensor("t", 0, [4])
    with pytest.raises(L.LfmError) as ei:
        w.write_tensor(0, np.zeros(4, np.float32))
    assert ei.value.code == L.LFM_ESTATE
    w.begin(str(tmp_path / "e.gguf"))
    with pytest.raises(L.LfmError, match="bytes given"):
        w.write_tensor(0, np.zeros(3, np.float32))
    with pytest.raises(L.LfmError, match="not written"):
        w.finish()
    w.close()
    w = L.GgufWriter()
    w.set_scalar("general.alignment", L.GGUF_U32, 48)
    with pytest.raises(L.LfmError, match="alignment"):
        w.begin(str(tmp_path / "e2.gguf"))
    w.close()


def test_synthetic_model_round_trip(tmp_path):
    hp = small_hparams(kinds=("conv", "attn", "conv"), dense_lead=1)
    opts = L.synth_opts(seed=77, bias_sigma=0.5)
    p = str(tmp_path / "syn.gguf")
    L.write_synthetic_gguf(p, hp, opts, threads=4)
    descs = L.model_tensor_descs(hp, opts)
    with L.GgufFile.open(p) as f:
        got = f.hparams(strict=False)
        assert bytes(got) == bytes(hp)
        assert f.get("general.architecture") == "lfm2moe"
        assert f.get("lfm2moe.attention.head_count_kv") == hp.kv_list()
        assert f.n_tensors == len(descs)
        for d, t in zip(descs, f.tensors):
            assert t.name == d.name and t.ggml_type == d.ggml_type and t.shape == d.shape
            assert t.file_offset % 32 == 0
            want = L.synth_tensor(d, opts, threads=4)
            assert np.array_equal(f.read_tensor(d.name.decode()), want.view(np.uint8))
    assert os.path.getsize(p) % 32 == 0
