"""Pins the oracle's Q6_K decode and matvec (and the host-side plane packer).

Checks, each of which fails on a plausible mistake (wrong nibble/field/scale
index, unsigned scales, fused d*sc*q order, dropped -32):
  * the reference's known answers (engine/src/q6k.rs:199-290) from the golden file;
  * the reference's mirror test (engine/tests/dequant_mirror.rs:48-91): its
    xorshift64 stream, forced bytes, per-element index formula, bit-exact;
  * an independent numpy closed form over random blocks (bit-exact, incl. the
    signed-zero rule of three float multiplies);
  * the f64 matvec against a numpy float64 brute force;
  * the GPU plane layout restated in numpy (lane mapping of the kernels) gives
    bit-identical weights, and pack/unpack round-trips.
"""
import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
KAT = json.load(open(os.path.join(HERE, "golden", "q6k_kat.json")))


def np_dequant(raw: np.ndarray) -> np.ndarray:
    """Closed form of a GGUF Q6_K element (ggml block_q6_K layout), float32 ops."""
    raw = raw.reshape(-1, 210)
    d = raw[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    k = np.arange(256)
    half, jj = k >> 7, k & 127
    sub, l = jj >> 5, jj & 31
    is_ = l >> 4
    qlb = raw[:, half * 64 + l + (sub & 1) * 32].astype(np.int32)
    nib = np.where(sub >> 1, qlb >> 4, qlb & 15)
    field = (raw[:, 128 + half * 32 + l].astype(np.int32) >> (2 * sub)) & 3
    q = (nib | (field << 4)) - 32
    s = raw[:, 192 + half * 8 + is_ + 2 * sub].view(np.int8).astype(np.float32)
    return ((d[:, None] * s) * q.astype(np.float32)).astype(np.float32)


def xorshift_blocks(nblocks=512, seed=0x9E3779B97F4A7C15):
    """dequant_mirror.rs:50-74: xorshift64 bytes, d = 0x3B00, forced scales."""
    s = seed
    mask = (1 << 64) - 1
    out = np.zeros((nblocks, 210), dtype=np.uint8)
    for b in range(nblocks):
        for i in range(210):
            s ^= (s << 13) & mask
            s ^= s >> 7
            s ^= (s << 17) & mask
            out[b, i] = (s >> 11) & 0xFF
        out[b, 208], out[b, 209] = KAT["mirror"]["d_bytes"]
        for k, v in KAT["mirror"]["forced"].items():
            out[b, int(k)] = v
    return out


def random_blocks(n, seed):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(n, 210), dtype=np.uint8)
    d = (rng.standard_normal(n) * 1e-3).astype(np.float16)
    raw[:, 208:210] = d.view(np.uint8).reshape(n, 2)
    return raw


def kat_block(spec):
    block = np.zeros(210, dtype=np.uint8)
    block[208], block[209] = spec["d_bytes"]
    block[192:208] = spec["scales"]
    block[0] = spec["ql0"]
    block[128] = spec["qh0"]
    return block


def test_fp16_known_answers(oracle):
    for value, bits in KAT["fp16_roundtrip"]:
        assert oracle.f32_to_f16_bits(value) == bits
        assert oracle.f16_to_f32(bits) == value


@pytest.mark.parametrize("name", ["dequant_single_known_block", "dequant_scale_and_d"])
def test_dequant_known_blocks(oracle, name):
    spec = KAT[name]
    out = oracle.dequant_block(kat_block(spec))
    for k, v in spec["expect"].items():
        assert out[int(k)] == np.float32(v), (k, out[int(k)], v)


def test_matvec_consistency_kat(oracle):
    """q6k.rs:252-290: 256x4 weight, d=1, scales 1, element 0 low nibble = o+1."""
    spec = KAT["matvec_consistency"]
    in_dim, out_dim = spec["in_dim"], spec["out_dim"]
    w = np.zeros((out_dim, 210), dtype=np.uint8)
    for o in range(out_dim):
        w[o, 208], w[o, 209] = spec["d_bytes"]
        w[o, 192:208] = spec["scales"]
        w[o, 0] = o + 1
    x = (np.arange(in_dim) % 7).astype(np.float32) * np.float32(0.5)
    got = oracle.q6k_matvec(w.reshape(-1), in_dim, out_dim, x)
    deq = oracle.dequant_rows(w.reshape(-1), out_dim, in_dim)
    expect = np.array([np.float32(np.dot(deq[o].astype(np.float64), x.astype(np.float64)))
                       for o in range(out_dim)], dtype=np.float32)
    assert np.array_equal(got, expect)
    # element 0 of row o is (o+1-32); every other element is -32 (d = 1, sc = 1)
    row0 = np.full(in_dim, -32.0, dtype=np.float64)
    row0[0] = 1 - 32
    assert got[0] == np.float32(row0 @ x.astype(np.float64))


def test_mirror_identity_bit_exact(oracle):
    """dequant_mirror.rs:48-91 restated: the per-element index formula equals
    the reference dequant bit for bit over 512 xorshift blocks."""
    blocks = xorshift_blocks()
    mism = 0
    for b in range(blocks.shape[0]):
        ref = oracle.dequant_block(blocks[b])
        mirror = np.array([oracle.mirror_elem(blocks[b], k) for k in range(256)], dtype=np.float32)
        mism += int(np.count_nonzero(ref.view(np.uint32) != mirror.view(np.uint32)))
    assert mism == 0
    # and both equal the numpy closed form
    assert np.array_equal(oracle.dequant_rows(blocks.reshape(-1), 512, 256).view(np.uint32),
                          np_dequant(blocks).view(np.uint32))


def test_dequant_matches_closed_form_bitwise(oracle):
    raw = random_blocks(4096, 1)
    # edge cases: zero scales and zero codes (signed zeros), subnormal and negative d
    raw[0, 192:208] = 0
    raw[1, 0:192] = 0x00
    raw[1, 128:192] = 0xAA  # field 2 everywhere -> q = 32 - 32 = 0 for low nibble 0
    raw[2, 208:210] = np.array([1e-7], dtype=np.float16).view(np.uint8)
    raw[3, 208:210] = np.array([-0.0], dtype=np.float16).view(np.uint8)
    got = oracle.dequant_rows(raw.reshape(-1), 4096, 256)
    exp = np_dequant(raw)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    assert np.any(np.signbit(got[0]) & (got[0] == 0))  # sign(d) xor sign(sc) xor sign(q)


def test_unsigned_scale_reading_would_fail(oracle):
    """The legacy u8 scale bug (q6k.rs:43-53) is detected by the closed form."""
    raw = random_blocks(8, 2)
    raw[:, 192] = 0x80  # -128
    wrong = np_dequant(raw)
    wrong_u8 = wrong.copy()
    wrong_u8[:, 0:16] *= -1.0  # what +128 instead of -128 would give
    got = oracle.dequant_rows(raw.reshape(-1), 8, 256)
    assert np.array_equal(got, wrong)
    assert not np.array_equal(got, wrong_u8)


def test_matvec_f64_brute_force(oracle):
    rows, in_dim = 96, 2048
    raw = random_blocks(rows * in_dim // 256, 3)
    x = np.random.default_rng(4).standard_normal(in_dim).astype(np.float32)
    got = oracle.q6k_matvec(raw.reshape(-1), in_dim, rows, x)
    w = np_dequant(raw).reshape(rows, in_dim).astype(np.float64)
    exp = np.array([np.float32(np.sum(w[o] * x.astype(np.float64))) for o in range(rows)])
    # f64 sums in a different order agree to f32 rounding
    assert np.allclose(got, exp, rtol=1e-6, atol=1e-6 * float(np.abs(exp).max()))


def test_aligned_repack_kat(oracle):
    """q6k.rs:189-197: every byte kept, two zero pad bytes per block."""
    for blocks in KAT["aligned_repack_blocks"]:
        raw = (np.arange(blocks * 210) % 256).astype(np.uint8)
        out = oracle.repack_aligned(raw).reshape(blocks, 212)
        assert np.array_equal(out[:, :210], raw.reshape(blocks, 210))
        assert not out[:, 210:].any()


def plane_dequant(packed: np.ndarray, rows: int, in_dim: int) -> np.ndarray:
    """numpy restatement of the kernels' lane mapping over the plane layout."""
    nb = in_dim // 256
    nblk = rows * nb
    ql = packed[: nblk * 128].reshape(nblk, 8, 16)
    qh = packed[nblk * 128: nblk * 192].reshape(nblk, 8, 8)
    sc = packed[nblk * 192: nblk * 208].reshape(nblk, 4, 4).view(np.int8)
    d = packed[nblk * 208:].view(np.float16).astype(np.float32)
    out = np.zeros((nblk, 256), dtype=np.float32)
    for c in range(8):
        A = ql[:, c, 0:8].astype(np.int32)
        B = ql[:, c, 8:16].astype(np.int32)
        H = qh[:, c, :].astype(np.int32)
        codes = [(A & 15) | ((H & 3) << 4), (B & 15) | (((H >> 2) & 3) << 4),
                 (A >> 4) | (((H >> 4) & 3) << 4), (B >> 4) | (((H >> 6) & 3) << 4)]
        for s in range(4):
            ds = d * sc[:, c >> 1, s].astype(np.float32)
            pos = (c >> 2) * 128 + s * 32 + (c & 3) * 8 + np.arange(8)
            out[:, pos] = ds[:, None] * (codes[s] - 32).astype(np.float32)
    return out.reshape(rows, in_dim)


def test_plane_layout_matches_reference_decode(lfm, oracle):
    rows, in_dim = 12, 1792
    raw = random_blocks(rows * in_dim // 256, 5).reshape(-1)
    packed = lfm.q6k_pack(raw, rows, in_dim)
    assert packed.nbytes == raw.nbytes
    got = plane_dequant(packed, rows, in_dim)
    exp = oracle.dequant_rows(raw, rows, in_dim)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    assert np.array_equal(lfm.q6k_unpack(packed, rows, in_dim), raw)
