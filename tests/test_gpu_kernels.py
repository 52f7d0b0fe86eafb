"""GPU parity of the Q6_K kernels and argmax against the oracle (C ABI calls).

Bars: Q6_K unpack bit-exact; matvec relative L2 <= 1e-5 against the f64
q6k_matvec oracle (engine/src/q6k.rs:167-183, relative-L2 convention of
bin/q6_check.rs:120-136); argmax index bit-exact (main.rs:112-141 semantics).
"""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu


def blocks(n, seed, d_sigma=1e-3, sc_lim=32):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(n, 210), dtype=np.uint8)
    raw[:, 192:208] = (rng.integers(-sc_lim, sc_lim, size=(n, 16))).astype(np.int8).view(np.uint8)
    d = (rng.standard_normal(n) * d_sigma).astype(np.float16)
    raw[:, 208:210] = d.view(np.uint8).reshape(n, 2)
    return raw


def test_dequant_bit_exact_cfg0_shape(gpu, oracle):
    rows, in_dim = 6144, 2048
    raw = gpu.synth_q6k_blocks(0x9E3779B97F4A7C15, "cfg0.weight", rows * in_dim // 256)
    w = gpu.Q6Weight(raw, rows, in_dim)
    got = w.dequant()
    exp = oracle.dequant_rows(raw, rows, in_dim)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_dequant_bit_exact_edge_blocks(gpu, oracle):
    raw = blocks(64, 11)
    raw[0, 192:208] = 0                          # zero scales -> signed zeros
    raw[1, :128] = 0; raw[1, 128:192] = 0xAA     # q - 32 == 0 everywhere
    raw[2, 208:210] = np.array([3e-7], np.float16).view(np.uint8)   # subnormal d
    raw[3, 208:210] = np.array([-0.0], np.float16).view(np.uint8)
    raw[4, 192:208] = np.array([-128, 127] * 8, np.int8).view(np.uint8)
    from test_oracle_q6k import xorshift_blocks
    mirror = xorshift_blocks(64)
    for r in (raw, mirror):
        w = gpu.Q6Weight(r.reshape(-1), 64, 256)
        got = w.dequant()
        exp = oracle.dequant_rows(r.reshape(-1), 64, 256)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_matvec_cfg0(gpu, oracle):
    """cfg0: W 6144x2048 Q6_K, x ~ N(0,1) f32, rel-L2 <= 1e-5 vs the f64 oracle."""
    rows, in_dim = 6144, 2048
    raw = gpu.synth_q6k_blocks(0x9E3779B97F4A7C15, "cfg0.weight", rows * in_dim // 256)
    x = gpu.synth_normal(0x9E3779B97F4A7C15, "cfg0.x", in_dim)
    y = gpu.Q6Weight(raw, rows, in_dim).matvec(x)
    ref = oracle.q6k_matvec(raw, in_dim, rows, x)
    err = rel_l2(y, ref)
    print(f"cfg0 rel-L2 {err:.3e}")
    assert err <= 1e-5


@pytest.mark.parametrize("rows,in_dim", [(1, 256), (3, 512), (513, 1792), (2048, 7168), (64, 8192),
                                         (1000, 2048), (7, 768)])
def test_matvec_shapes(gpu, oracle, rows, in_dim):
    raw = blocks(rows * in_dim // 256, rows + in_dim).reshape(-1)
    x = np.random.default_rng(rows).standard_normal(in_dim).astype(np.float32)
    y = gpu.Q6Weight(raw, rows, in_dim).matvec(x)
    ref = oracle.q6k_matvec(raw, in_dim, rows, x)
    assert rel_l2(y, ref) <= 1e-5


def test_matvec_full_int8_scales(gpu, oracle):
    """Sub-block scales over the whole int8 range, as quantizers write them into
    model files (the largest sub-block of a super-block gets |sc| = 128): the
    decode matvec forms sc * (q - 32) in fp32, so the 1e-5 bar still holds."""
    rows, in_dim = 2048, 2048
    raw = blocks(rows * in_dim // 256, 91, sc_lim=128).reshape(-1)
    x = np.random.default_rng(91).standard_normal(in_dim).astype(np.float32)
    y = gpu.Q6Weight(raw, rows, in_dim).matvec(x)
    assert rel_l2(y, oracle.q6k_matvec(raw, in_dim, rows, x)) <= 1e-5


def test_argmax_cases(gpu, oracle):
    from test_oracle_argmax_route import lcg_bits
    seed = 17
    for n in (1, 2, 7, 8, 9, 63, 64, 65, 255, 256, 257, 513, 4097):
        xs, seed = lcg_bits(n, seed)
        xs = xs.copy()
        assert gpu.argmax(xs)[0] == oracle.argmax(xs)
        for v in [np.nan, -np.inf, np.inf, 0.0, -0.0, 1.0]:
            xs.fill(v)
            assert gpu.argmax(xs)[0] == oracle.argmax(xs)
        if n > 8:
            xs[7] = 2.0
            xs[8] = 2.0
            assert gpu.argmax(xs)[0] == 7
    for n in (63, 513, 128003):
        xs = np.random.default_rng(n).standard_normal(n).astype(np.float32)
        xs[0] = np.nan
        xs[-1] = 100.0
        assert gpu.argmax(xs)[0] == n - 1
        xs[n // 2] = 100.0
        assert gpu.argmax(xs)[0] == n // 2


@pytest.mark.parametrize("rows,in_dim,T", [(6144, 2048, 200), (130, 256, 7), (1792, 2048, 129),
                                           (2048, 7168, 64), (256, 1792, 1), (2048, 2048, 31),
                                           (512, 1024, 32), (6144, 2048, 33), (1792, 2048, 128),
                                           (1000, 512, 150), (1000, 512, 40), (8192, 256, 2048),
                                           (3072, 2048, 64), (3200, 512, 64)])
def test_gemm_prefill_matches_f64(gpu, oracle, rows, in_dim, T):
    """Matrix-core GEMM (binary16 sc*(q-32) weights, hi/lo activations, fp32 d
    scaling) against the f64 q6k_matvec oracle per token: rel-L2 <= 1e-5.  Calls
    of up to 128 tokens read token-blocked activations (32-row tiles), so the
    tokens on either side of a tile edge are checked too.  The weights are read
    from a copy in 32-row tiles whose rows past the matrix are zero: 130 and
    1000 rows end inside a tile, with both the large-call and the 32-token tiles.
    Large calls run 64-token tiles when 128-token ones would make fewer than 512
    workgroups: 8192 rows x 2048 tokens is the case that runs the 128-token tiles.
    Small calls of up to 3072 rows run one 32-row tile per wave (3072 rows), wider
    ones two (3200)."""
    raw = blocks(rows * in_dim // 256, rows * 7 + T).reshape(-1)
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, in_dim)).astype(np.float32)
    x[0] *= 1000.0  # per-row scaling keeps large activations exact
    w = gpu.Q6Weight(raw, rows, in_dim)
    y = gpu.q6k_gemm(w, x)
    for t in sorted({0, T // 2, T - 1} | {t for t in (31, 32, 63, 64, 95, 96) if t < T}):
        ref = oracle.q6k_matvec(raw, in_dim, rows, x[t])
        err = rel_l2(y[t], ref)
        assert err <= 1e-5, (t, err)


@pytest.mark.parametrize("rows,in_dim,T", [(6144, 2048, 200), (1792, 2048, 129), (8192, 256, 2048),
                                           (1000, 512, 150), (2048, 7168, 300)])
def test_gemm_prefill_h16_copy_bit_identical(gpu, oracle, monkeypatch, rows, in_dim, T):
    """Large calls read the weights from a binary16 fragment copy made once
    (k_q6_tile_h16: the A fragments the Q6_K kernels decode in registers, k-step
    by k-step); with LFM_PREFILL_H16=0 they decode Q6_K in registers instead.  The
    two paths run the same products in the same order, so their outputs agree
    bit for bit; both stay within 1e-5 of the f64 oracle."""
    raw = blocks(rows * in_dim // 256, rows * 5 + T).reshape(-1)
    x = np.random.default_rng(T + 1).standard_normal((T, in_dim)).astype(np.float32)
    x[1] *= 1000.0
    w = gpu.Q6Weight(raw, rows, in_dim)
    y_h16 = gpu.q6k_gemm(w, x)
    monkeypatch.setenv("LFM_PREFILL_H16", "0")
    y_q6 = gpu.q6k_gemm(w, x)
    assert np.array_equal(y_h16.view(np.uint32), y_q6.view(np.uint32))
    for t in sorted({0, 1, T // 2, T - 1}):
        assert rel_l2(y_h16[t], oracle.q6k_matvec(raw, in_dim, rows, x[t])) <= 1e-5


@pytest.mark.parametrize("T", [130, 64, 5])
def test_gemm_prefill_block_scale_edges(gpu, oracle, T):
    """Super-block scales d that are zero (first, last, every other or every
    block of a row), -0.0, subnormal, or spread over eleven decades within one
    row: the GEMM folds d into its accumulators block by block, so every row
    is checked on its own against the f64 oracle (rel-L2 over tokens <= 1e-5;
    rows whose blocks all have d = 0 give exactly 0).  T = 130 runs the 128-token
    tiles; T <= 128 the split-K path with 32-token tiles, whose waves exchange the
    scales by lane shuffles."""
    rows, in_dim = 300, 2048
    nb = in_dim // 256
    raw = blocks(rows * nb, 77).reshape(rows, nb, 210)
    rng = np.random.default_rng(5)
    d = (rng.standard_normal((rows, nb)) * 1e-3).astype(np.float16)
    kind = np.arange(rows) % 8
    d[kind == 0] = 0
    d[kind == 1, 0] = 0
    d[kind == 2, nb - 1] = 0
    d[kind == 3, ::2] = 0
    spread = kind == 4
    mag = 10.0 ** rng.uniform(-7, 4.5, size=(int(spread.sum()), nb))
    d[spread] = (mag * rng.choice([-1.0, 1.0], size=mag.shape)).astype(np.float16)
    d[kind == 5, 1::3] = np.float16(-0.0)
    raw[:, :, 208:210] = d.view(np.uint8).reshape(rows, nb, 2)
    raw = raw.reshape(-1)
    x = rng.standard_normal((T, in_dim)).astype(np.float32)
    y = gpu.q6k_gemm(gpu.Q6Weight(raw, rows, in_dim), x)
    toks = sorted({0, T // 2, T - 1})
    ref = np.stack([oracle.q6k_matvec(raw, in_dim, rows, x[t]) for t in toks])
    got = y[toks]
    assert np.all(got[:, kind == 0] == 0)
    for r in np.flatnonzero(kind != 0):
        err = rel_l2(got[:, r], ref[:, r])
        assert err <= 1e-5, (r, kind[r], err)


@pytest.mark.parametrize("T,synth", [(130, False), (64, False), (200, True), (64, True), (1, True)])
def test_gemm_prefill_full_int8_scales(gpu, oracle, T, synth):
    """Sub-block scales over the whole int8 range (uniform int8, or the synthetic
    full-scale blocks: [-127, 127] with one -128 per super-block, as ggml's
    quantizer writes them).  A binary16 holds sc * (q - 32) exactly only up to
    magnitude 2048, so weights with such scales (the tile copy flags them) run
    the split-scale kernels, sc = (sc & ~15) + (sc & 15), both partial weights
    exact: against the f64 oracle the 1e-5 bar holds as for small scales.
    T = 200 runs the large-call kernel, T = 64 and 1 the small-call ones."""
    rows, in_dim = 1024, 2048
    if synth:
        raw = gpu.synth_q6k_blocks(93, "full.weight", rows * in_dim // 256, full_scales=True)
    else:
        raw = blocks(rows * in_dim // 256, 93, sc_lim=128).reshape(-1)
    x = np.random.default_rng(93).standard_normal((T, in_dim)).astype(np.float32)
    y = gpu.q6k_gemm(gpu.Q6Weight(raw, rows, in_dim), x)
    for t in sorted({0, T // 2, T - 1}):
        err = rel_l2(y[t], oracle.q6k_matvec(raw, in_dim, rows, x[t]))
        print(f"T={T} token {t}: rel-L2 {err:.2e}")
        assert err <= 1e-5, (t, err)


def encode_q6k(codes, scales, d):
    """GGUF block_q6_K bytes from 6-bit codes [n][256], int8 scales [n][16] and
    binary16 d [n]: element 128h + l + 32j of a block is code j of l in half h,
    low 4 bits in ql (j = 0, 1 low nibbles of ql[64h + l], ql[64h + 32 + l]; j = 2, 3
    their high nibbles), high 2 bits in qh[32h + l] bits 2j, 2j + 1."""
    n = codes.shape[0]
    raw = np.zeros((n, 210), dtype=np.uint8)
    for h in range(2):
        c = codes[:, 128 * h:128 * h + 128].reshape(n, 4, 32).astype(np.uint8)
        raw[:, 64 * h:64 * h + 32] = (c[:, 0] & 15) | ((c[:, 2] & 15) << 4)
        raw[:, 64 * h + 32:64 * h + 64] = (c[:, 1] & 15) | ((c[:, 3] & 15) << 4)
        raw[:, 128 + 32 * h:160 + 32 * h] = ((c[:, 0] >> 4) | ((c[:, 1] >> 4) << 2) | ((c[:, 2] >> 4) << 4)
                                            | ((c[:, 3] >> 4) << 6))
    raw[:, 192:208] = scales.astype(np.int8).view(np.uint8)
    raw[:, 208:210] = d.astype(np.float16).view(np.uint8).reshape(n, 2)
    return raw


@pytest.mark.parametrize("T,k0", [(256, 0), (64, 0), (64, 192), (8, 100)])
@pytest.mark.parametrize("lo,hi", [(-128, 128), (-64, 65)])
def test_gemm_prefill_weights_exact(gpu, oracle, T, k0, lo, hi):
    """Every weight the matrix-core GEMMs form, bit for bit: row r has scale
    lo + r % (hi - lo) in all sub-blocks, d = 1, and codes (k + r) % 64, so the
    rows hold every (scale, code) pair of the range; token t is the one-hot vector
    of column k0 + t, so y[t][r] is weight (r, k0 + t) times 1 with nothing else
    added, and must equal sc (q - 32) exactly.  Scales within [-64, 64] keep every
    product within binary16's exact integers (the default kernels); the whole int8
    range runs the split-scale kernels.  The encoding is checked against the
    oracle's dequant first.  T = 256 runs the large-call kernels, T <= 128 the
    32-token tiles."""
    rows, in_dim = 256, 256
    k = np.arange(in_dim)
    codes = (k[None, :] + np.arange(rows)[:, None]) % 64
    scales = np.repeat((lo + np.arange(rows) % (hi - lo))[:, None], 16, axis=1)
    raw = encode_q6k(codes, scales, np.ones(rows)).reshape(-1)
    exact = (scales[:, k // 16] * (codes - 32)).astype(np.float64)
    assert np.array_equal(oracle.dequant_rows(raw, rows, in_dim).astype(np.float64), exact)
    x = np.zeros((T, in_dim), dtype=np.float32)
    x[np.arange(T), k0 + np.arange(T)] = 1.0
    y = gpu.q6k_gemm(gpu.Q6Weight(raw, rows, in_dim), x)
    want = exact[:, k0:k0 + T].T.astype(np.float32)
    bad = np.argwhere(y.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, [(int(t), int(r), float(y[t, r]), float(want[t, r])) for t, r in bad[:8]]
