"""binary16 conversion (oracle and product host code) against numpy's IEEE
float16 (exhaustive over all f16 values and a dense sweep of f32 inputs), and the
seeded synthetic generator's determinism and distributions."""
import numpy as np


def test_f16_to_f32_all_values(oracle, lfm):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exp = bits.view(np.float16).astype(np.float32)
    got_o = np.array([oracle.f16_to_f32(int(b)) for b in bits[::7]], dtype=np.float32)
    assert np.array_equal(got_o.view(np.uint32)[~np.isnan(exp[::7])],
                          exp[::7].view(np.uint32)[~np.isnan(exp[::7])])
    got_p = np.array([lfm.lib().lfm_f16_to_f32(int(b)) for b in bits[::7]], dtype=np.float32)
    assert np.array_equal(got_p.view(np.uint32)[~np.isnan(exp[::7])],
                          exp[::7].view(np.uint32)[~np.isnan(exp[::7])])


def test_f32_to_f16_rne_sweep(oracle):
    # every f32 with the low 9 mantissa bits in a set that covers the rounding
    # boundary cases (0, 1, half-1, half, half+1, top), over all exponents/signs
    hi = np.arange(0, 1 << 23, dtype=np.uint32) << 9
    lows = np.array([0, 1, 0xFF, 0x100, 0x101, 0x1FF], dtype=np.uint32)
    x = (hi[:, None] | lows[None, :]).reshape(-1)
    x = np.concatenate([x[::3], x[1::3][:1 << 20]])
    f = x.view(np.float32)
    exp = f.astype(np.float16).view(np.uint16)
    got = oracle.f32_to_f16_array(f)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], exp[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all(got[nan] & 0x3FF)


def test_product_f32_to_f16_matches(oracle, lfm):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e-3),
        (rng.standard_normal(20000) * 1e-6).astype(np.float32),  # subnormal halves
        rng.standard_normal(2000).astype(np.float32) * np.float32(7e4),  # overflow
        np.array([6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 65504, 65519.99, 65520, -0.0, np.inf, -np.inf], np.float32),
    ])
    exp = x.astype(np.float16).view(np.uint16)
    got = np.array([lfm.f32_to_f16_bits(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, exp)


def test_synth_deterministic_and_thread_independent(lfm):
    a = lfm.synth_q6k_blocks(123, "blk.0.x", 5000, threads=1)
    b = lfm.synth_q6k_blocks(123, "blk.0.x", 5000, threads=7)
    c = lfm.synth_q6k_blocks(124, "blk.0.x", 5000, threads=7)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    n1 = lfm.synth_normal(5, "s", 10001, 0.0, 1.0, threads=1)
    n2 = lfm.synth_normal(5, "s", 10001, 0.0, 1.0, threads=5)
    assert np.array_equal(n1, n2)


def test_synth_distributions(lfm):
    blocks = lfm.synth_q6k_blocks(1, "t", 200000, d_sigma=1e-3, threads=8).reshape(-1, 210)
    sc = blocks[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    d = blocks[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
    assert abs(d.std() - 1e-3) < 2e-5 and abs(d.mean()) < 2e-5
    q = blocks[:, :192].astype(np.float64)
    assert abs(q.mean() - 127.5) < 0.2
    z = lfm.synth_normal(2, "n", 400000, 1.0, 0.02, threads=8).astype(np.float64)
    assert abs(z.mean() - 1.0) < 2e-4 and abs(z.std() - 0.02) < 2e-4


def test_model_tensor_table(lfm):
    hp = lfm.make_hparams()
    descs = lfm.model_tensor_descs(hp)
    names = {d.name.decode(): d for d in descs}
    assert names["token_embd.weight"].shape == (2048, 65536)
    assert names["blk.2.attn_k.weight"].shape == (2048, 512)
    assert names["blk.0.shortconv.in_proj.weight"].shape == (2048, 6144)
    assert names["blk.0.shortconv.conv.weight"].shape == (3, 2048)
    assert names["blk.0.ffn_down.weight"].shape == (7168, 2048)
    assert names["blk.5.ffn_down_exps.weight"].shape == (1792, 2048, 32)
    assert names["blk.5.exp_probs_b.bias"].shape == (32,)
    total = sum(lfm.lib().lfm_tensor_nbytes(d) for d in descs)
    q6 = sum(lfm.lib().lfm_tensor_nbytes(d) for d in descs if d.ggml_type == 14)
    # 6.84 GB model; decode streams every Q6 weight except the unused experts
    assert 6.8e9 < total < 6.9e9 and q6 > 0.99 * total


def test_full_scale_blocks(lfm):
    """The full-scale synthetic blocks: scales in [-127, 127] plus exactly one -128
    per super-block (ggml's quantizer maps a block's largest-magnitude scale to
    -128), the other bytes as in the default stream's layout."""
    raw = lfm.synth_q6k_blocks(7, "full.test", 4096, full_scales=True).reshape(-1, 210)
    sc = raw[:, 192:208].view(np.int8).astype(int)
    assert (sc == -128).sum(axis=1).tolist() == [1] * 4096
    assert sc.max() <= 127 and (np.abs(sc) > 64).mean() > 0.4
    default = lfm.synth_q6k_blocks(7, "full.test", 4096).reshape(-1, 210)
    assert np.array_equal(default[:, :192], raw[:, :192])  # same code bytes
    assert np.abs(default[:, 192:208].view(np.int8).astype(int)).max() <= 32
