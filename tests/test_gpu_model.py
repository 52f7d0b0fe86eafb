"""GPU parity of the decode-step layers and the token loop against the oracle.

Configurations (synthetic, seeded; same bytes to both sides):
  cfg1  MoE FFN step: dim 2048, 32 experts top-4, ff 1792 -> expert ids bit-exact,
        FFN output rel-L2 <= 1e-3 (bias = 0 and bias ~ N(0, 0.1)).
  cfg2  GQA decode attention: 32 q heads / 8 kv heads, head_dim 64, theta 1e6,
        f16 KV filled N(0,1) for L = 512, 2048, 4096 -> rel-L2 <= 1e-3.
  cfg3  gated short conv, 256 sequential tokens with a seeded 2-slot state ->
        rel-L2 <= 1e-3 per step for output and state.
  cfg4  token loop of a reduced model (4 layers, real widths) -> prompt logits
        rel-L2 <= 1e-3, tokens equal wherever the oracle's top-2 margin exceeds
        1e-3 * max|logit| (teacher-forced with the GPU's tokens).
Relative L2 = ||gpu - oracle|| / ||oracle|| (bin/q6_check.rs:120-136 convention).
"""
import numpy as np
import pytest

from conftest import rel_l2
from model_util import gpu_engine, model_tensors, oracle_engine, top2_margin

pytestmark = pytest.mark.gpu

SEED = 0x9E3779B97F4A7C15


def hparams(lfm, **kw):
    base = dict(dim=2048, heads=32, n_layers=1, attention_layers=(), kv=8, vocab=256, eos=1 << 30,
                n_expert=32, n_used=4, expert_ff=1792, n_ff=256, dense_lead=0)
    base.update(kw)
    return lfm.make_hparams(**base)


@pytest.mark.parametrize("bias_sigma", [0.0, 0.1])
def test_cfg1_moe_step(gpu, oracle, bias_sigma):
    hp = hparams(gpu)
    opts = gpu.synth_opts(SEED, bias_sigma=bias_sigma)
    tensors = model_tensors(hp, opts)
    g = gpu_engine(hp, tensors, ctx=16)
    o = oracle_engine(oracle, hp, tensors, ctx=16)
    for s in range(6):
        x = gpu.synth_normal(SEED + s, "cfg1.h", hp.dim)
        yg = g.run_ffn(0, x)
        ids_g, w_g = g.last_route()
        yo = o.run_ffn(0, x)
        ids_o, w_o, scores = o.last_route(0)
        srt = np.sort(scores)[::-1]
        margin = float(srt[3] - srt[4])
        print(f"bias {bias_sigma} sample {s}: ids {ids_g} margin4/5 {margin:.3e}")
        assert ids_g == ids_o
        assert np.allclose(w_g, w_o, rtol=1e-5, atol=1e-7)
        err = rel_l2(yg - x, yo - x)
        assert err <= 1e-3, err


@pytest.mark.parametrize("L", [512, 2048, 4096])
def test_cfg2_attention_decode(gpu, oracle, L):
    hp = hparams(gpu, attention_layers=(0,), dense_lead=1)
    tensors = model_tensors(hp)
    g = gpu_engine(hp, tensors, ctx=4096)
    o = oracle_engine(oracle, hp, tensors, ctx=4096)
    p = L - 1
    kv = gpu.synth_normal(SEED, f"cfg2.kv{L}", 2 * p * 8 * 64)
    kv = kv.astype(np.float16).astype(np.float32)  # the cache holds binary16 values
    snap = kv.tobytes()
    g.restore_session(p, snap)
    o.restore(p, snap)
    assert g.snapshot_resident_cache(p) == snap
    x = gpu.synth_normal(SEED, f"cfg2.x{L}", hp.dim)
    yg = g.run_mixer(0, x, p)
    yo = o.run_mixer(0, x, p)
    err = rel_l2(yg - x, yo - x)
    print(f"L={L} rel-L2 {err:.3e}")
    assert err <= 1e-3
    sg = np.frombuffer(g.snapshot_resident_cache(L), np.float32)
    so = np.frombuffer(o.snapshot(L), np.float32)
    assert np.array_equal(sg.reshape(2, L, 512)[:, :p], so.reshape(2, L, 512)[:, :p])
    assert rel_l2(sg.reshape(2, L, 512)[:, p], so.reshape(2, L, 512)[:, p]) <= 1e-3


def test_cfg3_shortconv_256_tokens(gpu, oracle):
    hp = hparams(gpu, dense_lead=1)
    tensors = model_tensors(hp)
    g = gpu_engine(hp, tensors, ctx=512)
    o = oracle_engine(oracle, hp, tensors, ctx=512)
    state = gpu.synth_normal(SEED, "cfg3.state", hp.dim * 2).tobytes()
    g.restore_session(0, state)
    o.restore(0, state)
    worst = 0.0
    for t in range(256):
        x = gpu.synth_normal(SEED + t, "cfg3.x", hp.dim)
        yg = g.run_mixer(0, x, t)
        yo = o.run_mixer(0, x, t)
        err = rel_l2(yg - x, yo - x)
        serr = rel_l2(np.frombuffer(g.snapshot_resident_cache(0), np.float32),
                      np.frombuffer(o.snapshot(0), np.float32))
        worst = max(worst, err, serr)
        assert err <= 1e-3 and serr <= 1e-3, (t, err, serr)
    print(f"cfg3 worst rel-L2 over 256 steps {worst:.3e}")


@pytest.fixture(scope="module")
def reduced_model(gpu):
    hp = gpu.make_hparams(dim=2048, heads=32, n_layers=4, attention_layers=(1, 3), kv=8,
                          vocab=8192, eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792,
                          n_ff=7168, dense_lead=2)
    return hp, model_tensors(hp)


def test_cfg4_reduced_token_loop(gpu, oracle, reduced_model):
    hp, tensors = reduced_model
    g = gpu_engine(hp, tensors, ctx=256)
    o = oracle_engine(oracle, hp, tensors, ctx=256)
    prompt = [int(t) for t in np.random.default_rng(1).integers(0, hp.vocab, 24)]
    lg = g.forward(prompt, 0)
    lo = o.forward(prompt, 0)
    err = rel_l2(lg, lo)
    print(f"prompt logits rel-L2 {err:.3e}")
    assert err <= 1e-3
    first = int(oracle.argmax(lg))
    tol = 1e-3 * float(np.abs(lo).max())
    if top2_margin(lo) > tol:
        assert first == oracle.argmax(lo)
    steps = 24
    toks = g.decode_run(first, len(prompt), steps)
    assert len(toks) == steps
    compared = 0
    feed = first
    for s in range(steps):
        lo = o.forward([feed], len(prompt) + s)
        if top2_margin(lo) > tol:
            assert toks[s] == oracle.argmax(lo), (s, toks[s], oracle.argmax(lo))
            compared += 1
        feed = toks[s]
    assert compared >= steps // 2
    # resident state after the loop matches the oracle's
    n = len(prompt) + steps
    sg = np.frombuffer(g.snapshot_resident_cache(n), np.float32)
    so = np.frombuffer(o.snapshot(n), np.float32)
    assert rel_l2(sg, so) <= 1e-3
    # forward_token (chunked prefill, api_stream.rs:58-63) agrees with forward
    g2 = gpu_engine(hp, tensors, ctx=256)
    nxt = g2.forward_token(prompt[:16], 0)
    nxt = g2.forward_token(prompt[16:], 16)
    assert nxt == first
    assert g2.forward_token([first], len(prompt)) == toks[0]


def test_real_vocab_head_and_chunked_prefill(gpu, oracle):
    """The real model's vocabulary (V = 128000, lfm.rs:117-125) through the tied
    head and argmax, and a prompt prefilled in 64-token chunks (api_stream.rs:57-63,
    work_bound.rs PREFILL_CHUNK) against the whole-prompt forward and the oracle."""
    hp = gpu.make_hparams(dim=2048, heads=32, n_layers=2, attention_layers=(1,), kv=8,
                          vocab=128000, eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792,
                          n_ff=7168, dense_lead=1)
    tensors = model_tensors(hp, gpu.synth_opts(SEED, bias_sigma=0.1))
    g = gpu_engine(hp, tensors, ctx=160)
    o = oracle_engine(oracle, hp, tensors, ctx=160)
    prompt = [int(t) for t in np.random.default_rng(9).integers(0, hp.vocab, 80)]
    prompt[-1] = hp.vocab - 1
    lg, lo = g.forward(prompt, 0), o.forward(prompt, 0)
    assert lg.shape == (128000,)
    err = rel_l2(lg, lo)
    print(f"V=128000 prompt logits rel-L2 {err:.3e}")
    assert err <= 1e-3
    first = int(oracle.argmax(lg))
    tol = 1e-3 * float(np.abs(lo).max())
    if top2_margin(lo) > tol:
        assert first == oracle.argmax(lo)
    toks = g.decode_run(first, len(prompt), 6)
    feed, clear = first, []
    for s, t in enumerate(toks):
        lo = o.forward([feed], len(prompt) + s)
        clear.append(top2_margin(lo) > tol)
        if clear[-1]:
            assert t == oracle.argmax(lo), (s, t, oracle.argmax(lo))
        feed = t
    assert sum(clear) >= 3
    # the same prompt in chunks of 64 and 16 tokens, then the same greedy tokens
    g2 = gpu_engine(hp, tensors, ctx=160)
    g2.forward_token(prompt[:64], 0)
    nxt = g2.forward_token(prompt[64:], 64)
    if top2_margin(lg) > tol:
        assert nxt == first
    feed = first
    for s in range(len(toks)):
        nxt = g2.forward_token([feed], len(prompt) + s)
        if clear[s]:
            assert nxt == toks[s], s
        feed = toks[s]


def test_engine_preconditions(gpu, reduced_model):
    hp, tensors = reduced_model
    g = gpu_engine(hp, tensors, ctx=64)
    with pytest.raises(gpu.LfmError) as e:
        g.forward([hp.vocab], 0)
    assert e.value.code == gpu.LFM_ERANGE
    with pytest.raises(gpu.LfmError) as e:
        g.forward([1] * 65, 0)
    assert e.value.code == gpu.LFM_ERANGE
    with pytest.raises(gpu.LfmError) as e:
        g.forward_token([1] * 65, 0)
    assert e.value.code == gpu.LFM_EINVAL
    with pytest.raises(gpu.LfmError):
        g.forward([], 0)
    with pytest.raises(gpu.LfmError):
        g.restore_session(3, b"\0" * 7)
    # eos stops the device-resident loop without storing it
    first = g.forward_token([1, 2, 3], 0)
    toks = g.decode_run(first, 3, 8, eos=hp.vocab + 5)
    assert len(toks) == 8
    g.reset_session()
    g.forward_token([1, 2, 3], 0)
    stop = toks[2]
    toks2 = g.decode_run(first, 3, 8, eos=stop)
    assert toks2 == toks[: toks.index(stop)]
