"""GPU parity of the batched (matrix-core) prefill against the oracle.

A multi-token forward (lfm.rs:290-694 with n > 1) runs every projection as a
Q6_K GEMM over the chunk's tokens.  Bars: last-token logits rel-L2 <= 1e-3
against the oracle's token-by-token forward and against the engine's own
one-decode-step-per-token mode; resident KV / conv state rel-L2 <= 1e-3;
greedy continuation equal wherever the oracle's top-2 margin exceeds
1e-3 * max|logit|.  Relative L2 = ||gpu - oracle|| / ||oracle||
(bin/q6_check.rs:120-136 convention).
"""
import numpy as np
import pytest

from conftest import rel_l2
from model_util import gpu_engine, model_tensors, oracle_engine, top2_margin

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def real_width(gpu):
    """Real widths (dim 2048, 32 experts top-4, ff 1792 / 7168), four layers."""
    hp = gpu.make_hparams(dim=2048, heads=32, n_layers=4, attention_layers=(1, 3), kv=8,
                          vocab=8192, eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792,
                          n_ff=7168, dense_lead=2)
    return hp, model_tensors(hp)


@pytest.fixture(scope="module")
def crowded(gpu):
    """8 experts top-2 so that experts take more than one 128-token tile."""
    hp = gpu.make_hparams(dim=512, heads=8, n_layers=4, attention_layers=(1, 3), kv=2,
                          vocab=1000, eos=1 << 30, n_expert=8, n_used=2, expert_ff=512,
                          n_ff=1024, dense_lead=1)
    return hp, model_tensors(hp, gpu.synth_opts(0x9E3779B97F4A7C15, bias_sigma=0.1))


def check_prefill(gpu, oracle, hp, tensors, n, ctx):
    prompt = [int(t) for t in np.random.default_rng(n).integers(0, hp.vocab, n)]
    g = gpu_engine(hp, tensors, ctx=ctx)
    o = oracle_engine(oracle, hp, tensors, ctx=ctx)
    lg = g.forward(prompt, 0)
    lo = o.forward(prompt, 0)
    err = rel_l2(lg, lo)
    sg = np.frombuffer(g.snapshot_resident_cache(n), np.float32)
    so = np.frombuffer(o.snapshot(n), np.float32)
    serr = rel_l2(sg, so)
    print(f"T={n}: logits rel-L2 {err:.3e}, state rel-L2 {serr:.3e}")
    assert err <= 1e-3
    assert serr <= 1e-3
    # the engine's token-by-token mode gives the same answer
    s = gpu_engine(hp, tensors, ctx=ctx)
    s.set_prefill_mode(True)
    ls = s.forward(prompt, 0)
    assert rel_l2(lg, ls) <= 1e-3
    return g, o, prompt, lg, lo


@pytest.mark.parametrize("n", [70, 200])
def test_prefill_wide_router(gpu, oracle, n):
    """48 experts top-4: the prefill routers' paths for more than 32 experts (at 70
    tokens the small call's; at 200 the large call's matrix-core router, whose second
    pass covers experts 32..47)."""
    hp = gpu.make_hparams(dim=256, heads=4, n_layers=2, attention_layers=(1,), kv=2, vocab=500,
                          eos=1 << 30, n_expert=48, n_used=4, expert_ff=256, n_ff=512,
                          dense_lead=1)
    tensors = model_tensors(hp, gpu.synth_opts(0x5EED, bias_sigma=0.1))
    check_prefill(gpu, oracle, hp, tensors, n, 256)


@pytest.mark.parametrize("n", [2, 24, 300])
def test_prefill_real_width(gpu, oracle, real_width, n):
    hp, tensors = real_width
    check_prefill(gpu, oracle, hp, tensors, n, ctx=512)


@pytest.mark.parametrize("n", [100, 128, 129, 400])
def test_prefill_crowded_experts(gpu, oracle, crowded, n):
    """8 experts top-2: at 100 and 128 tokens (small calls) experts hold more than one
    32-row tile of gathered activations; at 129 and 400 the large-call kernels run."""
    hp, tensors = crowded
    check_prefill(gpu, oracle, hp, tensors, n, ctx=512)


def test_prefill_chunks_then_decode(gpu, oracle, real_width):
    """Two batched chunks (the second at start > 0 reads the first's KV and conv
    state), then the device-resident greedy loop."""
    hp, tensors = real_width
    n, cut = 200, 130
    prompt = [int(t) for t in np.random.default_rng(7).integers(0, hp.vocab, n)]
    g = gpu_engine(hp, tensors, ctx=512)
    o = oracle_engine(oracle, hp, tensors, ctx=512)
    g.forward(prompt[:cut], 0)
    lg = g.forward(prompt[cut:], cut)
    lo = o.forward(prompt, 0)
    err = rel_l2(lg, lo)
    print(f"chunked prefill logits rel-L2 {err:.3e}")
    assert err <= 1e-3
    tol = 1e-3 * float(np.abs(lo).max())
    first = int(oracle.argmax(lg))
    if top2_margin(lo) > tol:
        assert first == oracle.argmax(lo)
    steps = 16
    toks = g.decode_run(first, n, steps)
    assert len(toks) == steps
    feed, compared = first, 0
    for s in range(steps):
        lo = o.forward([feed], n + s)
        if top2_margin(lo) > tol:
            assert toks[s] == oracle.argmax(lo), (s, toks[s], oracle.argmax(lo))
            compared += 1
        feed = toks[s]
    assert compared >= steps // 2


def test_prefill_64_token_chunks(gpu, oracle, real_width):
    """A 448-token prompt in 64-token chunks (api_stream.rs:57-63, work_bound.rs
    PREFILL_CHUNK): calls of up to 128 tokens take the split-K GEMM with 32-token
    tiles, and chunks from position 192 on split attention over key ranges.  The
    last logits and the resident state match the oracle and the engine's own
    whole-prompt forward."""
    hp, tensors = real_width
    n = 448
    prompt = [int(t) for t in np.random.default_rng(11).integers(0, hp.vocab, n)]
    g = gpu_engine(hp, tensors, ctx=512)
    for s in range(0, n, 64):
        lg = g.forward(prompt[s:s + 64], s)
    o = oracle_engine(oracle, hp, tensors, ctx=512)
    lo = o.forward(prompt, 0)
    err = rel_l2(lg, lo)
    sg = np.frombuffer(g.snapshot_resident_cache(n), np.float32)
    so = np.frombuffer(o.snapshot(n), np.float32)
    serr = rel_l2(sg, so)
    print(f"64-token chunks: logits rel-L2 {err:.3e}, state rel-L2 {serr:.3e}")
    assert err <= 1e-3
    assert serr <= 1e-3
    w = gpu_engine(hp, tensors, ctx=512)
    lw = w.forward(prompt, 0)
    assert rel_l2(lg, lw) <= 1e-3
    sw = np.frombuffer(w.snapshot_resident_cache(n), np.float32)
    assert rel_l2(sg, sw) <= 1e-3


def test_prefill_chunks_repeat_bit_exact(gpu, real_width):
    """Small calls take each token's slot in its experts' lists with an atomic add,
    so a token's row may sit elsewhere in its expert's tile from one run to the
    next; what is computed for it must not change: two engines prefilling the
    same 192 tokens in 64-token calls, then 300 more in one large call, give
    bit-identical logits and state."""
    hp, tensors = real_width
    prompt = [int(t) for t in np.random.default_rng(17).integers(0, hp.vocab, 492)]
    outs = []
    for _ in range(2):
        g = gpu_engine(hp, tensors, ctx=512)
        for s in range(0, 192, 64):
            lg = g.forward(prompt[s:s + 64], s)
        lw = g.forward(prompt[192:], 192)
        outs.append((lg.view(np.uint32).copy(), np.frombuffer(g.snapshot_resident_cache(192), np.uint32).copy(),
                     lw.view(np.uint32).copy(), np.frombuffer(g.snapshot_resident_cache(492), np.uint32).copy()))
        g.close()
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a, b)


def test_prefill_mixed_chunk_sizes(gpu, oracle, real_width):
    """One prompt in calls of 1, 127, 128, 129, 3 and 92 tokens: both sides of the
    128-token line between the split-K small-call GEMMs (one 32-row tile per wave up
    to 3072 rows, partial sums capped) and the large-call ones (64-token tiles for
    grids under 512 workgroups, which every projection here is), each call reading
    the KV and conv state the previous ones left.  The last logits and the resident
    state match the oracle's token-by-token forward and the engine's whole-prompt
    call."""
    hp, tensors = real_width
    sizes = [1, 127, 128, 129, 3, 92]
    n = sum(sizes)
    prompt = [int(t) for t in np.random.default_rng(23).integers(0, hp.vocab, n)]
    g = gpu_engine(hp, tensors, ctx=512)
    s = 0
    for c in sizes:
        lg = g.forward(prompt[s:s + c], s)
        s += c
    o = oracle_engine(oracle, hp, tensors, ctx=512)
    lo = o.forward(prompt, 0)
    err = rel_l2(lg, lo)
    sg = np.frombuffer(g.snapshot_resident_cache(n), np.float32)
    so = np.frombuffer(o.snapshot(n), np.float32)
    serr = rel_l2(sg, so)
    print(f"mixed chunks {sizes}: logits rel-L2 {err:.3e}, state rel-L2 {serr:.3e}")
    assert err <= 1e-3
    assert serr <= 1e-3
    w = gpu_engine(hp, tensors, ctx=512)
    lw = w.forward(prompt, 0)
    assert rel_l2(lg, lw) <= 1e-3


def test_prefill_full_int8_scales_model(gpu, oracle):
    """A real-width model whose Q6_K weights use the whole int8 scale range, as
    model files do (synthetic full_scales: one sub-block per super-block at -128).
    Its GEMMs take the split-scale kernels, so the whole-prompt call (large-call
    kernels, 300 tokens) and the same prompt in 64-token calls (small-call
    kernels) stay as close to the decode graph's stepwise forward (weights formed
    in fp32) as the synthetic model's prefill does, and match the oracle."""
    hp = gpu.make_hparams(dim=2048, heads=32, n_layers=4, attention_layers=(1, 3), kv=8,
                          vocab=4096, eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792,
                          n_ff=7168, dense_lead=1)
    tensors = model_tensors(hp, gpu.synth_opts(0x5EED, full_scales=1))
    raw = next(d for nm, _, _, d in tensors if nm == "blk.1.ffn_gate_exps.weight")
    sc = raw.reshape(-1, 210)[:, 192:208].view(np.int8)
    assert sc.min() == -128 and np.abs(sc.astype(int)).max() == 128
    n = 300
    prompt = [int(t) for t in np.random.default_rng(31).integers(0, hp.vocab, n)]
    g = gpu_engine(hp, tensors, ctx=512)
    lw = g.forward(prompt, 0)
    sw = np.frombuffer(g.snapshot_resident_cache(n), np.float32)
    g.reset_session()
    for s in range(0, n, 64):
        g.forward_token(prompt[s:s + 64], s)
    lc = g.snapshot_resident_logits()
    sc_ = np.frombuffer(g.snapshot_resident_cache(n), np.float32)
    g.reset_session()
    g.set_prefill_mode(True)
    ls = g.forward(prompt, 0)
    ss = np.frombuffer(g.snapshot_resident_cache(n), np.float32)
    g.close()
    o = oracle_engine(oracle, hp, tensors, ctx=512)
    lo = o.forward(prompt, 0)
    so = np.frombuffer(o.snapshot(n), np.float32)
    o.close()
    e = {"whole vs stepwise": (rel_l2(lw, ls), rel_l2(sw, ss)),
         "chunked vs stepwise": (rel_l2(lc, ls), rel_l2(sc_, ss)),
         "whole vs oracle": (rel_l2(lw, lo), rel_l2(sw, so)),
         "stepwise vs oracle": (rel_l2(ls, lo), rel_l2(ss, so))}
    print("full-scale model, logits / state rel-L2: "
          + "; ".join(f"{k} {a:.2e} / {b:.2e}" for k, (a, b) in e.items()))
    for k in ("whole vs stepwise", "chunked vs stepwise"):  # measured <= 3e-6
        assert e[k][0] <= 2e-5 and e[k][1] <= 2e-5, (k, e[k])
    for k in ("whole vs oracle", "stepwise vs oracle"):
        assert e[k][0] <= 1e-3 and e[k][1] <= 1e-3, (k, e[k])


def test_prefill_h16_copy_matches_q6_decode(gpu, real_width, monkeypatch):
    """The whole prompt with the large-call GEMMs on the binary16 fragment copies
    (the default) and with LFM_PREFILL_H16=0 (Q6_K decoded in registers, no copies
    made at finalize): logits and resident state bit-identical, at real widths
    (in_proj, out/o projections, q/k/v, dense and expert gate/up/down)."""
    hp, tensors = real_width
    prompt = [int(t) for t in np.random.default_rng(11).integers(0, hp.vocab, 300)]
    g = gpu_engine(hp, tensors, ctx=512)
    assert g.h16_bytes() > 0
    lg = g.forward(prompt, 0)
    sg = g.snapshot_resident_cache(len(prompt))
    g.close()
    monkeypatch.setenv("LFM_PREFILL_H16", "0")
    q = gpu_engine(hp, tensors, ctx=512)
    assert q.h16_bytes() == 0
    lq = q.forward(prompt, 0)
    sq = q.snapshot_resident_cache(len(prompt))
    q.close()
    assert np.array_equal(lg.view(np.uint32), lq.view(np.uint32))
    assert sg == sq


def test_forward_token_after_halted_decode(gpu, real_width):
    """A multi-token forward_token starts the decode state in its embedding launch
    (the ids travel in the launch's arguments, no state copy) and returns its
    result from pinned host memory: after a decode run that halted at its EOS
    token, the same call gives the same token and maximum logit, bit for bit, as
    on a fresh state, and so do the one-token call (decode graph) and the logits
    path."""
    hp, tensors = real_width
    g = gpu_engine(hp, tensors, ctx=512)
    prompt = [int(t) for t in np.random.default_rng(64).integers(0, hp.vocab, 64)]
    tok = g.forward_token(prompt, 0)
    val = g.last_max_logit
    first = g.decode_run(tok, 64, 2)
    assert len(first) == 2
    g.reset_session()
    one = g.forward_token(prompt[:1], 0)
    one_val = g.last_max_logit
    for _ in range(2):
        # halt: EOS is the token this continuation generates first
        g.reset_session()
        assert g.forward_token(prompt, 0) == tok
        assert g.decode_run(tok, 64, 4, eos=first[0]) == []
        g.reset_session()
        assert g.forward_token(prompt, 0) == tok
        assert np.float32(g.last_max_logit).tobytes() == np.float32(val).tobytes()
        assert g.decode_run(tok, 64, 4, eos=first[0]) == []
        g.reset_session()
        assert g.forward_token(prompt[:1], 0) == one
        assert np.float32(g.last_max_logit).tobytes() == np.float32(one_val).tobytes()
    g.reset_session()
    lg = g.forward(prompt, 0)
    assert int(np.argmax(lg)) == tok and np.float32(lg.max()).tobytes() == np.float32(val).tobytes()
