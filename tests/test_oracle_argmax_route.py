"""Pins greedy argmax (engine/src/main.rs:112-141, tests :287-317) and MoE routing
(engine/src/lfm.rs:613-637 with the GPU tie rule of kernels/resident.rs:58-99)."""
import numpy as np
import pytest


def lcg_bits(n, seed):
    """main.rs:299-305: seed = seed * 1664525 + 1013904223 (u32), value = f32::from_bits."""
    out = np.zeros(n, dtype=np.uint32)
    for i in range(n):
        seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = seed
    return out.view(np.float32), seed


def np_first_max(xs):
    """Scalar statement: first strictly greater value wins, NaN never, default 0."""
    best, value = 0, -np.inf
    for i, v in enumerate(xs):
        if v > value:
            best, value = i, v
    return best


def test_lane_argmax_matches_scalar_ties_nan_tails(oracle):
    seed = 17
    for n in range(257):
        xs, seed = lcg_bits(n, seed)
        xs = xs.copy()
        assert oracle.argmax(xs) == oracle.argmax_scalar(xs) == np_first_max(xs)
        for v in [np.nan, -np.inf, np.inf, 0.0, -0.0, 1.0]:
            xs.fill(v)
            assert oracle.argmax(xs) == oracle.argmax_scalar(xs) == np_first_max(xs)
        if n > 8:
            xs[7] = 2.0
            xs[8] = 2.0
            assert oracle.argmax(xs) == 7


@pytest.mark.parametrize("n", [1, 63, 513, 128003])
def test_argmax_lengths_and_specials(oracle, n):
    """optimization_check.rs:121-149 cases: NaN at 0, max at the last index."""
    rng = np.random.default_rng(n)
    xs = rng.standard_normal(n).astype(np.float32)
    xs[0] = np.nan
    xs[-1] = 100.0
    assert oracle.argmax(xs) == (n - 1 if n > 1 else 0) == np_first_max(xs)


def np_route(logits, bias, n_used):
    probs = (np.float32(1) / (np.float32(1) + np.exp(-logits.astype(np.float32)))).astype(np.float32)
    score = (probs + bias).astype(np.float32)
    order = sorted(range(len(score)), key=lambda e: (-float(score[e]), e))  # stable: low id first
    sel = order[:n_used]
    wsum = np.float32(0)
    for e in sel:
        wsum = np.float32(wsum + probs[e])
    wsum = max(wsum, np.float32(6.103515625e-5))
    return sel, np.array([probs[e] / wsum for e in sel], dtype=np.float32)


def test_route_matches_numpy_restatement(oracle):
    rng = np.random.default_rng(7)
    for trial in range(200):
        logits = (rng.standard_normal(32) * 2).astype(np.float32)
        bias = (rng.standard_normal(32) * 0.1).astype(np.float32) if trial % 2 else np.zeros(32, np.float32)
        sel, w, _ = oracle.route(logits, bias, 4)
        esel, ew = np_route(logits, bias, 4)
        assert sel == esel
        # exp differs from glibc expf in the last ulp at most
        assert np.allclose(w, ew, rtol=1e-6, atol=0)
        assert abs(float(np.sum(w, dtype=np.float64)) - 1.0) < 1e-5


def test_route_ties_prefer_lower_id_and_clamp(oracle):
    logits = np.zeros(32, np.float32)
    logits[[5, 9, 3, 30]] = 3.0  # four equal winners, any order in memory
    sel, w, _ = oracle.route(logits, np.zeros(32, np.float32), 4)
    assert sel == [3, 5, 9, 30]
    assert np.all(w == np.float32(0.25))
    # all-equal scores: ids 0..3; huge negative logits hit the 2^-14 clamp
    sel, w, _ = oracle.route(np.full(32, -200.0, np.float32), np.zeros(32, np.float32), 4)
    assert sel == [0, 1, 2, 3]
    assert np.all(w == np.float32(0.0))
    # bias reorders selection but not the weights' source (sigmoid probabilities)
    logits = np.linspace(-1, 1, 32).astype(np.float32)
    bias = np.zeros(32, np.float32)
    bias[0] = 10.0
    sel, w, _ = oracle.route(logits, bias, 4)
    assert sel[0] == 0 and sel[1:] == [31, 30, 29]
    p = 1 / (1 + np.exp(-logits.astype(np.float64)))
    assert np.allclose(w, p[sel] / p[sel].sum(), rtol=1e-6)


def test_powi_is_square_and_multiply(oracle):
    a = np.float32(np.power(np.float32(1e6), np.float32(-0.03125)))
    for p in range(32):
        r = np.float32(1.0)
        base, b = np.float32(a), p
        while True:
            if b & 1:
                r = np.float32(r * base)
            b //= 2
            if b == 0:
                break
            base = np.float32(base * base)
        assert oracle.powi(float(a), p) == r
        assert abs(float(r) / float(np.float64(a) ** p) - 1) < 1e-5


def test_route_layer_is_the_ffn_routing(oracle):
    """oracle_route_layer (the routing alone, used to check the GPU's fused router)
    is the routing run_ffn takes, and its logits match a float64 numpy statement of
    RMSNorm + the f32 router matmul (lfm.rs:599-607) to f32 rounding."""
    import lfm_hip
    from model_util import model_tensors, oracle_engine, small_hparams

    hp = small_hparams(kinds=("conv", "conv"), n_expert=16, dense_lead=1)
    tensors = model_tensors(hp, lfm_hip.synth_opts(0x51, bias_sigma=0.1))
    by_name = {name: data for name, _, _, data in tensors}
    o = oracle_engine(oracle, hp, tensors, ctx=8)
    norm_w = by_name["blk.1.ffn_norm.weight"].astype(np.float64)
    rw = by_name["blk.1.ffn_gate_inp.weight"].astype(np.float64).reshape(hp.n_expert, hp.dim)
    bias = by_name["blk.1.exp_probs_b.bias"].astype(np.float64)
    for s in range(20):
        x = lfm_hip.synth_normal(0x77 + s, "route.layer", hp.dim)
        ids, w, scores, logits = o.route_layer(1, x)
        o.run_ffn(1, x)
        ids2, w2, scores2 = o.last_route(1)
        assert ids == ids2 and np.array_equal(w, w2) and np.array_equal(scores, scores2)
        x64 = x.astype(np.float64)
        h = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * norm_w
        lg = rw @ h
        assert np.allclose(logits, lg, rtol=1e-5, atol=1e-6)
        p = 1.0 / (1.0 + np.exp(-lg))
        sc = p + bias
        assert np.allclose(scores, sc, rtol=0, atol=1e-6)
        order = np.argsort(-sc, kind="stable")
        if sc[order[3]] - sc[order[4]] > 1e-5:
            assert ids == [int(i) for i in order[:4]]
            assert np.allclose(w, p[order[:4]] / p[order[:4]].sum(), rtol=1e-5)
