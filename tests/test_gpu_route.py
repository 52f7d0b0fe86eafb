"""Expert selection of the decode step's own fused router, id for id, against the
oracle (engine/src/lfm.rs:599-637; GPU semantics engine/src/kernels/resident.rs:58-99;
the reference's hardware check engine/src/bin/resident_check.rs:35-84).

At the model's shape (dim 2048, 32 experts) the step does not run a router
kernel: the mixer's output projection (k_q6_matvec_route) leaves per-workgroup
partial sums of the router dot products and of x^2, and every wave of the
routed gate/up kernel (k_gateup8f) totals them, forms the logits and selects the
top 4.  lfm_engine_run_layer runs one layer exactly that way, returns the FFN
input x_mid, and the oracle routes the same x_mid with the reference's
arithmetic (f32 sequential RMSNorm and router matmul, expf sigmoid, stable
sort, clamped weight sum).

Selection contract (checked here over 2 x 1200 seeded inputs): the ids are
identical whenever the oracle's 4th and 5th selection scores differ by more than
ROUTE_MARGIN; the weights agree within 1e-6 (resident_check.rs:35-84).  Each
input gives the smallest margin seen and the count of near-ties below
ROUTE_MARGIN, which the test prints.
"""
import numpy as np
import pytest

from conftest import rel_l2
from model_util import gpu_engine, model_tensors, oracle_engine

pytestmark = pytest.mark.gpu

SEED = 0x9E3779B97F4A7C15
# The fused logits differ from the oracle's by reassociation of the 2048-term dot
# (256 partials of 8 rows) and the hardware reciprocal square root, and the
# sigmoid by the hardware exp2 / reciprocal: a few 1e-7 on a score.
ROUTE_MARGIN = 4e-6
N_INPUTS = 1200


def cfg1_hparams(gpu):
    # one conv layer (mixer) with the MoE FFN of the model: 32 experts, top 4, ff 1792
    return gpu.make_hparams(dim=2048, heads=32, n_layers=1, attention_layers=(), kv=8, vocab=256,
                            eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792, n_ff=256,
                            dense_lead=0)


@pytest.mark.parametrize("bias_sigma", [0.0, 0.1])
def test_fused_router_ids_match_oracle(gpu, oracle, bias_sigma):
    hp = cfg1_hparams(gpu)
    tensors = model_tensors(hp, gpu.synth_opts(SEED, bias_sigma=bias_sigma))
    g = gpu_engine(hp, tensors, ctx=16)
    o = oracle_engine(oracle, hp, tensors, ctx=16)
    assert g.fused_router(0), "the model's shape must take the fused router"
    min_margin, near, compared, worst_w, worst_ffn = np.inf, 0, 0, 0.0, 0.0
    for i in range(N_INPUTS):
        # residual scale varies over four decades so the logits do too
        scale = 10.0 ** ((i % 5) - 2)
        x = gpu.synth_normal(SEED + i, "route.x", hp.dim) * np.float32(scale)
        x_out, x_mid = g.run_layer(0, x, 0)
        ids_g, w_g = g.last_route()
        ids_o, w_o, scores, _ = o.route_layer(0, x_mid)
        srt = np.sort(scores)[::-1]
        margin = float(srt[3] - srt[4])
        min_margin = min(min_margin, margin)
        if margin <= ROUTE_MARGIN:
            near += 1
            continue
        compared += 1
        assert ids_g == ids_o, (i, scale, ids_g, ids_o, margin)
        worst_w = max(worst_w, float(np.abs(w_g - w_o).max()))
        assert np.allclose(w_g, w_o, rtol=0, atol=1e-6), (i, w_g, w_o)
        if i % 60 == 0:  # the FFN the step computed from this routing
            y_o = o.run_ffn(0, x_mid)
            err = rel_l2(x_out - x_mid, y_o - x_mid)
            worst_ffn = max(worst_ffn, err)
            assert err <= 1e-3, (i, err)
    print(f"bias {bias_sigma}: {compared}/{N_INPUTS} inputs compared id for id, 0 mismatches; "
          f"smallest 4th/5th score margin {min_margin:.3e}; {near} near-ties <= {ROUTE_MARGIN}; "
          f"max |w_gpu - w_oracle| {worst_w:.2e}; FFN rel-L2 <= {worst_ffn:.2e}")
    assert compared >= N_INPUTS - 10


def test_fused_and_unfused_routers_agree(gpu, oracle):
    """The single-half entry points (separate k_router + k_gateup4) and the
    step's fused router pick the same experts for the same FFN input."""
    hp = cfg1_hparams(gpu)
    tensors = model_tensors(hp, gpu.synth_opts(SEED, bias_sigma=0.1))
    g = gpu_engine(hp, tensors, ctx=16)
    o = oracle_engine(oracle, hp, tensors, ctx=16)
    for i in range(40):
        x = gpu.synth_normal(SEED + 7 * i, "route.y", hp.dim)
        _, x_mid = g.run_layer(0, x, 0)
        fused = g.last_route()
        g.run_ffn(0, x_mid)
        plain = g.last_route()
        _, _, scores, _ = o.route_layer(0, x_mid)
        srt = np.sort(scores)[::-1]
        if srt[3] - srt[4] > ROUTE_MARGIN:
            assert fused[0] == plain[0], (i, fused, plain)
            assert np.allclose(fused[1], plain[1], rtol=0, atol=1e-6)
