"""The decode step's fused conv mixer against the kernel chain it replaces.

k_conv_mixer / k_conv_mixer_r (selected with LFM_FUSED_MIXER=1 at finalize;
the default step keeps the two-kernel chain, which measures faster) compute
every value exactly as k_conv_inproj4 followed by k_q6_matvec4 /
k_q6_matvec_route (same staging sums, lane products, reductions and
epilogues), so the step must be bit-identical either way: decode tokens,
per-step logits and the resident state.  The fused step runs fewer kernels,
which the dispatch counts show.
"""
import os

import numpy as np
import pytest

from model_util import model_tensors

pytestmark = pytest.mark.gpu


def engine(gpu, hp, tensors, fused):
    old = os.environ.get("LFM_FUSED_MIXER")
    os.environ["LFM_FUSED_MIXER"] = "1" if fused else "0"
    try:
        return gpu.GpuEngine.load(hp, tensors, ctx=256)
    finally:
        if old is None:
            os.environ.pop("LFM_FUSED_MIXER", None)
        else:
            os.environ["LFM_FUSED_MIXER"] = old


@pytest.mark.parametrize("dense_lead", [2, 1])
def test_fused_conv_mixer_bit_identical(gpu, dense_lead):
    """Conv layers 1 and 2 (a dense FFN after layer 1 when dense_lead = 2, MoE
    with the fused router otherwise), attention layer 3, real widths."""
    hp = gpu.make_hparams(dim=2048, heads=32, n_layers=4, attention_layers=(3,), kv=8,
                          vocab=4096, eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792,
                          n_ff=7168, dense_lead=dense_lead)
    tensors = model_tensors(hp)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, hp.vocab, 40)]
    runs = []
    for fused in (True, False):
        g = engine(gpu, hp, tensors, fused)
        first = int(np.argmax(g.forward(prompt, 0)))
        d0 = g.dispatch_count()
        toks = g.decode_run(first, len(prompt), 24, eos=1 << 31)
        per_step = (g.dispatch_count() - d0) // 24
        snap = g.snapshot_resident_cache(len(prompt) + 24)
        # one decode step per call from the prompt state: logits of every step
        g.restore_session(len(prompt) + 24, snap)
        logits = [g.forward([t], len(prompt) + 24 + i).view(np.uint32).copy() for i, t in enumerate(toks[:8])]
        runs.append((toks, snap, logits, per_step))
        g.close()
    (ft, fs, fl, fd), (ct, cs, cl, cd) = runs
    print(f"dense_lead {dense_lead}: fused step {fd} kernels, chain {cd}")
    assert ft == ct
    assert fs == cs
    assert all(np.array_equal(a, b) for a, b in zip(fl, cl))
    assert fd == cd - 2  # conv layers 1 and 2 run as one launch each
