"""Chunked prefill at depth against the oracle, decision by decision.

The reference's api_stream prefills a prompt in 64-token forward_token calls
(engine/src/bin/api_stream.rs:57-63); its qualification ran 3840 + 256 that way
(validation/qualification.json:93-124).  Here a real-width model (dim 2048, 32
experts top-4, ff 1792 / 7168; conv layers 0 and 2, GQA attention layers 1 and
3 at ctx 4096) takes a 1300-token prompt as twenty 64-token calls and a final
20-token call.  Every call runs the small-call path: split-K GEMMs at growing
positions, attention over key ranges out to 1300 keys, and the MoE routing that
the grouped split does itself from the out projection's router partial sums,
taking list slots with atomic adds.

Checks against the oracle run token by token over the same prompt:
* every routing decision (position, MoE layer) that the calls log: ids in rank
  order equal, except at near-ties -- a differing selection must be the first
  of its run (tests/route_audit.py) and lie within twice the score drift of the
  clean decisions; the drift itself is at most DRIFT_CAP; the weights of equal
  selections agree within 1e-6;
* the last layer routes only each call's last row (first row = T - 1);
* the last logits (rel-L2 <= 1e-3) and the resident state per layer
  (rel-L2 <= 1e-3 over the positions no flip touched) after the last call.
"""
import numpy as np
import pytest

from conftest import rel_l2
from model_util import gpu_engine, model_tensors, oracle_engine
from route_audit import Audit, sigmoid_scores, state_errors

pytestmark = pytest.mark.gpu

CTX = 4096
CHUNKS = [64] * 20 + [20]
# Largest score difference allowed between the GPU's small-call routing and the
# oracle's at a clean decision: the routing reads an FFN input that carries the
# prefill's binary16 hi + lo products and reassociated sums (rel. ~1e-6 per
# layer), scaled by |d score / d x| <= 0.25 * |logit| / ||x||.
DRIFT_CAP = 2e-5


@pytest.fixture(scope="module")
def deep(gpu):
    hp = gpu.make_hparams(dim=2048, heads=32, n_layers=4, attention_layers=(1, 3), kv=8,
                          vocab=4096, eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792,
                          n_ff=7168, dense_lead=1)
    return hp, model_tensors(hp)


def test_chunked_prefill_depth_against_oracle(gpu, oracle, deep):
    hp, tensors = deep
    n = sum(CHUNKS)
    moe = list(range(hp.dense_lead, hp.n_layers))
    bias = {l: next(d for nm, _, _, d in tensors if nm == f"blk.{l}.exp_probs_b.bias") for l in moe}
    prompt = [int(t) for t in np.random.default_rng(29).integers(0, hp.vocab, n)]

    g = gpu_engine(hp, tensors, ctx=CTX)
    g.set_route_log(True)
    routes = {}  # (pos, layer) -> (ids, weights, scores)
    s = 0
    for c in CHUNKS:
        g.forward_token(prompt[s:s + c], s)
        for l in moe:
            first, ids, w, lg = g.prefill_routes(l)
            assert lg is not None
            if l == hp.n_layers - 1:  # the last layer routes the call's last row only
                assert (first, len(ids)) == (c - 1, 1), (l, first, len(ids))
            else:
                assert (first, len(ids)) == (0, c), (l, first, len(ids))
            for j in range(len(ids)):
                routes[(s + first + j, l)] = (ids[j], w[j], sigmoid_scores(lg[j], bias[l]))
        s += c
    lg_gpu = g.snapshot_resident_logits()
    sg = g.snapshot_resident_cache(n)
    g.close()

    o = oracle_engine(oracle, hp, tensors, ctx=CTX)
    audit = Audit(hp.n_used)
    wdiff = 0.0
    for p in range(n):
        lo = o.forward([prompt[p]], p)
        for l in moe:
            if (p, l) not in routes:
                continue
            oids, ow, osc = o.last_route(l)
            ids, w, sc = routes[(p, l)]
            audit.add(p, l, ids, sc, oids, osc)
            if list(ids) == list(oids):
                wdiff = max(wdiff, float(np.abs(w - ow).max()))
    so = o.snapshot(n)
    o.close()

    drift = audit.clean_drift()
    print(f"chunked {n} tokens: {audit.summary()}; weights of equal selections within {wdiff:.2e}")
    for key in audit.first_flips():
        ids, ref_ids, d, m = audit.rows[key]
        print(f"  flip at position {key[0]} layer {key[1]}: gpu {ids} oracle {ref_ids}, oracle margin "
              f"{m:.2e}, score drift there {d:.2e}")
        assert m <= 2 * drift + 1e-6, (key, m, drift)
    assert drift <= DRIFT_CAP, drift
    assert wdiff <= 1e-6, wdiff

    err = rel_l2(lg_gpu, lo)
    errs, dropped = state_errors(hp, sg, so, n, audit.flips())
    print(f"last logits rel-L2 {err:.2e}; state per layer " + " ".join(f"{l}:{e:.1e}" for l, e in errs.items())
          + f" ({dropped} positions near flips left out)")
    assert err <= 1e-3
    assert max(errs.values()) <= 1e-3, errs
