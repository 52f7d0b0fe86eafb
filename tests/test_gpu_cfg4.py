"""The full token loop at its real size against the oracle: 24 layers (conv
mixers, GQA attention at layers 2, 6, 10, 14, 18, 21), dense SwiGLU ff 7168 in
layers 0-1, MoE 32 experts top-4 ff 1792 in layers 2-23, vocab 65536 tied head,
seeded random Q6_K weights; a 3840-token prompt of uniform ids, then 256 greedy
tokens at positions 3840..4095 (ctx 4096).

The reference audits this workload teacher-forced, comparing every step's full
logits and requiring exact greedy tokens (engine/src/bin/teacher_audit.rs:6-17;
its qualification ran 3840 + 256 with 64-token prefill chunks,
validation/qualification.json:93-124, bin/api_stream.rs:57-63).  Running the
oracle's own 3840-token prefill is minutes of host work, so the prompt is
checked three ways on the GPU and the oracle is brought in where the paths
disagree:

* the prompt runs as one matrix-core call (whole), as sixty 64-token calls
  (chunked, the api_stream path) and as one decode step per token (stepwise,
  the decode graph's kernels); every routing decision (3840 positions x 22 MoE
  layers) of each path is logged and compared with the stepwise one;
* where two paths pick different experts, the oracle restored from the
  stepwise state at that position computes it: its 4th/5th score margin must
  be within twice the measured score drifts (tests/route_audit.py);
* the resident states match per layer (rel-L2 <= 1e-3) outside the positions
  such a flip touched, and the last logits and next tokens agree;
* position 3839 by the oracle restored at 3839 against the whole call.

The decode half: 256 greedy steps from the whole-prompt state, replayed
teacher-forced one token per call with their routing records; against the
oracle teacher-forced from the same state, every step's full logits (rel-L2 <=
1e-3 where no routing flip touched the step), every routing decision (flips
only at near-ties within twice the measured drift, drift <= DECODE_DRIFT_CAP),
tokens equal wherever the oracle's top-2 margin exceeds 1e-3 * max|logit|, and
the state at 4096.  The decode kernels' own records must also rank exactly by
the scores they logged.
"""
import os
import time

import numpy as np
import pytest

from conftest import rel_l2
from model_util import top2_margin
from route_audit import Audit, margin, reach, sigmoid_scores, state_errors, top_ids

pytestmark = pytest.mark.gpu

SEED = 0x9E3779B97F4A7C15
N_PROMPT, N_DECODE, CTX = 3840, 256, 4096
# Score drift caps at clean decisions (no flip reaches them, route_audit.Audit),
# about 2-3x the largest drift measured on the MI355X.  Decode vs oracle: both
# start from the same state at 3840; the drift grows with depth (3e-6 at layer
# 2 to 1.7e-5 at layer 23: the residual carries every layer's rounding) and
# over the first ~10 steps (the new positions' K/V and conv state), then stays
# level (1e-5 +- 0.5e-5 to step 255); after a flip every later position also
# attends to the flipped position's changed K/V.
# Whole or chunked prompt vs stepwise: two GPU paths over 3840 positions, whose
# states differ per layer by up to ~6e-5 rel-L2 outside flips (binary16 hi + lo
# products and reassociated sums in the GEMMs; measured 9.5e-6 and 6.8e-6).
DECODE_DRIFT_CAP = 3e-5
DECODE_CARRIED_CAP = 5e-5
PROMPT_DRIFT_CAP = 3e-5
ORACLE_STEP_CAP = 1e-5  # oracle vs the stepwise kernels from the same state, one position (3.6e-6)


def say(msg):
    print(f"[cfg4] {msg}", flush=True)


def check_flips(audit, label, extra_drift=None):
    """Every run-starting flip within twice the drift of the clean decisions
    (plus the oracle's own distance at that decision when given)."""
    drift = audit.clean_drift()
    say(f"{label}: {audit.summary()}")
    for key in audit.first_flips():
        ids, ref_ids, d, m = audit.rows[key]
        bar = 2 * (drift + (extra_drift or {}).get(key, 0.0)) + 1e-6
        say(f"  {label} {audit.kind(key)} flip at position {key[0]} layer {key[1]}: {ids} vs {ref_ids}, "
            f"margin {m:.2e} (bar {bar:.2e}), drift there {d:.2e}")
        assert m <= bar, (label, key, m, bar)
    return drift


def test_cfg4_full_size_against_oracle(gpu, oracle):
    t0 = time.perf_counter()
    hp = gpu.make_hparams()  # the model's geometry
    assert (hp.n_layers, hp.vocab, hp.dim, hp.n_expert) == (24, 65536, 2048, 32)
    opts = gpu.synth_opts(SEED)
    moe = list(range(hp.dense_lead, hp.n_layers))
    descs = {d.name.decode(): d for d in gpu.model_tensor_descs(hp, opts)}
    bias = {l: gpu.synth_tensor(descs[f"blk.{l}.exp_probs_b.bias"], opts) for l in moe}
    g = gpu.GpuEngine.load_synthetic(hp, opts, ctx=CTX, threads=16)
    g.set_route_log(True)
    prompt = [int(v) for v in np.random.default_rng(SEED & 0xFFFFFFFF).integers(0, hp.vocab, N_PROMPT)]
    say(f"GPU engine loaded ({time.perf_counter() - t0:.1f} s)")

    def call_routes(out, start):
        for l in moe:
            first, ids, _, lg = g.prefill_routes(l)
            for j in range(len(ids)):
                out[(start + first + j, l)] = (ids[j], sigmoid_scores(lg[j], bias[l]))

    # whole prompt in one matrix-core call (and the state after 3839 tokens)
    g.forward(prompt[:N_PROMPT - 1], 0)
    s3839 = g.snapshot_resident_cache(N_PROMPT - 1)
    g.reset_session()
    lg = g.forward(prompt, 0)
    s_whole = g.snapshot_resident_cache(N_PROMPT)
    whole = {}
    call_routes(whole, 0)
    first = int(oracle.argmax(lg))

    # the api_stream path: sixty 64-token forward_token calls
    g.reset_session()
    chunk = {}
    for s0 in range(0, N_PROMPT, 64):
        nxt_chunk = g.forward_token(prompt[s0:s0 + 64], s0)
        call_routes(chunk, s0)
    s_chunk = g.snapshot_resident_cache(N_PROMPT)

    # one decode step per token, with the decode kernels' routing records
    g.reset_session()
    step, inconsistent = {}, 0
    for p in range(N_PROMPT):
        g.forward_token([prompt[p]], p)
        for l, (ids, _, _, sc) in g.route_records().items():
            step[(p, l)] = (ids, sc)
            inconsistent += ids != top_ids(sc, hp.n_used)
    lst = g.snapshot_resident_logits()
    s_step = g.snapshot_resident_cache(N_PROMPT)
    say(f"whole, chunked and stepwise prompts done ({time.perf_counter() - t0:.1f} s)")
    assert inconsistent == 0, f"{inconsistent} decode routing records do not rank by their own scores"

    audits = {}
    for name, rec in (("whole", whole), ("chunked", chunk)):
        a = Audit(hp.n_used)
        for key, (ids, sc) in rec.items():
            a.add(key[0], key[1], ids, sc, *step[key])
        audits[name] = a
    assert len(audits["whole"].rows) == (N_PROMPT * (len(moe) - 1) + 1)
    assert len(audits["chunked"].rows) == N_PROMPT * (len(moe) - 1) + N_PROMPT // 64

    # stepwise state before every run-starting flip, for the oracle
    need = sorted({p for a in audits.values() for p, _ in a.first_flips()})
    snaps = {}
    if need:
        g.reset_session()
        g.set_prefill_mode(True)
        cur = 0
        for p in need:
            if p > cur:
                g.forward(prompt[cur:p], cur)
            snaps[p] = g.snapshot_resident_cache(p)
            cur = p
        g.set_prefill_mode(False)

    # decode: 256 greedy steps from the whole-prompt state, then the same tokens
    # replayed one per call with the routing records of every step
    g.restore_session(N_PROMPT, s_whole)
    toks = g.decode_run(first, N_PROMPT, N_DECODE, eos=1 << 31)
    assert len(toks) == N_DECODE
    s4096 = g.snapshot_resident_cache(CTX)
    g.restore_session(N_PROMPT, s_whole)
    glog = np.empty((N_DECODE, hp.vocab), dtype=np.float32)
    grec, feed = [], first
    for s in range(N_DECODE):
        glog[s] = g.forward([feed], N_PROMPT + s)
        grec.append(g.route_records())
        assert int(oracle.argmax(glog[s])) == toks[s], (s, toks[s])  # the graph's own kernels
        feed = toks[s]
    assert g.snapshot_resident_cache(CTX) == s4096
    g.close()
    say(f"GPU decode + replay done ({time.perf_counter() - t0:.1f} s)")

    oracle.set_threads(min(16, len(os.sched_getaffinity(0))))
    o = oracle.OracleEngine(hp, ctx=CTX, kv_f16=True)
    for d in descs.values():
        o.set_tensor(d.name.decode(), int(d.ggml_type), d.shape, gpu.synth_tensor(d, opts, threads=16))
    o.finalize()
    say(f"oracle loaded ({time.perf_counter() - t0:.1f} s)")

    # the oracle at every prompt position where two GPU paths route differently:
    # restored from the stepwise state there, it starts from the stepwise
    # kernels' own inputs, so their scores agree within ORACLE_STEP_CAP up to
    # the first layer where they themselves pick differently (a near-tie)
    ostep = Audit(hp.n_used)
    for p in need:
        o.restore(p, snaps[p])
        o.forward([prompt[p]], p)
        for l in moe:
            if (p, l) in step:
                oids, _, osc = o.last_route(l)
                ostep.add(p, l, *step[(p, l)], oids, osc)
    if need:
        check_flips(ostep, "stepwise vs oracle")
        assert ostep.clean_drift() <= ORACLE_STEP_CAP, ostep.clean_drift()
    oracle_gap = {k: r[2] for k, r in ostep.rows.items()}
    for name, a in audits.items():
        for key in a.first_flips():
            ids, oids, gap, ref_m = (a.rows[key][0],) + ostep.rows[key][1:]
            bar = 2 * (a.clean_drift() + gap) + 1e-6
            say(f"  oracle at {name} {a.kind(key)} flip {key}: oracle {oids}, stepwise {step[key][0]}, "
                f"{name} {ids}, oracle margin {ref_m:.2e} (bar {bar:.2e}), stepwise vs oracle {gap:.2e}")
            assert ref_m <= bar, (name, key, ref_m, bar)
    for name, a in audits.items():
        drift = check_flips(a, f"{name} vs stepwise", oracle_gap)
        assert drift <= PROMPT_DRIFT_CAP, (name, drift)

    # the prompt states and logits
    for name, snap in (("whole", s_whole), ("chunked", s_chunk)):
        errs, dropped = state_errors(hp, snap, s_step, N_PROMPT, audits[name].flips())
        say(f"{name} vs stepwise state per layer " + " ".join(f"{l}:{e:.1e}" for l, e in errs.items())
            + f" ({dropped} positions near flips left out)")
        assert max(errs.values()) <= 1e-3, (name, errs)
    cw = state_errors(hp, s_chunk, s_whole, N_PROMPT, audits["whole"].flips() + audits["chunked"].flips())[0]
    assert max(cw.values()) <= 1e-3, cw
    say(f"whole vs stepwise logits rel-L2 {rel_l2(lg, lst):.2e}; next token whole {first}, "
        f"chunked {nxt_chunk}")
    assert rel_l2(lg, lst) <= 1e-3
    if top2_margin(lg) > 1e-3 * float(np.abs(lg).max()):
        assert nxt_chunk == first

    o.restore(N_PROMPT - 1, s3839)
    lo = o.forward([prompt[-1]], N_PROMPT - 1)
    err = rel_l2(lg, lo)
    tol = 1e-3 * float(np.abs(lo).max())
    say(f"position 3839 logits rel-L2 {err:.2e}, top-2 margin {top2_margin(lo):.3e} (tol {tol:.3e})")
    assert err <= 1e-3
    if top2_margin(lo) > tol:
        assert first == oracle.argmax(lo)

    # decode, teacher-forced from the same state
    o.restore(N_PROMPT, s_whole)
    dec = Audit(hp.n_used)
    feed, compared, lerr = first, 0, np.zeros(N_DECODE)
    for s in range(N_DECODE):
        lo = o.forward([feed], N_PROMPT + s)
        lerr[s] = rel_l2(glog[s], lo)
        for l in moe:
            oids, _, osc = o.last_route(l)
            ids, _, _, sc = grec[s][l]
            assert ids == top_ids(sc, hp.n_used), (s, l)
            dec.add(N_PROMPT + s, l, ids, sc, oids, osc)
        tol = 1e-3 * float(np.abs(lo).max())
        if top2_margin(lo) > tol:
            assert toks[s] == oracle.argmax(lo), (s, toks[s], oracle.argmax(lo))
            compared += 1
        feed = toks[s]
        if s % 64 == 63:
            say(f"teacher-forced {s + 1}/{N_DECODE} steps, {compared} margin-clear tokens equal "
                f"({time.perf_counter() - t0:.1f} s)")
    so = o.snapshot(CTX)
    o.close()
    drift = check_flips(dec, "decode vs oracle")
    per_step = np.zeros(N_DECODE)
    per_layer = {l: 0.0 for l in moe}
    fl = dec.flips()
    for (p, l), r in dec.rows.items():
        if r[0] == r[1] and not dec.carried((p, l), fl):
            per_step[p - N_PROMPT] = max(per_step[p - N_PROMPT], r[2])
            per_layer[l] = max(per_layer[l], r[2])
    say("decode drift per step (every 8th): " + " ".join(f"{s}:{per_step[s]:.1e}" for s in range(0, N_DECODE, 8)))
    say("decode drift per layer: " + " ".join(f"{l}:{d:.1e}" for l, d in per_layer.items()))
    # level, not growing: the last 64 steps drift no more than twice the first 64
    assert per_step[-64:].max() <= 2 * per_step[:64].max(), (per_step[:64].max(), per_step[-64:].max())
    assert dec.pre_flip_drift() <= DECODE_DRIFT_CAP, dec.pre_flip_drift()
    assert drift <= DECODE_CARRIED_CAP, drift
    # the logits of a step read the residual after the last layer (layer 24's input)
    touched = {p - N_PROMPT for f in dec.flips() for p in reach(hp.n_layers, f)}
    clean = [s for s in range(N_DECODE) if s not in touched]
    worst = int(np.argmax(lerr))
    say(f"per-step logits rel-L2: worst {lerr[worst]:.2e} at step {worst}, worst clean "
        f"{lerr[clean].max():.2e} ({len(clean)} of {N_DECODE} steps clean); {compared}/{N_DECODE} "
        f"margin-clear tokens equal")
    assert lerr[clean].max() <= 1e-3
    assert compared >= N_DECODE * 3 // 4
    errs, dropped = state_errors(hp, s4096, so, CTX, dec.flips())
    say("state at 4096 vs oracle per layer " + " ".join(f"{l}:{e:.1e}" for l, e in errs.items())
        + f" ({dropped} positions near flips left out; {time.perf_counter() - t0:.1f} s)")
    assert max(errs.values()) <= 1e-3, errs
