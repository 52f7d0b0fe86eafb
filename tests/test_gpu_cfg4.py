"""The full token loop at its real size against the oracle: 24 layers (conv
mixers, GQA attention at layers 2, 6, 10, 14, 18, 21), dense SwiGLU ff 7168 in
layers 0-1, MoE 32 experts top-4 ff 1792 in layers 2-23, vocab 65536 tied head,
seeded random Q6_K weights; a 3840-token prompt of uniform ids prefilled in one
call, then 256 greedy tokens at positions 3840..4095 (ctx 4096).

The reference audits this workload with a teacher-forced, margin-checked run
(engine/src/bin/teacher_audit.rs:6-17; its qualification ran 3840 + 256,
validation/qualification.json:93-124).  Running the oracle's own 3840-token
prefill would take minutes of host work, so the oracle starts from the GPU's
state instead and checks every step it takes:

1. last prompt position: the oracle restored from the GPU's state after the
   first 3839 prompt tokens computes position 3839; its logits must match the
   whole-prompt GPU call's (rel-L2 <= 1e-3) and pick the same token when the
   top-2 margin is clear;
2. the whole-prompt (matrix-core) state at 3840 must match the state of the same
   prompt run one decode step per token (rel-L2 <= 1e-3 per layer, outside
   routing near-ties, below);
3. the oracle restored at 3840 is teacher-forced with the GPU's 256 tokens:
   tokens equal wherever the oracle's top-2 margin exceeds 1e-3 * max|logit|,
   and the resident state at 4096 matches (rel-L2 <= 1e-3 per layer outside
   routing near-ties).

Routing near-ties: expert ids are identical only where the 4th and 5th selection
scores are apart (the selection contract; the reassociated router sums differ in
the last bits).  Over 3840 x 22 routing decisions a few fall inside that margin;
a different expert at one position changes that position's residual, hence its
K/V in later attention layers and, through the 3-tap convolution, the next few
positions.  Such positions are found per position (largest K/V difference
against the state's rms above 1e-2) and come in short runs of consecutive
positions (the convolution state carries the difference on while it decays).
At most 1 % of positions may be such; in the decode comparison every run must
start at, or one position after, an oracle routing margin below 1e-4; and the
rel-L2 bar applies to the remaining positions.
"""
import os
import time

import numpy as np
import pytest

from conftest import rel_l2
from model_util import top2_margin

pytestmark = pytest.mark.gpu

SEED = 0x9E3779B97F4A7C15
N_PROMPT, N_DECODE, CTX = 3840, 256, 4096


def say(msg):
    print(f"[cfg4] {msg}", flush=True)


def layer_errors(hp, a, b, valid):
    """rel-L2 per layer of two reference-format snapshots (K then V per
    attention layer, [ch][2] conv state per conv layer)."""
    fa, fb = np.frombuffer(a, np.float32), np.frombuffer(b, np.float32)
    assert fa.size == fb.size
    out, off = [], 0
    for l in range(hp.n_layers):
        n = 2 * valid * 64 * hp.kv_heads[l] if hp.kv_heads[l] else 2 * hp.dim
        out.append(rel_l2(fa[off:off + n], fb[off:off + n]))
        off += n
    assert off == fa.size
    return out


OUTLIER_REL = 1e-2  # per position: max |K/V difference| / rms of the layer's state
OUTLIER_SHARE = 0.01
NEAR_TIE = 1e-4     # oracle 4th/5th routing score margin that can explain an outlier


def attention_positions(hp, a, b, valid):
    """Per attention layer: (K/V arrays [valid, kv*64] of both snapshots)."""
    fa, fb = np.frombuffer(a, np.float32), np.frombuffer(b, np.float32)
    out, off = {}, 0
    for l in range(hp.n_layers):
        kv = hp.kv_heads[l]
        if not kv:
            off += 2 * hp.dim
            continue
        n = valid * 64 * kv
        ka, kb = fa[off:off + n].reshape(valid, -1), fb[off:off + n].reshape(valid, -1)
        va, vb = fa[off + n:off + 2 * n].reshape(valid, -1), fb[off + n:off + 2 * n].reshape(valid, -1)
        out[l] = (np.concatenate([ka, va], axis=1), np.concatenate([kb, vb], axis=1))
        off += 2 * n
    return out


def outlier_positions(hp, a, b, valid):
    """Positions whose largest K/V difference (any attention layer) exceeds
    OUTLIER_REL times that layer's state rms."""
    bad = np.zeros(valid, dtype=bool)
    for l, (xa, xb) in attention_positions(hp, a, b, valid).items():
        rms = np.sqrt(np.mean(xb.astype(np.float64) ** 2))
        bad |= np.abs(xa - xb).max(axis=1) > OUTLIER_REL * rms
    return np.flatnonzero(bad)


def masked_errors(hp, a, b, valid, drop):
    """rel-L2 per attention layer over the positions not in `drop`."""
    keep = np.ones(valid, dtype=bool)
    keep[drop] = False
    return {l: rel_l2(xa[keep], xb[keep]) for l, (xa, xb) in attention_positions(hp, a, b, valid).items()}


def attention_detail(hp, a, b, valid, label):
    """For attention layers whose state differs by more than 1e-4: K and V
    separately, the binary16 ulp distance of the differing elements and where
    (position, kv head) the largest differences sit."""
    fa, fb = np.frombuffer(a, np.float32), np.frombuffer(b, np.float32)
    off = 0
    for l in range(hp.n_layers):
        kv = hp.kv_heads[l]
        if not kv:
            off += 2 * hp.dim
            continue
        n = valid * 64 * kv
        for part in ("K", "V"):
            xa, xb = fa[off:off + n], fb[off:off + n]
            off += n
            e = rel_l2(xa, xb)
            if e <= 1e-4:
                continue
            ha = xa.astype(np.float16).view(np.int16).astype(np.int32)
            hb = xb.astype(np.float16).view(np.int16).astype(np.int32)
            ulp = np.abs(ha - hb)
            diff = np.abs(xa - xb).reshape(valid, kv, 64)
            per_pos = diff.max(axis=(1, 2))
            worst = np.argsort(per_pos)[::-1][:4]
            say(f"{label} layer {l} {part}: rel-L2 {e:.2e}, |x| max {np.abs(xb).max():.3g} rms "
                f"{np.sqrt(np.mean(xb.astype(np.float64) ** 2)):.3g}; {np.count_nonzero(ulp)} of {n} "
                f"differ, ulp hist {np.bincount(np.minimum(ulp, 4))[1:].tolist()}; worst positions "
                + ", ".join(f"{int(p)}:{per_pos[p]:.3g}" for p in worst))


def test_cfg4_full_size_against_oracle(gpu, oracle):
    t0 = time.perf_counter()
    hp = gpu.make_hparams()  # the model's geometry
    assert (hp.n_layers, hp.vocab, hp.dim, hp.n_expert) == (24, 65536, 2048, 32)
    opts = gpu.synth_opts(SEED)
    g = gpu.GpuEngine.load_synthetic(hp, opts, ctx=CTX, threads=16)
    prompt = [int(v) for v in np.random.default_rng(SEED & 0xFFFFFFFF).integers(0, hp.vocab, N_PROMPT)]
    say(f"GPU engine loaded ({time.perf_counter() - t0:.1f} s)")

    g.forward(prompt[:N_PROMPT - 1], 0)
    s3839 = g.snapshot_resident_cache(N_PROMPT - 1)
    g.reset_session()
    lg = g.forward(prompt, 0)
    s3840 = g.snapshot_resident_cache(N_PROMPT)
    first = int(oracle.argmax(lg))
    g.reset_session()
    g.set_prefill_mode(True)
    lst = g.forward(prompt, 0)
    g.set_prefill_mode(False)
    s3840_step = g.snapshot_resident_cache(N_PROMPT)
    errs = layer_errors(hp, s3840, s3840_step, N_PROMPT)
    say(f"whole-prompt vs stepwise: logits rel-L2 {rel_l2(lg, lst):.2e}, state per layer "
        + " ".join(f"{l}:{e:.1e}" for l, e in enumerate(errs)))
    attention_detail(hp, s3840, s3840_step, N_PROMPT, "whole vs stepwise")
    assert rel_l2(lg, lst) <= 1e-3
    out = outlier_positions(hp, s3840, s3840_step, N_PROMPT)
    merr = masked_errors(hp, s3840, s3840_step, N_PROMPT, out)
    say(f"whole vs stepwise: {len(out)} routing-flip positions {out.tolist()[:12]}; attention "
        f"layers without them <= {max(merr.values()):.2e}")
    assert len(out) <= OUTLIER_SHARE * N_PROMPT
    assert max(merr.values()) <= 1e-3, merr
    assert max(e for l, e in enumerate(errs) if not hp.kv_heads[l]) <= 1e-3, errs

    g.restore_session(N_PROMPT, s3840)
    toks = g.decode_run(first, N_PROMPT, N_DECODE, eos=1 << 31)
    assert len(toks) == N_DECODE
    s4096 = g.snapshot_resident_cache(CTX)
    g.close()
    say(f"GPU prefill + stepwise + 256 decode done ({time.perf_counter() - t0:.1f} s)")

    oracle.set_threads(min(16, len(os.sched_getaffinity(0))))
    o = oracle.OracleEngine(hp, ctx=CTX, kv_f16=True)
    for d in gpu.model_tensor_descs(hp, opts):
        o.set_tensor(d.name.decode(), int(d.ggml_type), d.shape, gpu.synth_tensor(d, opts, threads=16))
    o.finalize()
    say(f"oracle loaded ({time.perf_counter() - t0:.1f} s)")

    o.restore(N_PROMPT - 1, s3839)
    lo = o.forward([prompt[-1]], N_PROMPT - 1)
    err = rel_l2(lg, lo)
    tol = 1e-3 * float(np.abs(lo).max())
    say(f"position 3839 logits rel-L2 {err:.2e}, top-2 margin {top2_margin(lo):.3e} (tol {tol:.3e})")
    assert err <= 1e-3
    if top2_margin(lo) > tol:
        assert first == oracle.argmax(lo)

    o.restore(N_PROMPT, s3840)
    feed, compared = first, 0
    moe_layers = list(range(hp.dense_lead, hp.n_layers))
    margin = np.zeros(N_DECODE)  # smallest 4th/5th routing score margin at each step
    for s in range(N_DECODE):
        lo = o.forward([feed], N_PROMPT + s)
        m = np.inf
        for l in moe_layers:
            srt = np.sort(o.last_route(l)[2])[::-1]
            m = min(m, float(srt[3] - srt[4]))
        margin[s] = m
        tol = 1e-3 * float(np.abs(lo).max())
        if top2_margin(lo) > tol:
            assert toks[s] == oracle.argmax(lo), (s, toks[s], oracle.argmax(lo))
            compared += 1
        feed = toks[s]
        if s % 64 == 63:
            say(f"teacher-forced {s + 1}/{N_DECODE} steps, {compared} margin-clear tokens equal "
                f"({time.perf_counter() - t0:.1f} s)")
    so = o.snapshot(CTX)
    errs = layer_errors(hp, s4096, so, CTX)
    attention_detail(hp, s4096, so, CTX, "decode vs oracle")
    o.close()
    say(f"{compared}/{N_DECODE} margin-clear tokens equal; state at 4096 per layer "
        + " ".join(f"{l}:{e:.1e}" for l, e in enumerate(errs)) + f"; {time.perf_counter() - t0:.1f} s")
    assert compared >= N_DECODE * 3 // 4
    out = outlier_positions(hp, s4096, so, CTX)
    merr = masked_errors(hp, s4096, so, CTX, out)
    say(f"decode vs oracle: smallest routing margin {margin.min():.2e} at position "
        f"{N_PROMPT + int(margin.argmin())}; routing-flip positions "
        + ", ".join(f"{p} (margin {margin[p - N_PROMPT]:.1e})" for p in out.tolist())
        + f"; attention layers without them <= {max(merr.values()):.2e}")
    assert len(out) <= OUTLIER_SHARE * CTX
    for p in out.tolist():
        assert p >= N_PROMPT, p  # the prompt positions were restored unchanged
        if p - 1 in out:
            continue  # inside a run: carried on by the convolution state
        # a run starts where a near-tie routed the position (or, for a flip after
        # the last attention layer, the position before) to another expert
        window = margin[max(0, p - N_PROMPT - 1):p - N_PROMPT + 1]
        assert window.min() < NEAR_TIE, (p, window)
    assert max(merr.values()) <= 1e-3, merr
    assert max(e for l, e in enumerate(errs) if not hp.kv_heads[l]) <= 1e-3, errs
