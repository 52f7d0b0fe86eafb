#!/usr/bin/env python3
"""Benchmark: batch-1 greedy decode of the synthetic LFM2.5-8B-A1B-shaped Q6_K
model at 4096 context on one MI355X, plus the Q6_K matvec HBM roofline and the
CPU restatement of the reference path timed on the host.

Workload: 24 layers (18 gated short-conv, 6 GQA at layers 2,6,10,14,18,21),
dense SwiGLU ff 7168 in layers 0-1, MoE 32 experts top-4 ff 1792 in layers
2-23, vocab 65536 tied Q6_K head; seeded random weights; a 3840-token prompt
of uniform ids prefilled in one call, then greedy decode at positions
3840..4095 (ctx 4096).  One step = one decode token.  The K timed steps run in
segments: each restores the resident state (untimed) to the end of the prompt,
takes the W warmup steps from there (untimed, positions 3840..3840+W-1) and
times the next at most 256 - W steps, so every timed token is a token of the
3840 + 256 workload whatever K is, and the timed steps follow warm ones.  The
whole 256-token decode from 3840 is also timed once, right after a restore
(cold), and reported as `decode_256`.

Prints one JSON line: metric, value (tok/s), ms_per_step, roofline of the
dominant kernel, the CPU baseline and prefill figures.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "lfm2-w9100-rust_amd"))

import lfm_hip  # noqa: E402

METRIC = "decode tok/s (bs=1, ctx 4096) + Q6_K matvec HBM GB/s vs ~8 TB/s peak"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense binary16 matrix-core peak
# HBM bytes per k_gateup8f launch from two rocprofv3 PMC passes over this bench
# (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0 KiB per dispatch; the scales are what the two
# counters read for a plain 512 MiB copy), and the SHA-256 of the decode code object
# those passes ran: the figure is reported only for that same code object.
GATEUP_TRAFFIC_BYTES = 24579564
GATEUP_TRAFFIC_CODE_OBJECT = "03d8e3b9b411c98add4de5827727c985eec1ff7da8579b7fe648957e4cd8471c"
SEED = 0x9E3779B97F4A7C15
CTX = 4096          # context of the workload (positions 0..4095)
N_PROMPT = 3840     # prompt tokens prefilled before decode
DECODE_TOKENS = 256  # greedy tokens of the workload (positions 3840..4095)
PREFILL_SAMPLE = 64  # prompt tokens the CPU baseline prefills (a bounded sample)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def decode_segments(steps, start=N_PROMPT, ctx=CTX):
    """Lengths of the decode runs that make up `steps` timed steps: each run
    starts at `start` (after a state restore) and stays below ctx."""
    if steps < 1:
        raise ValueError("steps must be >= 1")
    span = ctx - start
    if span < 1:
        raise ValueError("no decode positions left between start and ctx")
    full, rest = divmod(steps, span)
    return [span] * full + ([rest] if rest else [])


def cpu_decode_steps(max_steps, n_gpu_tokens, start, ctx=CTX):
    """How many teacher-forced oracle steps can run: one per GPU token, at
    positions start.. below ctx, at most max_steps."""
    return max(0, min(max_steps, n_gpu_tokens, ctx - start))


def affinity_cores():
    """Host threads this process may use: the affinity mask, capped by
    OMP_NUM_THREADS when the environment sets it."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def decode_bytes_per_token(hp, positions):
    """Algorithmic HBM bytes of one decode step: every weight read once (the head
    reads the whole tied embedding; 4 of 32 experts per MoE layer), the token's
    embedding row, and the binary16 K/V of positions 0..p of each attention layer."""
    w = 0
    for d in lfm_hip.model_tensor_descs(hp):
        nb = lfm_hip.lib().lfm_tensor_nbytes(d)
        if d.n_dims == 3:
            nb = nb * hp.n_used // hp.n_expert
        if d.name == b"token_embd.weight":
            nb += hp.dim // 256 * 210
        w += nb
    n_attn = sum(1 for l in range(hp.n_layers) if hp.kv_heads[l])
    kv = np.mean([n_attn * 2 * 8 * 64 * 2 * (p + 1) for p in positions])
    return int(w), float(kv)


def prefill_flops(hp, n):
    """Algorithmic FLOPs of prefilling n tokens (2 per multiply-add): every
    projection of every token (4 of 32 experts per MoE token), the router, the
    causal attention scores and value sums, and the head for the last token."""
    dim, macs = hp.dim, 0
    for l in range(hp.n_layers):
        kv = hp.kv_heads[l]
        if kv:
            macs += n * (2 * dim * dim + 2 * 64 * kv * dim)
            macs += 2 * 64 * hp.heads * n * (n + 1) // 2  # q.k and p.v over positions 0..t
        else:
            macs += n * 4 * dim * dim
        if l < hp.dense_lead:
            macs += n * 3 * hp.n_ff * dim
        else:
            macs += n * (hp.n_expert * dim + hp.n_used * 3 * hp.expert_ff * dim)
    macs += hp.vocab * dim
    return 2 * macs


def code_object_sha256():
    import hashlib
    path = os.path.join(REPO, "lfm2-w9100-rust_amd", "lfm_kernels.hsaco")
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def matvec_roofline(iters=200):
    """6144x2048 Q6_K matvec kernel, 64 rotating weight copies (660 MB > the
    256 MB Infinity Cache), HIP-event timing on the launch stream."""
    rows, in_dim, ncopies = 6144, 2048, 64
    size = lfm_hip.q6k_nbytes(rows, in_dim)
    raw = lfm_hip.synth_q6k_blocks(SEED, "cfg0.weight", rows * in_dim // 256, threads=16)
    packed = lfm_hip.q6k_pack(raw, rows, in_dim)
    wbuf = lfm_hip.DeviceBuffer(size * ncopies)
    for c in range(ncopies):
        wbuf.upload(packed, c * size)
    x = lfm_hip.DeviceBuffer.from_array(lfm_hip.synth_normal(SEED, "cfg0.x", in_dim))
    y = lfm_hip.DeviceBuffer(rows * 4)
    ms_hbm = lfm_hip.q6k_matvec_time(wbuf, ncopies, rows, in_dim, x, y, iters)
    ms_mall = lfm_hip.q6k_matvec_time(wbuf, 1, rows, in_dim, x, y, iters)
    algo = size + in_dim * 4 + rows * 4  # 10 354 688 B
    wbuf.free()
    return algo, ms_hbm, ms_mall


def full_scale_prefill(hp, prompt):
    """The same prompt through a model whose Q6_K sub-block scales span the whole
    int8 range with one -128 per super-block, as model files have them: its GEMMs
    run the split-scale kernels (exact binary16 weights for every scale)."""
    e = lfm_hip.GpuEngine.load_synthetic(hp, lfm_hip.synth_opts(SEED, full_scales=1), ctx=CTX,
                                         threads=16)
    e.forward(prompt[:256], 0)  # untimed: first launches
    e.reset_session()
    lfm_hip.lib().lfm_dev_synchronize()
    t = time.perf_counter()
    logits = e.forward(prompt, 0)
    lfm_hip.lib().lfm_dev_synchronize()
    whole = time.perf_counter() - t
    e.reset_session()
    lfm_hip.lib().lfm_dev_synchronize()
    t = time.perf_counter()
    for s0 in range(0, len(prompt), 64):
        nxt = e.forward_token(prompt[s0:s0 + 64], s0)
    lfm_hip.lib().lfm_dev_synchronize()
    chunked = time.perf_counter() - t
    e.close()
    flops = prefill_flops(hp, len(prompt))
    return {"tokens": len(prompt), "ms": round(whole * 1e3, 1), "tok_s": round(len(prompt) / whole, 1),
            "algorithmic_tflops": round(flops / whole / 1e12, 1),
            "mfma_frac": round(flops / whole / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "chunked_ms": round(chunked * 1e3, 1),
            "next_token_equals_whole_prompt": nxt == int(np.argmax(logits)),
            "note": "synthetic weights with int8 sub-block scales over the whole range (one -128 per "
                    "super-block): the GEMMs run the split-scale kernels, four matrix-core passes "
                    "per product"}


# ---------------------------------------------------------------- CPU baseline
def _timed(fn, min_s, max_reps):
    """Mean seconds per call of fn() over at least one call, repeated until
    min_s has passed or max_reps calls ran; returns (seconds, last result)."""
    out, reps = None, 0
    t0 = time.perf_counter()
    while True:
        out = fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_s or reps >= max_reps:
            return dt / reps, out


def _layer_hparams(**kw):
    base = dict(dim=2048, heads=32, n_layers=1, attention_layers=(), kv=8, vocab=256,
                eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792, n_ff=256, dense_lead=0)
    base.update(kw)
    return lfm_hip.make_hparams(**base)


def _oracle_engine(lfm_oracle, hp, opts, ctx, threads):
    o = lfm_oracle.OracleEngine(hp, ctx=ctx, kv_f16=True)
    for d in lfm_hip.model_tensor_descs(hp, opts):
        o.set_tensor(d.name.decode(), int(d.ggml_type), d.shape,
                     lfm_hip.synth_tensor(d, opts, threads=threads))
    o.finalize()
    return o


def cpu_layer_baselines(lfm_oracle, cores):
    """The single-op configurations on the oracle, on 1 thread (the reference's
    CPU path is single-threaded) and on `cores` threads; the multi-threaded
    results must be bit-identical to the 1-thread ones (only independent rows
    and heads are split)."""
    res = {}

    def both(name, setup, run, unit_bytes=None, min_s=0.3, max_reps=20):
        state = setup()
        out = {}
        ref = None
        for th in (1, cores):
            lfm_oracle.set_threads(th)
            sec, val = _timed(lambda: run(state), min_s, max_reps)
            key = "1_thread" if th == 1 else f"{th}_threads"
            out[key] = {"us": round(sec * 1e6, 1)}
            if unit_bytes:
                out[key]["gbs"] = round(unit_bytes / sec / 1e9, 3)
            if ref is None:
                ref = val
            else:
                out["bit_identical"] = bool(np.array_equal(ref.view(np.uint32), val.view(np.uint32)))
        res[name] = out
        if not out["bit_identical"]:
            raise RuntimeError(f"oracle {name}: {cores}-thread result differs from 1 thread")

    # cfg0: 6144x2048 Q6_K matvec, f64 accumulation (q6k.rs:161-183)
    def s0():
        raw = lfm_hip.synth_q6k_blocks(SEED, "cfg0.weight", 6144 * 2048 // 256, threads=cores)
        return raw, lfm_hip.synth_normal(SEED, "cfg0.x", 2048)
    both("cfg0_q6k_matvec_6144x2048", s0, lambda s: lfm_oracle.q6k_matvec(s[0], 2048, 6144, s[1]),
         unit_bytes=10354688)

    # cfg1: one MoE FFN step (RMSNorm, router, top-4, 4 x SwiGLU experts, combine)
    def s1():
        hp = _layer_hparams()
        o = _oracle_engine(lfm_oracle, hp, lfm_hip.synth_opts(SEED), 16, cores)
        return o, lfm_hip.synth_normal(SEED, "cfg1.h", hp.dim)
    both("cfg1_moe_step", s1, lambda s: s[0].run_ffn(0, s[1]), min_s=0.5, max_reps=10)

    # cfg2: attention layer at L = 4096 (query at position 4095)
    def s2():
        hp = _layer_hparams(attention_layers=(0,), dense_lead=1)
        o = _oracle_engine(lfm_oracle, hp, lfm_hip.synth_opts(SEED), CTX, cores)
        p = CTX - 1
        kv = lfm_hip.synth_normal(SEED, "cfg2.kv4096", 2 * p * 8 * 64).astype(np.float16)
        snap = kv.astype(np.float32).tobytes()
        return o, p, snap, lfm_hip.synth_normal(SEED, "cfg2.x4096", hp.dim)

    def r2(s):
        o, p, snap, x = s
        o.restore(p, snap)
        return o.run_mixer(0, x, p)
    both("cfg2_attention_L4096", s2, r2, min_s=0.5, max_reps=10)

    # cfg3: gated short-conv block, one token from a seeded 2-slot state
    def s3():
        hp = _layer_hparams(dense_lead=1)
        o = _oracle_engine(lfm_oracle, hp, lfm_hip.synth_opts(SEED), 512, cores)
        state = lfm_hip.synth_normal(SEED, "cfg3.state", hp.dim * 2).tobytes()
        return o, state, lfm_hip.synth_normal(SEED, "cfg3.x", hp.dim)

    def r3(s):
        o, state, x = s
        o.restore(0, state)
        return o.run_mixer(0, x, 0)
    both("cfg3_shortconv_step", s3, r3, min_s=0.3, max_reps=20)
    return res


def cpu_baseline(hp, snapshot, start_pos, gpu_tokens, first, cores, prompt, budget_s=12.0,
                 max_steps=128):
    """The oracle (C restatement of the reference CPU path) on the host cores:
    resident state restored from the GPU at the end of the prompt, then greedy
    decode steps teacher-forced with the GPU's tokens until ~budget_s, at most
    one per GPU token and never past ctx.  Also times the single-op
    configurations on 1 thread and on all cores."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import lfm_oracle

    t_layers = time.perf_counter()
    layers = cpu_layer_baselines(lfm_oracle, cores)
    log(f"[bench] cpu single-op configurations timed in {time.perf_counter() - t_layers:.1f} s")

    lfm_oracle.set_threads(cores)
    o = _oracle_engine(lfm_oracle, hp, lfm_hip.synth_opts(SEED), CTX, cores)
    # prefill sample: the prompt's first PREFILL_SAMPLE tokens in one forward from an
    # empty state (the whole 3840-token prompt is minutes of host work)
    tp = time.perf_counter()
    o.forward(prompt[:PREFILL_SAMPLE], 0)
    pdt = time.perf_counter() - tp
    o.restore(start_pos, snapshot)
    limit = cpu_decode_steps(max_steps, len(gpu_tokens), start_pos)
    feed, steps, agree, compared = first, 0, 0, 0
    t0 = time.perf_counter()
    while steps < limit and time.perf_counter() - t0 < budget_s:
        lo = o.forward([feed], start_pos + steps)
        srt = np.sort(lo)
        if srt[-1] - srt[-2] > 1e-3 * np.abs(lo).max():
            compared += 1
            agree += int(lfm_oracle.argmax(lo) == gpu_tokens[steps])
        feed = gpu_tokens[steps]
        steps += 1
    dt = time.perf_counter() - t0
    o.close()
    return {"value": round(steps / dt, 3) if steps else None, "unit": "tok/s", "cores": cores,
            "kind": "port",
            "sample": f"{steps} greedy decode steps of the full model at positions "
                      f"{start_pos}..{start_pos + steps - 1} (ctx {CTX}) on {cores} threads, "
                      f"oracle state restored from the GPU after the {start_pos}-token prefill, "
                      f"teacher-forced with the GPU's tokens; {dt:.1f} s",
            "tokens_compared": compared, "tokens_agree": agree,
            "single_op": layers,
            "prefill": {"tokens": PREFILL_SAMPLE, "positions": f"0..{PREFILL_SAMPLE - 1}",
                        "s": round(pdt, 2), "tok_s": round(PREFILL_SAMPLE / pdt, 2), "cores": cores,
                        "note": "the prompt's first tokens in one forward from an empty state; "
                                "the whole 3840-token prefill is minutes of host work"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=DECODE_TOKENS)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--no-decode-256", action="store_true",
                    help="skip the extra full 256-token decode pass reported as decode_256 (not part "
                         "of value; traced runs use it: a rocprofv3 kernel trace once faulted on a "
                         "host-side buffer inside one 256-replay decode call)")
    ap.add_argument("--no-full-scale", action="store_true",
                    help="skip the second prefill figure (the model with full-range int8 scales)")
    ap.add_argument("--synthetic-state", action="store_true",
                    help="skip the prefill: restore a seeded binary16 KV / conv state for the "
                         "prompt positions instead (isolates decode kernels for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the batch-1 decode path runs on a single GPU and is "
              "not sharded here; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        sys.exit("--steps must be >= 1 and --warmup >= 0")
    assert lfm_hip.device_count() > 0, "no HIP device"
    cores = affinity_cores()

    hp = lfm_hip.make_hparams()
    t = time.perf_counter()
    eng = lfm_hip.GpuEngine.load_synthetic(hp, lfm_hip.synth_opts(SEED), ctx=CTX, threads=16)
    log(f"[bench] model generated + uploaded in {time.perf_counter() - t:.1f} s on {eng.device_name}")
    n_prompt = N_PROMPT
    prompt = [int(v) for v in np.random.default_rng(SEED & 0xFFFFFFFF).integers(0, hp.vocab, n_prompt)]

    t = time.perf_counter()
    if args.synthetic_state:
        nbytes = eng.snapshot_bytes(n_prompt)
        state = lfm_hip.synth_normal(SEED, "bench.state", nbytes // 4, threads=16)
        eng.restore_session(n_prompt, state.astype(np.float16).astype(np.float32).tobytes())
        first = prompt[-1]
    else:
        eng.forward(prompt[:256], 0)  # untimed: first launches of the prefill kernels
        eng.reset_session()
        lfm_hip.lib().lfm_dev_synchronize()
        t = time.perf_counter()
        logits = eng.forward(prompt, 0)  # one batched matrix-core prefill of the prompt
        first = int(np.argmax(logits))
    prefill_s = time.perf_counter() - t
    pf_flops = prefill_flops(hp, n_prompt)
    log(f"[bench] {'state restore' if args.synthetic_state else 'prefill'} {n_prompt} tokens: "
        f"{prefill_s * 1e3:.1f} ms")
    snap = eng.snapshot_resident_cache(n_prompt)

    if args.warmup >= CTX - n_prompt:
        sys.exit(f"--warmup must leave decode positions: at most {CTX - n_prompt - 1}")
    # timed: K steps in runs that each restore the prompt state, take the W warmup
    # steps from it (untimed) and time the steps that follow
    toks, dt, fdt = [], 0.0, None
    t_start = n_prompt + args.warmup  # first timed position
    for seg in decode_segments(args.steps, start=t_start):
        eng.restore_session(n_prompt, snap)
        warm, feed = [], first
        if args.warmup:
            warm = eng.decode_run(first, n_prompt, args.warmup, eos=1 << 31)
            feed = warm[-1]
        lfm_hip.lib().lfm_dev_synchronize()
        t0 = time.perf_counter()
        out = eng.decode_run(feed, t_start, seg, eos=1 << 31)
        lfm_hip.lib().lfm_dev_synchronize()
        sdt = time.perf_counter() - t0
        dt += sdt
        assert len(warm) == args.warmup and len(out) == seg
        if not toks:
            toks = warm + out  # the tokens of positions 3840 ..
            if args.warmup == 0 and seg == DECODE_TOKENS:
                fdt = sdt
        elif warm + out != toks[:args.warmup + seg]:
            raise RuntimeError("decode from the same state gave different tokens")
    ms_per_step = dt * 1e3 / args.steps
    tok_s = args.steps / dt
    timed_pos = range(t_start, t_start + min(args.steps, CTX - t_start))
    wbytes, kvbytes = decode_bytes_per_token(hp, timed_pos)
    decode_gbs = (wbytes + kvbytes) * tok_s / 1e9
    log(f"[bench] decode {args.steps} steps: {ms_per_step:.3f} ms/step, {tok_s:.1f} tok/s, "
        f"{decode_gbs:.0f} GB/s algorithmic")

    decode_256 = None
    if fdt is None and not args.no_decode_256:
        eng.restore_session(n_prompt, snap)
        lfm_hip.lib().lfm_dev_synchronize()
        t0 = time.perf_counter()
        full = eng.decode_run(first, n_prompt, DECODE_TOKENS, eos=1 << 31)
        lfm_hip.lib().lfm_dev_synchronize()
        fdt = time.perf_counter() - t0
        if full[:len(toks)] != toks:
            raise RuntimeError("decode from the same state gave different tokens")
        toks = full
    if fdt is not None:
        fw, fkv = decode_bytes_per_token(hp, range(n_prompt, CTX))
        decode_256 = {"tokens": DECODE_TOKENS, "positions": f"{n_prompt}..{CTX - 1}",
                      "ms": round(fdt * 1e3, 2), "tok_s": round(DECODE_TOKENS / fdt, 1),
                      "hbm_gbs_algorithmic": round((fw + fkv) * DECODE_TOKENS / fdt / 1e9, 1)}
        log(f"[bench] decode 256 tokens at {n_prompt}..{CTX - 1}: {fdt * 1e3:.1f} ms")

    chunked = None
    if not args.synthetic_state:
        # the same prompt as 64-token lfm_forward_token calls, the chunking the
        # reference's api_stream uses (work_bound.rs PREFILL_CHUNK)
        eng.reset_session()
        lfm_hip.lib().lfm_dev_synchronize()
        t = time.perf_counter()
        for s0 in range(0, n_prompt, 64):
            nxt = eng.forward_token(prompt[s0:s0 + 64], s0)
        lfm_hip.lib().lfm_dev_synchronize()
        cs = time.perf_counter() - t
        chunked = {"tokens": n_prompt, "chunk": 64, "ms": round(cs * 1e3, 1),
                   "tok_s": round(n_prompt / cs, 1), "next_token_equals_whole_prompt": nxt == first}
        log(f"[bench] prefill {n_prompt} tokens in 64-token chunks: {cs * 1e3:.1f} ms")

    roof = None
    extra = {}
    if not args.no_roofline:
        # dominant kernel of the decode step: routed MoE gate/up (k_gateup8f, router
        # fused), timed with HIP events over a graph of its launches across all 22
        # MoE layers' experts
        us, nbytes = eng.time_moe_gateup(reps=10)
        gbs = nbytes / (us * 1e-6) / 1e9
        same_build = code_object_sha256() == GATEUP_TRAFFIC_CODE_OBJECT
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4),
                "traffic": GATEUP_TRAFFIC_BYTES if same_build else None,
                "traffic_source": "profiles/k_gateup_traffic.md, FETCH_SIZE / WRITE_SIZE passes over this "
                                  "code object (sha256 " + GATEUP_TRAFFIC_CODE_OBJECT[:12] + ")"
                                  if same_build else "null: the code object differs from the one the "
                                  "PMC passes measured",
                "kernel": "k_gateup8f (MoE router total + top-4 + routed gate+up+SwiGLU, "
                          "4 experts x 2 x 1792x2048 Q6_K)",
                "algorithmic_bytes": nbytes, "us_per_launch": round(us, 3),
                "timing": "HIP events over a graph of 220 launches (launch gaps included)"}
        log(f"[bench] k_gateup8f (MoE): {us:.2f} us/launch = {gbs:.0f} GB/s")
        # largest single Q6_K matvec of a step: final norm + tied head (vocab x 2048),
        # over 3 rotating copies of the embedding planes (beyond the Infinity Cache)
        hus, hbytes = eng.time_head(ncopies=3, reps=15)
        hgbs = hbytes / (hus * 1e-6) / 1e9
        extra["q6k_head"] = {
            "kernel": "k_head4 (final RMSNorm + %dx%d tied head + argmax partials)" % (hp.vocab, hp.dim),
            "algorithmic_bytes": hbytes, "us_per_launch": round(hus, 3), "hbm_gbs": round(hgbs, 1),
            "frac_of_peak": round(hgbs / HBM_PEAK_GBS, 4),
            "timing": "HIP events over a graph of 45 launches rotating 3 weight copies (gaps included)"}
        log(f"[bench] k_head4: {hus:.2f} us/launch = {hgbs:.0f} GB/s ({hgbs / HBM_PEAK_GBS:.1%} of 8 TB/s)")
        algo, ms_hbm, ms_mall = matvec_roofline()
        extra["q6k_matvec_6144x2048"] = {
            "shape": "6144x2048", "algorithmic_bytes": algo,
            "us_per_launch": round(ms_hbm * 1e3, 3),
            "hbm_gbs": round(algo / (ms_hbm * 1e-3) / 1e9, 1),
            "cache_resident_gbs": round(algo / (ms_mall * 1e-3) / 1e9, 1),
            "timing": "HIP events over 200 back-to-back launches (launch gaps included)"}
        copy_bytes = 512 << 20
        copy_us = lfm_hip.copy_time(copy_bytes, reps=10)
        extra["hbm_copy"] = {"bytes_each_way": copy_bytes, "us": round(copy_us, 2),
                             "gbs_read_plus_write": round(2 * copy_bytes / (copy_us * 1e-6) / 1e9, 1)}
        log(f"[bench] plain copy {copy_bytes >> 20} MiB: {copy_us:.1f} us = "
            f"{extra['hbm_copy']['gbs_read_plus_write']:.0f} GB/s read+write")
        log(f"[bench] q6k matvec 6144x2048: {ms_hbm * 1e3:.2f} us/launch = "
            f"{extra['q6k_matvec_6144x2048']['hbm_gbs']:.0f} GB/s (HBM, 64 rotating copies), "
            f"{extra['q6k_matvec_6144x2048']['cache_resident_gbs']:.0f} GB/s cache-resident")

    # the engine is released here, while the runtime (and a tracer attached to
    # it) is up, not by its finalizer at interpreter exit
    eng.close()
    full_scale = None
    if not args.synthetic_state and not args.no_full_scale:
        full_scale = full_scale_prefill(hp, prompt)
        log(f"[bench] full-range scales: prefill {n_prompt} tokens {full_scale['ms']} ms, in 64-token "
            f"chunks {full_scale['chunked_ms']} ms")
    cpu = None
    if not args.no_cpu_baseline:
        log(f"[bench] cpu baseline (oracle) on {cores} threads ...")
        cpu = cpu_baseline(hp, snap, n_prompt, toks, first, cores, prompt)
        log(f"[bench] cpu baseline {cpu['value']} tok/s on {cpu['cores']} threads, "
            f"{cpu['tokens_agree']}/{cpu['tokens_compared']} margin-clear tokens agree")

    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded random-init Q6_K weights and prompt ids)",
        "config": {"workload": f"prefill {n_prompt} + {DECODE_TOKENS} greedy decode steps at "
                               f"ctx {CTX} (LFM2.5-8B-A1B-shaped Q6_K token loop, bs=1)",
                   "timed_steps": f"{args.steps} decode tokens from position {t_start}, in runs of at "
                                  f"most {CTX - t_start}, each after restoring the prompt state and "
                                  f"{args.warmup} untimed steps from it",
                   "layers": 24, "conv_layers": 18, "attention_layers": 6, "vocab": hp.vocab,
                   "experts": "32 top-4", "ctx": CTX, "parallelism": "single GPU"},
        "roofline": roof, "cpu_baseline": cpu,
        "decode_hbm_gbs": round(decode_gbs, 1),
        "decode_bytes_per_token": int(wbytes + kvbytes),
        "decode_256": decode_256,
        "prefill": None if args.synthetic_state else {
            "tokens": n_prompt, "ms": round(prefill_s * 1e3, 1),
            "tok_s": round(n_prompt / prefill_s, 1),
            "algorithmic_tflops": round(pf_flops / prefill_s / 1e12, 1),
            "mfma_peak_tflops": MFMA_F16_PEAK_TFLOPS,
            "mfma_frac": round(pf_flops / prefill_s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "note": "algorithmic FLOPs (projections, router, causal attention, last-token head); "
                    "each GEMM product runs as two binary16 matrix-core passes (hi, lo)"},
        "prefill_chunked": chunked,
        "prefill_full_int8_scales": full_scale,
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
