#!/usr/bin/env python3
"""Benchmark: batch-1 greedy decode of the synthetic LFM2.5-8B-A1B-shaped Q6_K
model at 4096 context on one MI355X, plus the Q6_K matvec HBM roofline and the
CPU restatement of the reference path timed on the host.

Workload (one step = one decode token): 24 layers (18 gated short-conv, 6 GQA at
layers 2,6,10,14,18,21), dense SwiGLU ff 7168 in layers 0-1, MoE 32 experts top-4
ff 1792 in layers 2-23, vocab 65536 tied Q6_K head; seeded random weights;
prompt of (4096 - steps) uniform ids prefilled, then `steps` greedy tokens at
positions 3840..4095.  Warmup steps run first and the resident state is then
restored to the end of the prompt, so the timed steps are exactly the workload.

Prints one JSON line: metric, value (tok/s), ms_per_step, roofline of the dominant
kernel, the CPU baseline and prefill figures.
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
# counters read for a plain 512 MiB copy): 1.02 x the algorithmic 24 155 264 bytes.
GATEUP_TRAFFIC_BYTES = 24584196
SEED = 0x9E3779B97F4A7C15


def log(msg):
    print(msg, file=sys.stderr, flush=True)


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


def matvec_roofline(iters=200):
    """cfg0 kernel: 6144x2048 Q6_K matvec, 64 rotating weight copies (660 MB >
    the 256 MB Infinity Cache), HIP-event timing on the launch stream."""
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


def cpu_baseline(hp, snapshot, start_pos, gpu_tokens, first, budget_s=15.0, max_steps=128):
    """The oracle (C restatement of the reference CPU path) on the host cores:
    resident state restored from the GPU at the end of the prompt, then greedy
    decode steps teacher-forced with the GPU's tokens until ~budget_s."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import lfm_oracle

    threads = min(16, len(os.sched_getaffinity(0)))
    lfm_oracle.set_threads(threads)
    o = lfm_oracle.OracleEngine(hp, ctx=4096, kv_f16=True)
    for d in lfm_hip.model_tensor_descs(hp):
        o.set_tensor(d.name.decode(), int(d.ggml_type), d.shape, lfm_hip.synth_tensor(d, threads=threads))
    o.finalize()
    o.restore(start_pos, snapshot)
    feed, steps, agree, compared = first, 0, 0, 0
    t0 = time.perf_counter()
    while steps < max_steps and time.perf_counter() - t0 < budget_s:
        lo = o.forward([feed], start_pos + steps)
        srt = np.sort(lo)
        if srt[-1] - srt[-2] > 1e-3 * np.abs(lo).max():
            compared += 1
            agree += int(lfm_oracle.argmax(lo) == gpu_tokens[steps])
        feed = gpu_tokens[steps]
        steps += 1
    dt = time.perf_counter() - t0
    o.close()
    return {"value": steps / dt, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{steps} greedy decode steps of the full model at positions "
                      f"{start_pos}..{start_pos + steps - 1} (ctx 4096), oracle state restored "
                      f"from the GPU after prefill; {dt:.1f} s",
            "tokens_compared": compared, "tokens_agree": agree}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--synthetic-state", action="store_true",
                    help="skip the prefill: restore a seeded binary16 KV / conv state for the "
                         "prompt positions instead (isolates decode kernels for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the batch-1 decode path runs on a single GPU and is "
              "not sharded here; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    assert lfm_hip.device_count() > 0, "no HIP device"
    if args.steps < 1 or args.steps + 1 > args.ctx:
        sys.exit("steps must be in 1..ctx-1")

    hp = lfm_hip.make_hparams()
    t = time.perf_counter()
    eng = lfm_hip.GpuEngine.load_synthetic(hp, lfm_hip.synth_opts(SEED), ctx=args.ctx, threads=16)
    log(f"[bench] model generated + uploaded in {time.perf_counter() - t:.1f} s on {eng.device_name}")
    n_prompt = args.ctx - args.steps
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

    if args.warmup > 0:
        eng.decode_run(first, n_prompt, min(args.warmup, args.steps), eos=1 << 31)
        eng.restore_session(n_prompt, snap)
    lfm_hip.lib().lfm_dev_synchronize()
    t0 = time.perf_counter()
    toks = eng.decode_run(first, n_prompt, args.steps, eos=1 << 31)
    lfm_hip.lib().lfm_dev_synchronize()
    dt = time.perf_counter() - t0
    assert len(toks) == args.steps
    ms_per_step = dt * 1e3 / args.steps
    tok_s = args.steps / dt
    wbytes, kvbytes = decode_bytes_per_token(hp, range(n_prompt, n_prompt + args.steps))
    decode_gbs = (wbytes + kvbytes) * tok_s / 1e9
    log(f"[bench] decode {args.steps} steps: {ms_per_step:.3f} ms/step, {tok_s:.1f} tok/s, "
        f"{decode_gbs:.0f} GB/s algorithmic")

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
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": GATEUP_TRAFFIC_BYTES,
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
        extra["q6k_matvec_cfg0"] = {
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
        log(f"[bench] q6k matvec cfg0: {ms_hbm * 1e3:.2f} us/launch = "
            f"{extra['q6k_matvec_cfg0']['hbm_gbs']:.0f} GB/s (HBM, 64 rotating copies), "
            f"{extra['q6k_matvec_cfg0']['cache_resident_gbs']:.0f} GB/s cache-resident")

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (oracle) ...")
        cpu = cpu_baseline(hp, snap, n_prompt, toks, first)
        log(f"[bench] cpu baseline {cpu['value']:.3f} tok/s on {cpu['cores']} threads")

    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded random-init Q6_K weights and prompt ids)",
        "config": {"workload": f"LFM2.5-8B-A1B-shaped Q6_K token loop, bs=1: prefill {n_prompt} "
                               f"+ {args.steps} greedy decode steps at ctx {args.ctx}",
                   "layers": 24, "conv_layers": 18, "attention_layers": 6, "vocab": hp.vocab,
                   "experts": "32 top-4", "ctx": args.ctx, "parallelism": "single GPU"},
        "roofline": roof, "cpu_baseline": cpu,
        "decode_hbm_gbs": round(decode_gbs, 1),
        "decode_bytes_per_token": int(wbytes + kvbytes),
        "prefill": None if args.synthetic_state else {
            "tokens": n_prompt, "ms": round(prefill_s * 1e3, 1),
            "tok_s": round(n_prompt / prefill_s, 1),
            "algorithmic_tflops": round(pf_flops / prefill_s / 1e12, 1),
            "mfma_peak_tflops": MFMA_F16_PEAK_TFLOPS,
            "mfma_frac": round(pf_flops / prefill_s / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "note": "algorithmic FLOPs (projections, router, causal attention, last-token head); "
                    "each GEMM product runs as two binary16 matrix-core passes (hi, lo)"},
        "prefill_chunked": chunked,
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
