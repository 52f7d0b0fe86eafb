"""The command-line drivers on the GPU, against the oracle and against the same
engine driven in-process.

lfm2-greedy (engine/src/main.rs:157-280, --tokens form): the result object's keys
and tokens, the BENCH_TIMING line, and LFM_FORWARD_OUT_DIR's per-step logits.
api_stream (engine/src/bin/api_stream.rs:33-85): ready / accepted / delta / result
events, a prompt longer than one 64-token prefill chunk, a second request on a
fresh session, and a validation error in between.  The in-process replica makes
the same engine calls, so tokens must be identical.  Every token the drivers
print is also checked against the oracle (fed from the seeded generator, not the
file), teacher-forced with the drivers' own tokens: equal wherever the oracle's
top-2 margin exceeds 1e-3 * max|logit|."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import PKG
from model_util import model_tensors, oracle_engine, top2_margin

pytestmark = pytest.mark.gpu
OPTS_SEED = 11

GREEDY = os.path.join(PKG, "lfm2-greedy")
API = os.path.join(PKG, "api_stream")
ENV = dict(os.environ, LFM_ANY_GEOMETRY="1")


def cli_hparams(L):
    return L.make_hparams(dim=512, heads=8, n_layers=3, attention_layers=(1,), kv=2, vocab=1000,
                          eos=1 << 30, n_expert=8, n_used=4, expert_ff=512, n_ff=1024,
                          dense_lead=1)


@pytest.fixture(scope="module")
def model(gpu, tmp_path_factory):
    L = gpu
    p = str(tmp_path_factory.mktemp("cli") / "cli.gguf")
    L.write_synthetic_gguf(p, cli_hparams(L), L.synth_opts(seed=OPTS_SEED, bias_sigma=0.1),
                           threads=16)
    return p


@pytest.fixture(scope="module")
def cli_oracle(gpu, oracle):
    hp = cli_hparams(gpu)
    o = oracle_engine(oracle, hp, model_tensors(hp, gpu.synth_opts(seed=OPTS_SEED, bias_sigma=0.1)),
                      ctx=4096)
    yield o
    o.close()


def oracle_check(oracle, o, prompt, tokens):
    """The greedy tokens a driver printed for `prompt` (tokens[0] from the prompt's
    last logits) against the oracle, teacher-forced; returns how many were
    margin-clear (all of those must be equal)."""
    o.reset()
    lo = o.forward(prompt, 0)
    compared = 0
    for s, t in enumerate(tokens):
        if top2_margin(lo) > 1e-3 * float(np.abs(lo).max()):
            assert t == oracle.argmax(lo), (s, t, oracle.argmax(lo))
            compared += 1
        if s + 1 < len(tokens):
            lo = o.forward([t], len(prompt) + s)
    return compared


def test_lfm2_greedy_tokens(gpu, oracle, cli_oracle, model, tmp_path):
    L = gpu
    prompt, n = [5, 999, 0, 17, 256, 3], 12
    print("lfm2-greedy", prompt, n, flush=True)
    r = subprocess.run([GREEDY, "--model", model, "--tokens", ",".join(map(str, prompt)),
                        "--n", str(n)], capture_output=True, text=True, env=ENV, timeout=120)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    assert list(out) == ["prompt_tokens", "tokens", "decoded_text", "greedy", "device",
                         "gpu_dispatch_count", "eos", "n_vocab"]
    assert out["prompt_tokens"] == prompt and out["decoded_text"] is None
    assert out["greedy"] is True and out["n_vocab"] == 1000 and out["eos"] == 1 << 30
    assert "gfx950" in out["device"] and out["gpu_dispatch_count"] > 0
    timing = [x for x in r.stderr.splitlines() if x.startswith("BENCH_TIMING ")]
    assert len(timing) == 1
    t = json.loads(timing[0][len("BENCH_TIMING "):])
    assert list(t) == ["load_ms", "tokenize_ms", "warmup_ms", "prompt_ms", "gen_ms",
                       "n_prompt_tokens", "n_gen_tokens"]
    assert t["n_prompt_tokens"] == len(prompt) and t["n_gen_tokens"] == n

    e = L.GpuEngine.from_gguf(model, ctx=len(prompt) + n + 16, strict=False)
    logits = e.forward(prompt, 0)
    first = int(np.argmax(logits))
    want = [first] + e.decode_run(first, len(prompt), n - 1)
    e.close()
    assert out["tokens"] == want
    compared = oracle_check(oracle, cli_oracle, prompt, out["tokens"])
    print(f"lfm2-greedy: {compared}/{n} margin-clear tokens equal to the oracle's")
    assert compared >= n // 2

    # host loop with every step's logits kept (main.rs:155-165, 192-219)
    keep = tmp_path / "steps"
    keep.mkdir()
    r2 = subprocess.run([GREEDY, "--model", model, "--tokens", ",".join(map(str, prompt)),
                         "--n", "4"], capture_output=True, text=True, timeout=120,
                        env=dict(ENV, LFM_FORWARD_OUT_DIR=str(keep)))
    assert r2.returncode == 0, r2.stderr
    assert json.loads(r2.stdout)["tokens"] == want[:4]
    files = sorted(os.listdir(keep))
    assert files == [f"forward-{i}.logits.bin" for i in range(5)]
    l0 = np.fromfile(keep / "forward-0.logits.bin", dtype=np.float32)
    assert np.array_equal(l0, logits)


def test_api_stream_session(gpu, oracle, cli_oracle, model):
    L = gpu
    long_prompt = [int(x) for x in np.random.default_rng(2).integers(0, 1000, 100)]
    reqs = [{"id": "r1", "tokens": long_prompt, "n": 6},
            {"id": "bad", "tokens": [1000], "n": 1},
            {"id": "r2", "tokens": [7, 8, 9], "n": 4}]
    print("api_stream", [(q["id"], len(q["tokens"]), q["n"]) for q in reqs], flush=True)
    r = subprocess.run([API, "--model", model], input="".join(json.dumps(q) + "\n" for q in reqs),
                       capture_output=True, text=True, env=ENV, timeout=180)
    assert r.returncode == 0, r.stderr
    ev = [json.loads(x) for x in r.stdout.splitlines()]
    assert list(ev[0]) == ["type", "model_load_count", "pid", "load_ms", "vram_before",
                           "weight_bytes"]
    with L.GgufFile.open(model) as f:
        weights = sum(int(t.nbytes) for t in f.tensors)
    assert ev[0]["type"] == "ready" and ev[0]["weight_bytes"] == weights
    types = [x["type"] for x in ev]
    assert types == (["ready", "accepted"] + ["delta"] * 6 + ["result", "validation_error",
                                                            "accepted"] + ["delta"] * 4 +
                     ["result"])
    res = [x for x in ev if x["type"] == "result"]
    assert list(res[0]) == ["type", "id", "prompt_tokens", "tokens", "text", "finish_reason",
                            "request_count", "model_load_count", "pid", "prefill_ms",
                            "request_ms", "gpu_dispatches"]
    assert [x["request_count"] for x in res] == [1, 2]
    assert all(x["finish_reason"] == "length" and x["text"] is None for x in res)
    deltas = [x for x in ev if x["type"] == "delta"]
    assert list(deltas[0]) == ["type", "id", "text", "token"]

    # in-process replica: fresh session, 64-token prefill chunks, one token at a time
    e = L.GpuEngine.from_gguf(model, ctx=4096, strict=False)
    for q, got in zip([reqs[0], reqs[2]], res):
        e.reset_session()
        pos, nxt = 0, 0
        for c in range(0, len(q["tokens"]), 64):
            chunk = q["tokens"][c:c + 64]
            nxt = e.forward_token(chunk, pos)
            pos += len(chunk)
        toks = []
        for _ in range(q["n"]):
            toks.append(nxt)
            nxt = e.forward_token([nxt], pos)
            pos += 1
        assert got["tokens"] == toks, (q["id"], got["tokens"], toks)
        assert [d["token"] for d in deltas if d["id"] == q["id"]] == toks
        compared = oracle_check(oracle, cli_oracle, q["tokens"], got["tokens"])
        print(f"api_stream {q['id']}: {compared}/{q['n']} margin-clear tokens equal to the oracle's")
        assert compared >= q["n"] // 2
    e.close()
