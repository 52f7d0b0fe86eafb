"""Command-line drivers without a GPU: lfm2-greedy's argument grammar and checks
(engine/src/main.rs:28-113 and its tests at main.rs:283-346), api_stream's request
validation (engine/src/bin/api_stream.rs:12-27, --validate-only needs no device)
and the JSON number and string layout the drivers print."""
import json
import os
import subprocess

import pytest

import lfm_hip as L
from conftest import PKG, REPO
from model_util import small_hparams

GREEDY = os.path.join(PKG, "lfm2-greedy")
API = os.path.join(PKG, "api_stream")


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("cli") / "tiny.gguf")
    L.write_synthetic_gguf(p, small_hparams(vocab=300), L.synth_opts(seed=5), threads=4)
    return p


def run(exe, args, stdin=None, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([exe] + args, input=stdin, capture_output=True, text=True, env=e,
                          timeout=120)


@pytest.mark.parametrize("args,msg", [
    (["--model"], "--model needs a value"),
    (["--model", "m", "--tokens", "1", "--text", "hi"], "choose exactly one of"),
    (["--model", "m", "--text", "hi", "--cpu"], "--cpu is only an explicit --tokens diagnostic"),
    (["--model", "m", "--tokens", "1", "--n", "-1"], "invalid digit found in string"),
    (["--model", "m"], "need --tokens, --text or --chat-json"),
    (["--tokens", "1"], "need --model"),
    (["--model", "m", "--tokens", "1", "--bogus"], "unknown arg --bogus"),
    (["--model", "m", "--tokens", "1", "--eos", "4294967296"], "too large"),
    (["--model", "m", "--text", "hi"], "need the reference's tokenizer"),
    (["--model", "m", "--tokens", "1", "--stream"], "stream decoder"),
    (["--model", "m", "--tokens", "1", "--cpu"], "CPU diagnostic"),
])
def test_greedy_argument_errors(args, msg):
    r = run(GREEDY, args)
    assert r.returncode == 1 and r.stdout == ""
    assert r.stderr.startswith("Error: ") and msg in r.stderr, r.stderr


def test_greedy_token_checks(model):
    env = {"LFM_ANY_GEOMETRY": "1"}
    r = run(GREEDY, ["--model", model, "--tokens", "1,-1"], env=env)
    assert r.returncode == 1 and 'bad token id "-1"' in r.stderr
    r = run(GREEDY, ["--model", model, "--tokens", " , ,"], env=env)
    assert "prompt token list must not be empty" in r.stderr
    r = run(GREEDY, ["--model", model, "--tokens", "1,300"], env=env)
    assert "prompt contains an out-of-range token ID" in r.stderr
    r = run(GREEDY, ["--model", model, "--tokens", "1, +2 ,299", "--n", "5000"], env=env)
    assert "exceeds 4096" in r.stderr
    # without LFM_ANY_GEOMETRY the reference's fixed geometry is required
    r = run(GREEDY, ["--model", model, "--tokens", "1,2"])
    assert "unsupported geometry" in r.stderr
    # a valid request passes every check and reaches the device
    if L.device_count() == 0:
        r = run(GREEDY, ["--model", model, "--tokens", "1, 2", "--n", "0"], env=env)
        assert r.returncode == 1 and "no HIP device" in r.stderr, r.stderr
    r = run(GREEDY, ["--model", os.path.join(REPO, "nope.gguf"), "--tokens", "1"])
    assert "open model file" in r.stderr


def events(r):
    return [json.loads(x) for x in r.stdout.splitlines()]


def test_api_stream_validation(model):
    reqs = [
        '{"id":"a","tokens":[1,2],"n":4}',
        '{"id":"","tokens":[1],"n":1}',
        '{"id":"' + "x" * 129 + '","tokens":[1],"n":1}',
        '{"id":"b","tokens":[1],"n":0}',
        '{"id":"b","tokens":[1],"n":1025}',
        '{"id":"b","tokens":[1],"text":"hi","n":1}',
        '{"id":"b","n":1}',
        '{"id":"b","text":"hi","n":1}',
        '{"id":"b","tokens":[],"n":1}',
        '{"id":"b","tokens":[' + ",".join(["1"] * 4000) + '],"n":97}',
        '{"id":"b","tokens":[300],"n":1}',
        '{"id":"b","tokens":[1],"n":1,"extra":0}',
        '{"id":"b","tokens":[1]}',
        '{"id":"b","id":"c","tokens":[1],"n":1}',
        '{"id":"b","tokens":[-1],"n":1}',
        '{"id":"b","tokens":[1.0],"n":1}',
        '{"id":"b","tokens":[1],"n":1} x',
        'not json',
        '{"id":"\\ud83d\\ude00 \\"q\\"\\u0001","chat":null,"tokens":[299],"n":1024}',
    ]
    r = run(API, ["--validate-only", model], stdin="\n".join(reqs) + "\n")
    assert r.returncode == 0, r.stderr
    ev = events(r)
    assert len(ev) == len(reqs)
    assert r.stdout.splitlines()[0] == '{"type":"validated","id":"a","prompt_tokens":[1,2]}'
    msgs = [e.get("message") for e in ev]
    assert [e["type"] for e in ev] == ["validated"] + ["validation_error"] * 17 + ["validated"]
    want = ["invalid id", "invalid id", "max_tokens must be 1..1024", "max_tokens must be 1..1024",
            "exactly one input required", "exactly one input required", "tokenizer",
            "empty or context exceeds 4096", "empty or context exceeds 4096",
            "out-of-range token", "unknown field `extra`", "missing field `n`",
            "duplicate field `id`", "expected u32", "expected u32", "trailing characters",
            "expected value"]
    for m, w in zip(msgs[1:-1], want):
        assert w in m, (m, w)
    # surrogate pair decoded, then printed as raw UTF-8 with \" and \u0001 escaped
    assert ev[-1]["id"] == "\U0001F600 \"q\"\x01"
    assert '"id":"\U0001F600 \\"q\\"\\u0001"' in r.stdout.splitlines()[-1]
    r = run(API, ["--model"])
    assert r.returncode == 1 and "usage: api_stream --model|--validate-only MODEL" in r.stderr


def test_json_number_layout(tmp_path):
    """f64 printed as serde_json (ryu) prints it: shortest round-trip digits,
    plain decimal for exponents -5 < kk <= 16, else d.ddde<exp>."""
    cases = [(1.0, "1.0"), (0.1, "0.1"), (-2.5, "-2.5"), (1234.5678, "1234.5678"),
             (100.0, "100.0"), (1e15, "1000000000000000.0"), (1e16, "1e16"),
             (1.2345678901234568e17, "1.2345678901234568e17"), (1e-5, "0.00001"),
             (1.5e-5, "0.000015"), (1e-6, "1e-6"), (1.25e-7, "1.25e-7"), (5e-324, "5e-324"),
             (1.7976931348623157e308, "1.7976931348623157e308"),
             (0.30000000000000004, "0.30000000000000004"), (0.0, "0.0"), (-0.0, "-0.0"),
             (float("nan"), "null"), (float("inf"), "null"), (12345678.9, "12345678.9")]
    src = tmp_path / "num.cpp"
    vals = ",".join(repr(v) if v == v and abs(v) != float("inf") else
                    ("NAN" if v != v else "INFINITY") for v, _ in cases)
    src.write_text('#include "json.h"\n#include <cmath>\nint main(){double v[]={' + vals +
                   '};for(double x: v) printf("%s\\n", lfmjson::num(x).c_str());'
                   'printf("%s\\n", lfmjson::str(std::string("a\\"\\\\\\b\\f\\n\\r\\t\\x01\\x1f\\x7f") +'
                   ' "\\xc3\\xa9").c_str());}\n')
    exe = tmp_path / "num"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(PKG, "cli"), str(src), "-o",
                    str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    lines = out.splitlines()
    assert lines[:-1] == [w for _, w in cases]
    assert lines[-1] == '"a\\"\\\\\\b\\f\\n\\r\\t\\u0001\\u001f\x7fé"'
