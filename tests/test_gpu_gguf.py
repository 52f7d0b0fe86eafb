"""An engine loaded from a GGUF file (C++ reader -> lfm_engine_upload_tensor, the
reference's ModelFile + GpuEngine::load staging loop, engine/src/gpu_lfm.rs:51-97,
engine/src/model_file.rs:100-109) against the oracle, and exactly what an engine
loaded with the same bytes directly computes.

The oracle takes the tensors from the seeded generator, not from the file, so the
whole chain file -> reader -> upload -> kernels is checked against an independent
source: prompt logits rel-L2 <= 1e-3 and greedy tokens equal wherever the oracle's
top-2 margin exceeds 1e-3 * max|logit| (teacher-forced with the GPU's tokens).

Model: real widths (dim 2048, 32 heads / 8 kv heads, 32 experts top-4, ff 1792,
dense ff 7168), one dense conv layer and one MoE attention layer, vocab 4096,
router bias ~ N(0, 0.1).  The kernels reduce in a fixed order, so the logits and
the greedy tokens must be identical, not merely close."""
import numpy as np
import pytest

from conftest import rel_l2
from model_util import model_tensors, oracle_engine, top2_margin

pytestmark = pytest.mark.gpu

SEED = 0x5EED_6600


def test_gguf_loaded_engine_matches_direct_load(gpu, oracle, tmp_path):
    L = gpu
    hp = L.make_hparams(dim=2048, heads=32, n_layers=2, attention_layers=(1,), kv=8, vocab=4096,
                        eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792, n_ff=7168,
                        dense_lead=1)
    opts = L.synth_opts(SEED, bias_sigma=0.1)
    path = str(tmp_path / "lfm2_small.gguf")
    L.write_synthetic_gguf(path, hp, opts, threads=16)
    print(f"wrote {path}", flush=True)

    direct = L.GpuEngine.load_synthetic(hp, opts, ctx=64)
    from_file = L.GpuEngine.from_gguf(path, ctx=64, strict=False)
    assert bytes(from_file.hp) == bytes(hp)

    prompt = [3, 4095, 17, 0, 2048, 999, 5]
    la, lb = direct.forward(prompt, 0), from_file.forward(prompt, 0)
    assert np.array_equal(la, lb)
    first = int(np.argmax(la))
    ta = direct.decode_run(first, len(prompt), 8)
    tb = from_file.decode_run(first, len(prompt), 8)
    assert ta == tb
    direct.close()
    from_file.close()

    # the file-loaded engine against the oracle fed from the generator
    tensors = model_tensors(hp, opts)
    with L.GgufFile.open(path) as f:
        for name, _, _, data in tensors:  # the file holds the generator's bytes
            assert f.read_tensor(name).tobytes() == data.tobytes(), name
    o = oracle_engine(oracle, hp, tensors, ctx=64)
    lo = o.forward(prompt, 0)
    err = rel_l2(lb, lo)
    tol = 1e-3 * float(np.abs(lo).max())
    assert err <= 1e-3, err
    if top2_margin(lo) > tol:
        assert first == oracle.argmax(lo)
    feed, compared = first, 0
    for s, t in enumerate(tb):
        lo = o.forward([feed], len(prompt) + s)
        if top2_margin(lo) > 1e-3 * float(np.abs(lo).max()):
            assert t == oracle.argmax(lo), (s, t, oracle.argmax(lo))
            compared += 1
        feed = t
    print(f"GGUF-loaded engine vs oracle: prompt logits rel-L2 {err:.2e}, "
          f"{compared}/{len(tb)} margin-clear tokens equal")
    assert compared >= len(tb) // 2
    o.close()

    # the two-step form: open, create with the file's hparams, upload, finalize
    with L.GgufFile.open(path) as f:
        e = L.GpuEngine(f.hparams(strict=False), ctx=64)
        e.load_gguf(f)
    e.finalize()
    assert np.array_equal(e.forward(prompt, 0), la)
    e.close()

    # the reference's loader accepts only the LFM2.5-8B-A1B geometry
    with pytest.raises(L.LfmError, match="unsupported geometry"):
        L.GpuEngine.from_gguf(path, ctx=64, strict=True)
