"""Seeded synthetic models shared by the oracle and GPU parity tests."""
import numpy as np

import lfm_hip


def small_hparams(dim=256, heads=4, kinds=("conv", "attn"), kv=2, vocab=300, n_expert=8,
                  n_used=4, expert_ff=256, n_ff=512, dense_lead=1, eos=None):
    """A model with the reference's structure at small sizes (kinds per layer)."""
    attn = tuple(i for i, k in enumerate(kinds) if k == "attn")
    hp = lfm_hip.make_hparams(dim=dim, heads=heads, n_layers=len(kinds), attention_layers=attn,
                              kv=kv, vocab=vocab, eps=1e-5, rope_theta=1e6,
                              eos=vocab + 1 if eos is None else eos, n_expert=n_expert,
                              n_used=n_used, expert_ff=expert_ff, n_ff=n_ff, dense_lead=dense_lead)
    return hp


def model_tensors(hp, opts=None, threads=8):
    """[(name, ggml_type, shape, data)] for every tensor of the model."""
    out = []
    for d in lfm_hip.model_tensor_descs(hp, opts):
        data = lfm_hip.synth_tensor(d, opts, threads)
        out.append((d.name.decode(), int(d.ggml_type), d.shape, data))
    return out


def oracle_engine(oracle_mod, hp, tensors, ctx=4096):
    e = oracle_mod.OracleEngine(hp, ctx=ctx, kv_f16=True)
    for name, t, shape, data in tensors:
        e.set_tensor(name, t, shape, data)
    e.finalize()
    return e


def gpu_engine(hp, tensors, ctx=4096):
    return lfm_hip.GpuEngine.load(hp, tensors, ctx=ctx)


def top2_margin(logits):
    s = np.sort(logits[np.isfinite(logits)])
    return float(s[-1] - s[-2])
