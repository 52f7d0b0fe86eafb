"""Pins the oracle's model arithmetic (engine/src/lfm.rs:205-694) at small sizes.

* A float64 numpy restatement of the LFM2 forward (RMSNorm, per-head norm, NEOX
  RoPE, f16-rounded KV, causal GQA softmax attention, gated short conv with its
  2-slot state, dense SwiGLU, sigmoid+bias top-k MoE, tied head) must agree with
  the oracle's f32 logits to float32 accuracy.  A dropped term, a transposed
  weight, a wrong RoPE pair or a wrong conv tap order each move the logits by
  orders of magnitude more than the tolerance.
* One n-token forward equals n one-token forwards bit for bit (every operation
  is per token in the reference), and snapshot/restore round-trips exactly.
"""
import numpy as np
import pytest

from model_util import model_tensors, oracle_engine, small_hparams


def np_model(hp, tensors):
    W = {}
    for name, t, shape, data in tensors:
        if t == 14:
            from test_oracle_q6k import np_dequant
            rows = int(np.prod(shape[1:]))
            W[name] = np_dequant(data).reshape(rows, shape[0]).astype(np.float64)
        else:
            W[name] = data.astype(np.float64).reshape(tuple(reversed(shape)))
    return W


def np_rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def np_forward(hp, W, ids, state):
    dim, hd = hp.dim, 64
    eps = float(np.float32(hp.eps))
    logits = None
    for j, tok in enumerate(ids):
        pos = state["pos"]
        x = W["token_embd.weight"][tok].copy()
        for l in range(hp.n_layers):
            p = f"blk.{l}."
            h = np_rms(x, W[p + "attn_norm.weight"], eps)
            kv = hp.kv_heads[l]
            if kv:
                q = (W[p + "attn_q.weight"] @ h).reshape(hp.heads, hd)
                k = (W[p + "attn_k.weight"] @ h).reshape(kv, hd)
                v = (W[p + "attn_v.weight"] @ h).reshape(kv, hd)
                q = q / np.sqrt(np.mean(q * q, axis=1, keepdims=True) + eps) * W[p + "attn_q_norm.weight"]
                k = k / np.sqrt(np.mean(k * k, axis=1, keepdims=True) + eps) * W[p + "attn_k_norm.weight"]
                theta = pos * float(np.float32(hp.rope_theta)) ** (-2.0 * np.arange(hd // 2) / hd)
                c, s = np.cos(theta), np.sin(theta)

                def rope(a):
                    a0, a1 = a[:, : hd // 2].copy(), a[:, hd // 2:].copy()
                    return np.concatenate([a0 * c - a1 * s, a0 * s + a1 * c], axis=1)

                q, k = rope(q), rope(k)
                K = state.setdefault(("K", l), [])
                V = state.setdefault(("V", l), [])
                K.append(k.astype(np.float32).astype(np.float16).astype(np.float64))
                V.append(v.astype(np.float32).astype(np.float16).astype(np.float64))
                Ks, Vs = np.stack(K), np.stack(V)  # [t][kv][hd]
                a = np.zeros((hp.heads, hd))
                for hh in range(hp.heads):
                    kh = hh * kv // hp.heads
                    sc = Ks[:, kh, :] @ q[hh] / np.sqrt(hd)
                    w = np.exp(sc - sc.max())
                    a[hh] = (w / w.sum()) @ Vs[:, kh, :]
                x = x + W[p + "attn_output.weight"] @ a.reshape(-1)
            else:
                bcx = W[p + "shortconv.in_proj.weight"] @ h
                B, Cc, X = bcx[:dim], bcx[dim:2 * dim], bcx[2 * dim:]
                st = state.setdefault(("conv", l), np.zeros((dim, 2)))
                cw = W[p + "shortconv.conv.weight"]  # [dim][3]
                bx = B * X
                co = st[:, 0] * cw[:, 0] + st[:, 1] * cw[:, 1] + bx * cw[:, 2]
                state[("conv", l)] = np.stack([st[:, 1], bx], axis=1)
                x = x + W[p + "shortconv.out_proj.weight"] @ (Cc * co)
            f = np_rms(x, W[p + "ffn_norm.weight"], eps)
            if l < hp.dense_lead:
                g = W[p + "ffn_gate.weight"] @ f
                u = W[p + "ffn_up.weight"] @ f
                x = x + W[p + "ffn_down.weight"] @ (g / (1 + np.exp(-g)) * u)
            else:
                lg = W[p + "ffn_gate_inp.weight"] @ f
                pr = 1 / (1 + np.exp(-lg))
                score = pr + W[p + "exp_probs_b.bias"]
                sel = sorted(range(hp.n_expert), key=lambda e: (-score[e], e))[: hp.n_used]
                wsel = pr[sel] / max(pr[sel].sum(), 6.103515625e-5)
                eff = hp.expert_ff
                Wg = W[p + "ffn_gate_exps.weight"].reshape(hp.n_expert, eff, dim)
                Wu = W[p + "ffn_up_exps.weight"].reshape(hp.n_expert, eff, dim)
                Wd = W[p + "ffn_down_exps.weight"].reshape(hp.n_expert, dim, eff)
                acc = np.zeros(dim)
                for r, e in enumerate(sel):
                    g, u = Wg[e] @ f, Wu[e] @ f
                    acc += (Wd[e] @ (g / (1 + np.exp(-g)) * u)) * wsel[r]
                x = x + acc
        state["pos"] = pos + 1
        xn = np_rms(x, W["token_embd_norm.weight"], eps)
        logits = W["token_embd.weight"] @ xn
    return logits


@pytest.fixture(scope="module")
def small_model():
    hp = small_hparams(kinds=("conv", "attn", "conv", "attn"), dense_lead=1)
    tensors = model_tensors(hp)
    return hp, tensors


def test_oracle_forward_matches_float64_restatement(oracle, small_model):
    hp, tensors = small_model
    W = np_model(hp, tensors)
    e = oracle_engine(oracle, hp, tensors, ctx=64)
    ids = [5, 17, 299, 0, 42, 42, 7]
    got = e.forward(ids, 0)
    exp = np_forward(hp, W, ids, {"pos": 0})
    rel = np.linalg.norm(got - exp) / np.linalg.norm(exp)
    assert rel < 2e-4, rel
    nxt = int(np.argmax(exp))
    got2 = e.forward([nxt], len(ids))
    exp2 = np_forward(hp, W, ids + [nxt], {"pos": 0})
    assert np.linalg.norm(got2 - exp2) / np.linalg.norm(exp2) < 2e-4


def test_oracle_prefix_consistency_bit_exact(oracle, small_model):
    hp, tensors = small_model
    ids = [3, 1, 4, 1, 5, 9, 2, 6]
    a = oracle_engine(oracle, hp, tensors, ctx=32)
    full = a.forward(ids, 0)
    b = oracle_engine(oracle, hp, tensors, ctx=32)
    for j, t in enumerate(ids):
        step = b.forward([t], j)
    assert np.array_equal(full.view(np.uint32), step.view(np.uint32))
    assert a.snapshot(len(ids)) == b.snapshot(len(ids))


def test_oracle_snapshot_restore_roundtrip(oracle, small_model):
    hp, tensors = small_model
    a = oracle_engine(oracle, hp, tensors, ctx=32)
    a.forward([9, 8, 7, 6], 0)
    snap = a.snapshot(4)
    assert len(snap) == a.state_bytes(4)
    b = oracle_engine(oracle, hp, tensors, ctx=32)
    b.restore(4, snap)
    assert b.snapshot(4) == snap
    assert np.array_equal(a.forward([1], 4), b.forward([1], 4))


def test_oracle_thread_count_does_not_change_results(oracle, small_model):
    hp, tensors = small_model
    res = []
    for th in (1, 4):
        oracle.set_threads(th)
        e = oracle_engine(oracle, hp, tensors, ctx=16)
        res.append(e.forward([11, 12, 13], 0))
    oracle.set_threads(8)
    assert np.array_equal(res[0].view(np.uint32), res[1].view(np.uint32))


def test_oracle_rejects_out_of_range(oracle, small_model):
    hp, tensors = small_model
    e = oracle_engine(oracle, hp, tensors, ctx=4)
    with pytest.raises(ValueError):
        e.forward([hp.vocab], 0)
    with pytest.raises(ValueError):
        e.forward([1, 2, 3, 4, 5], 0)
