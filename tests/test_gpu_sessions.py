"""Multi-session switching through snapshot and restore, as the reference's
persistent server does it (engine/src/bin/persistent.rs:140-220): one engine,
sessions keyed by id, the active session's resident cache snapshotted when
another session takes the engine and restored when it comes back, prompts
prefilled in 64-token forward_token calls, greedy tokens one forward_token
call each with the next token kept per session.

Interleaved requests over three sessions must give every request the tokens
that the same session's requests give when it has the engine to itself, and
every session must end with the same resident cache, byte for byte.
"""
import numpy as np
import pytest

from model_util import gpu_engine, model_tensors

pytestmark = pytest.mark.gpu

CONTEXT, GENERATION, MAX_SESSIONS, CHUNK = 4096, 1024, 8, 64


class Sessions:
    """The session rules of persistent.rs:139-220 over a GpuEngine."""

    def __init__(self, engine, vocab, eos):
        self.g, self.vocab, self.eos = engine, vocab, eos
        self.sessions = {}  # id -> [prefix, cache, next]
        self.active = None

    def request(self, sid, action, tokens=(), n=0):
        assert 0 < len(sid) <= 128, "invalid session ID"
        assert action in ("fresh", "continue", "reset", "interleave"), "invalid action"
        assert n <= GENERATION, "generation exceeds 1024"
        suffix = [int(t) for t in tokens]
        assert all(t < self.vocab for t in suffix), "out-of-range token"
        new = action in ("fresh", "reset") or (action == "interleave" and sid not in self.sessions)
        assert action != "fresh" or sid not in self.sessions, "fresh session already exists"
        assert new or sid in self.sessions, "unknown continuation session"
        old_len = 0 if new else len(self.sessions[sid][0])
        assert 0 < old_len + len(suffix) and old_len + len(suffix) + n <= CONTEXT, \
            "context exceeds 4096 or empty prompt"
        assert sid in self.sessions or len(self.sessions) < MAX_SESSIONS, "at most eight sessions"
        if self.active != sid:
            if self.active is not None:
                s = self.sessions[self.active]
                s[1] = self.g.snapshot_resident_cache(len(s[0]))
            if not new:
                s = self.sessions[sid]
                self.g.restore_session(len(s[0]), s[1])
        if new:
            self.g.reset_session()
            self.sessions[sid] = [[], b"", 0]
        self.active = sid
        s = self.sessions[sid]
        for i in range(0, len(suffix), CHUNK):
            chunk = suffix[i:i + CHUNK]
            s[2] = self.g.forward_token(chunk, len(s[0]))
            s[0].extend(chunk)
        out = []
        for _ in range(n):
            tok = s[2]
            if tok == self.eos:
                break
            out.append(tok)
            s[2] = self.g.forward_token([tok], len(s[0]))
            s[0].append(tok)
        return out

    def final_cache(self, sid):
        s = self.sessions[sid]
        if self.active == sid:
            return self.g.snapshot_resident_cache(len(s[0]))
        return s[1]


def test_interleaved_sessions_match_uninterrupted(gpu):
    hp = gpu.make_hparams(dim=2048, heads=32, n_layers=4, attention_layers=(1, 3), kv=8,
                          vocab=4096, eos=1 << 30, n_expert=32, n_used=4, expert_ff=1792,
                          n_ff=7168, dense_lead=1)
    rng = np.random.default_rng(41)
    ids = lambda k: [int(t) for t in rng.integers(0, hp.vocab, k)]
    script = [  # (session, action, prompt tokens, n)
        ("a", "fresh", ids(150), 8),
        ("b", "fresh", ids(70), 5),
        ("a", "continue", ids(40), 6),
        ("c", "interleave", ids(10), 4),
        ("b", "continue", [], 7),
        ("a", "interleave", ids(64), 3),
        ("c", "continue", ids(129), 2),
        ("b", "reset", ids(30), 4),
        ("a", "continue", ids(1), 5),
    ]
    g = gpu_engine(hp, model_tensors(hp), ctx=CONTEXT)
    mixed = Sessions(g, hp.vocab, hp.eos)
    got = [mixed.request(sid, act, toks, n) for sid, act, toks, n in script]
    caches = {sid: mixed.final_cache(sid) for sid in "abc"}
    lengths = {sid: len(mixed.sessions[sid][0]) for sid in "abc"}
    with pytest.raises(AssertionError, match="fresh session already exists"):
        mixed.request("a", "fresh", ids(4), 1)
    with pytest.raises(AssertionError, match="unknown continuation session"):
        mixed.request("d", "continue", ids(4), 1)

    for sid in "abc":
        alone = Sessions(g, hp.vocab, hp.eos)  # the engine for this session only
        want = [alone.request(s, act, toks, n) for s, act, toks, n in script if s == sid]
        have = [t for (s, _, _, _), t in zip(script, got) if s == sid]
        print(f"session {sid}: {lengths[sid]} tokens, requests {have}")
        assert have == want, sid
        assert alone.final_cache(sid) == caches[sid], sid
    g.close()
