"""Decision-by-decision comparison of MoE expert selections.

The reference routes every token at every MoE layer by the scores
s_e = sigmoid(logit_e) + bias_e, top n_used by a stable descending sort, so
equal scores keep the lower expert id first (engine/src/lfm.rs:613-637).  Two
implementations whose scores differ by at most D in every expert can only pick
different experts where the 4th and 5th scores of either lie within 2 D of each
other: if one picks i over j and the other j over i, then
    s'_j - s'_i <= (s'_j - s_j) + (s_i - s'_i) <= 2 D.
The same holds for the rank order of the picks (the combine adds the experts
in rank order): if the ordered picks first differ at rank k, the reference's
gap between its k-th and (k+1)-th scores is at most 2 D.  The tests below
therefore measure D (the score drift) at every decision and require every
selection that differs to sit at such a near-tie.
"""
import numpy as np


def _rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def sigmoid_scores(logits, bias):
    """Scores p + bias in float32 (p = 1 / (1 + exp(-logit)), lfm.rs:616-618)."""
    lg = np.asarray(logits, dtype=np.float32)
    p = (np.float32(1.0) / (np.float32(1.0) + np.exp(-lg))).astype(np.float32)
    return (p + np.asarray(bias, dtype=np.float32)).astype(np.float32)


def top_ids(scores, n_used):
    """Rank order of the picks: descending score, ties to the lower id."""
    s = np.asarray(scores, dtype=np.float32)
    order = sorted(range(s.size), key=lambda e: (-float(s[e]), e))
    return order[:n_used]


def margin(scores, n_used):
    """Smallest gap between consecutive scores over the picks and the best
    excluded one: the distance from a decision with other picks or another
    rank order."""
    s = np.sort(np.asarray(scores, dtype=np.float64))[::-1]
    return float(np.min(s[:n_used] - s[1:n_used + 1]))


def select_margin(scores, n_used):
    """Gap between the last pick's score and the best excluded one."""
    s = np.sort(np.asarray(scores, dtype=np.float64))[::-1]
    return float(s[n_used - 1] - s[n_used])


class Audit:
    """Decisions (position, layer) of one implementation against a reference.

    add() records one decision; a decision is a flip when the ordered picks
    differ (another expert set, or the same set in another rank order).  A flip
    at (q, l') can change the input of the decision at (p, l) when p == q and
    l > l', or when p > q and p - q <= 2 (l - l'): the flip changes the residual
    of position q after layer l', and each short-convolution layer after it
    carries a changed residual two positions on.  A flip no other flip can
    reach starts a run; decisions that are neither flips nor reachable from one
    are clean, and their score differences measure the drift."""

    def __init__(self, n_used):
        self.n_used = n_used
        self.rows = {}  # (pos, layer) -> (ids, ref_ids, drift, ref_margin)

    def add(self, pos, layer, ids, scores, ref_ids, ref_scores):
        ids, ref_ids = [int(i) for i in ids], [int(i) for i in ref_ids]
        d = float(np.max(np.abs(np.asarray(scores, np.float64) - np.asarray(ref_scores, np.float64))))
        self.rows[(int(pos), int(layer))] = (ids, ref_ids, d, margin(ref_scores, self.n_used))

    def flips(self):
        return sorted(k for k, r in self.rows.items() if r[0] != r[1])

    @staticmethod
    def reaches(flip, key):
        (q, lq), (p, l) = flip, key
        return (p == q and l > lq) or (p > q and p - q <= 2 * (l - lq))

    def first_flips(self):
        f = self.flips()
        return [k for k in f if not any(self.reaches(q, k) for q in f if q != k)]

    def carried(self, key, flips=None):
        """Whether a flip can have changed the decision's input."""
        fl = self.flips() if flips is None else flips
        return any(self.reaches(q, key) for q in fl if q != key)

    def kind(self, key):
        ids, ref_ids = self.rows[key][:2]
        return "order" if sorted(ids) == sorted(ref_ids) else "set"

    def clean_drift(self):
        """Largest score difference over the clean decisions (0 when none)."""
        fl = self.flips()
        ds = [r[2] for k, r in self.rows.items() if r[0] == r[1] and not self.carried(k, fl)]
        return max(ds) if ds else 0.0

    def pre_flip_drift(self):
        """Largest score difference before the first flip (positions before it,
        and its own position's lower layers): arithmetic alone, with no flip
        behind it.  Later clean decisions also see a flip's position through
        attention, which reads every earlier position's K/V."""
        fl = self.flips()
        if not fl:
            return self.clean_drift()
        p0, l0 = min(fl)
        ds = [r[2] for (p, l), r in self.rows.items() if p < p0 or (p == p0 and l < l0)]
        return max(ds) if ds else 0.0

    def summary(self):
        fl = self.flips()
        return (f"{len(self.rows)} decisions, {len(fl)} flips ({len(self.first_flips())} run starts), "
                f"clean drift {self.clean_drift():.2e} ({self.pre_flip_drift():.2e} before the first "
                f"flip), smallest reference margin "
                f"{min(r[3] for r in self.rows.values()):.2e}")


def split_state(hp, snap, valid):
    """Per layer: K|V rows [valid, kv*64*2] (attention) or the conv state [dim*2]."""
    f = np.frombuffer(snap, np.float32)
    out, off = [], 0
    for l in range(hp.n_layers):
        kv = hp.kv_heads[l]
        if kv:
            n = valid * 64 * kv
            out.append(np.concatenate([f[off:off + n].reshape(valid, -1),
                                       f[off + n:off + 2 * n].reshape(valid, -1)], axis=1))
            off += 2 * n
        else:
            out.append(f[off:off + 2 * hp.dim])
            off += 2 * hp.dim
    assert off == f.size
    return out


def reach(l, flip):
    """Positions of layer l's mixer input that a flip at (q, l') can change: q
    and, through the convolution layers between, 2 (l - l') - 1 more."""
    q, lq = flip
    return range(q, q + 2 * (l - lq)) if l > lq else range(0)


def state_errors(hp, a, b, valid, flips):
    """rel-L2 per layer over the positions no flip reaches (attention K/V rows),
    and of the conv states (the last two positions) no flip reaches."""
    out, dropped = {}, 0
    for l, (x, y) in enumerate(zip(split_state(hp, a, valid), split_state(hp, b, valid))):
        keep = np.ones(valid, dtype=bool)
        for f in flips:
            r = reach(l, f)
            keep[r.start:min(r.stop, valid)] = False
        if hp.kv_heads[l]:
            out[l] = _rel_l2(x[keep], y[keep])
            dropped = max(dropped, int((~keep).sum()))
        elif keep[valid - 2:].all():
            out[l] = _rel_l2(x, y)
    return out, dropped
