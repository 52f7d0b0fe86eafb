"""The routing audit helper (tests/route_audit.py) on hand-made decisions."""
import numpy as np

from route_audit import Audit, margin, select_margin, sigmoid_scores, top_ids


def test_top_ids_ties_and_order():
    # equal scores keep the lower id first (lfm.rs:623-626 stable sort)
    s = np.array([0.5, 0.9, 0.5, 0.9, 0.1], dtype=np.float32)
    assert top_ids(s, 4) == [1, 3, 0, 2]
    assert top_ids(-s, 2) == [4, 0]
    assert select_margin(s, 1) == 0.0 and select_margin(s, 3) == 0.0
    assert abs(select_margin(s, 2) - 0.4) < 1e-7 and abs(select_margin(s, 4) - 0.4) < 1e-7
    # the decision margin also sees the tie inside the picks
    assert margin(s, 2) == 0.0 and margin(s, 4) == 0.0
    t = np.array([0.9, 0.7, 0.6, 0.1], dtype=np.float32)
    assert abs(margin(t, 2) - 0.1) < 1e-7 and abs(select_margin(t, 2) - 0.1) < 1e-7
    assert abs(margin(t, 1) - 0.2) < 1e-7


def test_sigmoid_scores_match_float64():
    lg = np.linspace(-8, 8, 33).astype(np.float32)
    b = np.linspace(-0.1, 0.1, 33).astype(np.float32)
    ref = 1.0 / (1.0 + np.exp(-lg.astype(np.float64))) + b
    assert np.abs(sigmoid_scores(lg, b) - ref).max() < 3e-7


def test_audit_runs_and_drift():
    a = Audit(2)
    base = np.array([0.9, 0.8, 0.7, 0.1], dtype=np.float32)
    # clean decisions with a small score difference
    for p in range(12):
        for l in (2, 3, 4, 5):
            a.add(p, l, [0, 1], base + 1e-6, [0, 1], base)
    # position 4, layer 3: a flip at a near-tie (reference margin 1e-6)
    tie = np.array([0.9, 0.8, 0.8 - 1e-6, 0.1], dtype=np.float32)
    a.add(4, 3, [0, 2], tie, [0, 1], tie)
    # reached from it (one position on, one layer up), with a large drift
    a.add(5, 4, [2, 3], base, [0, 1], base + 0.5)
    # a flip the first cannot reach (layer 2 is below it): another run
    a.add(5, 2, [1, 0], base, [0, 1], base)
    assert a.flips() == [(4, 3), (5, 2), (5, 4)]
    assert a.first_flips() == [(4, 3), (5, 2)]
    assert a.kind((4, 3)) == "set" and a.kind((5, 2)) == "order"
    # (4, 3) reaches position 4 above layer 3 and, at layer l, 2 (l - 3) positions on
    assert a.carried((4, 4)) and not a.carried((4, 2)) and not a.carried((4, 3))
    assert a.carried((6, 4)) and a.carried((8, 5)) and not a.carried((10, 4))
    # (5, 2) reaches (7, 3) and (9, 4); nothing reaches (8, 3)
    assert a.carried((7, 3)) and a.carried((9, 4)) and not a.carried((8, 3))
    # the flips' and reached decisions' drifts are not clean drift
    assert abs(a.clean_drift() - 1e-6) < 1e-7
    ids, ref_ids, d, m = a.rows[(4, 3)]
    assert m < 2e-6
