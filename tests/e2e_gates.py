"""End-to-end comparison of two PP-DocLayoutV3 results (dets + masks).

Restates the reference's parity gates (bench/run_ggml.py:37-87 for labels,
scores, boxes, masks and the matched-set check; bench/oracle_all.py:107-124
for relative reading order with tie groups), at this project's tolerances:
every detection scoring >= 0.3 in the expected result must be present in the
other one with the same label, score within 3e-5, box within 0.01 px, and the
confident detections must keep their relative reading order.
"""
import numpy as np

CONF_T = 0.30  # gate tier
POOL_T = 0.28  # matching pool reaches below the gate (threshold straddlers)
MATCH_PX = 0.25  # box-match radius for the set check
SCORE_TOL = 3e-5
BOX_TOL_PX = 0.01
MASK_IOU_MIN = 0.95


def _match(od, gd):
    """Pairs (r, j): each confident expected row r to the same-class row j of
    the other result with the nearest box."""
    pairs = []
    used = np.zeros(len(gd), bool)
    for r in np.where(od[:, 1] >= CONF_T)[0]:
        cand = np.where(~used & (gd[:, 0].astype(int) == int(od[r, 0])))[0]
        if len(cand) == 0:
            pairs.append((int(r), -1))
            continue
        d = np.abs(gd[cand, 2:6] - od[r, 2:6]).max(axis=1)
        j = int(cand[np.argmin(d)])
        used[j] = True
        pairs.append((int(r), j))
    return pairs


def _set_miss(a, b):
    used = np.zeros(len(b), bool)
    miss = 0
    for r in a:
        cand = np.where(~used & (b[:, 0].astype(int) == int(r[0])))[0]
        if len(cand) == 0:
            miss += 1
            continue
        d = np.abs(b[cand, 2:6] - r[2:6]).max(axis=1)
        if d.min() > MATCH_PX:
            miss += 1
        else:
            used[cand[np.argmin(d)]] = True
    return miss


def relative_order_ok(od, gd, pairs):
    """Sorted by the expected rank, the other ranks must strictly increase
    across tie groups (one query selected under several classes shares a
    rank) and be constant within each group."""
    seq = sorted(pairs, key=lambda p: int(od[p[0], 6]))
    k = 0
    while k < len(seq):
        k2 = k
        while k2 < len(seq) and int(od[seq[k2][0], 6]) == int(od[seq[k][0], 6]):
            k2 += 1
        gs = {int(gd[j, 6]) for _, j in seq[k:k2]}
        if len(gs) != 1:
            return False
        k = k2
        if k < len(seq) and gs.pop() >= int(gd[seq[k][1], 6]):
            return False
    return True


def compare(od, om, gd, gm):
    """od/gd: (300, 7) dets; om/gm: (300, 200, 200) or (300, 40000) masks.
    Returns the gate metrics."""
    pairs = _match(od, gd)
    missing = sum(1 for _, j in pairs if j < 0)
    good = [(r, j) for r, j in pairs if j >= 0]
    om = np.asarray(om).reshape(len(od), -1) != 0
    gm = np.asarray(gm).reshape(len(gd), -1) != 0

    def iou(r, j):
        inter = int((om[r] & gm[j]).sum())
        union = int((om[r] | gm[j]).sum())
        return inter / union if union else 1.0

    return {
        "n_conf": len(pairs),
        "missing_conf": missing,
        "score_maxdiff_conf": max((abs(float(od[r, 1] - gd[j, 1])) for r, j in good), default=0.0),
        "box_maxdiff_px": max((float(np.abs(od[r, 2:6] - gd[j, 2:6]).max()) for r, j in good), default=0.0),
        "mask_iou_min": min((iou(r, j) for r, j in good), default=1.0),
        "order_rel_ok": relative_order_ok(od, gd, good) if not missing else False,
        "set_sym_diff": _set_miss(od[od[:, 1] >= POOL_T], gd) + _set_miss(gd[gd[:, 1] >= POOL_T], od),
    }


def passes(m):
    return (m["missing_conf"] == 0 and m["score_maxdiff_conf"] <= SCORE_TOL and m["box_maxdiff_px"] <= BOX_TOL_PX
            and m["order_rel_ok"] and m["mask_iou_min"] >= MASK_IOU_MIN and m["set_sym_diff"] == 0)
