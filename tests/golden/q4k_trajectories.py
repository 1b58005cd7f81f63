"""Exact-fraction trajectories of make_qkx1_quants(nmax = 15, ntry = 5) for the two
multi-iteration sub-blocks of tests/test_oracle_q4k_from_float.py (FIVE and STOP).

Run: python tests/golden/q4k_trajectories.py.  It prints, per iteration, the quants,
whether any changed, scale and min as exact fractions, and the smallest distance of
any rounded product from a tie; then the end point with four iterations and without
the early stop.  The algorithm is the one stated in that test module's docstring,
carried out in exact rational arithmetic (no float rounding), which the f32 oracle
matches to within 1e-7 relative on these inputs (every rounding decision is at least
0.011 from a tie).  It reads nothing but its own constants.
"""
from fractions import Fraction as F

FIVE = [-28, 48, -7, 172, 148, -31, 94, 138, -31, -7, 58, 41, 102, -11, -31, 14, 14, 41, 138, 18, 48, 14, 18, 58,
        41, 41, 66, 41, 29, 14, 58, 14]
STOP = [-39, 92, 35, -39, 123, 35, 87, 92, -39, 123, 123, 19, 87, 123, 92, 92, 87, 92, 35, 92, 123, 35, 92, 92, -39,
        92, 19, 19, 92, 35, 35, -39]


def round_half_away(v: F) -> int:
    r = (abs(v) + F(1, 2)).__floor__()
    return r if v >= 0 else -r


def trajectory(x, ntry=5, early_stop=True):
    n = len(x)
    if max(x) == min(x):
        return F(0), F(0), []
    mn = min(min(x), F(0))
    iscale = F(15) / (max(x) - mn)
    q = [0] * n
    rows = []
    scale = 1 / iscale
    for it in range(ntry):
        changed, margin = False, F(1)
        for i, v in enumerate(x):
            t = iscale * (v - mn)
            margin = min(margin, abs(abs(t) - abs(t).__floor__() - F(1, 2)))
            li = max(0, min(15, round_half_away(t)))
            if li != q[i]:
                q[i], changed = li, True
        scale = sum((v - mn) * li for v, li in zip(x, q)) / sum(li * li for li in q)
        mn = min(sum(v - scale * li for v, li in zip(x, q)) / n, F(0))
        iscale = 1 / scale
        rows.append((it + 1, changed, list(q), scale, mn, margin))
        if early_stop and not changed:
            break
    return scale, -mn, rows


if __name__ == "__main__":
    for name, vals in (("FIVE", FIVE), ("STOP", STOP)):
        x = [F(v, 16) for v in vals]
        s, m, rows = trajectory(x)
        print(name)
        for it, changed, q, sc, mn, margin in rows:
            print(f"  iteration {it}: changed={changed} quants={q}")
            print(f"    scale={sc} ({float(sc):.8f}) min={mn} ({float(mn):.8f}) closest tie {float(margin):.4f}")
        s4, m4, _ = trajectory(x, ntry=4)
        sn, mnn, _ = trajectory(x, early_stop=False)
        print(f"  end point {float(s):.8f} {float(m):.8f}; four iterations {float(s4):.8f} {float(m4):.8f}; "
              f"no early stop {float(sn):.8f} {float(mnn):.8f}")
