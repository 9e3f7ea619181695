"""Host side of the Winograd conv family (lokinfer_amd/winograd.py), no GPU: the transform tables are exact
Toom-Cook correlations (checked over the rationals, as the reference's test_winograd_gpu.py:29-37 does in float64
at 1e-12), and the weight transform U plus the table tr, replayed in float64 with the kernels' tile / tap-group
indexing, equal torch's conv1d for every kernel size the family accepts."""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from lokinfer_amd import winograd as W

rng = np.random.default_rng(7)


@pytest.mark.parametrize("m,r,pts", [(4, 3, None), (4, 4, None), (2, 3, W.POINTS_TILE2)])
def test_transforms_exact_over_rationals(m, r, pts):
    at, g, bt = W.transforms_exact(m, r, pts)
    alpha = m + r - 1
    assert len(at) == m and len(g) == alpha and len(bt) == alpha
    for trial in range(5):
        d = [Fraction(int(v), 7) for v in rng.integers(-50, 50, alpha)]
        w = [Fraction(int(v), 3) for v in rng.integers(-50, 50, r)]
        gw = [sum(g[i][k] * w[k] for k in range(r)) for i in range(alpha)]
        bd = [sum(bt[i][j] * d[j] for j in range(alpha)) for i in range(alpha)]
        y = [sum(at[o][i] * gw[i] * bd[i] for i in range(alpha)) for o in range(m)]
        assert y == [sum(w[k] * d[o + k] for k in range(r)) for o in range(m)]
    for row in bt:  # each BT row scaled to max |.| = 1
        assert max(abs(v) for v in row) == 1


def test_points_and_variants():
    assert W.POINTS[3] == [0, 1, -1, 2, -2] and W.POINTS[4][-1] == Fraction(-1, 2)
    assert W.variant(3) == (3, 1) and W.variant(4) == (4, 2) and W.variant(8) == (4, 2) and W.variant(11) == (4, 3)
    assert [W.alpha_of(k) for k in (3, 7, 11)] == [6, 7, 7] and W.alpha_of(3, 2) == 4
    for k in (1, 2, 13):
        with pytest.raises(ValueError):
            W.variant(k)
    with pytest.raises(ValueError):
        W.wino_weights(np.zeros((64, 16, 7), np.float32), tile=2)


def _replay(x, u, tr, k, tile, pad, d):
    """float64 replay of the kernels' algorithm: V[rho, xi, r, c] = sum_j BT[xi, j] h[rho + d (r M + j) - pad],
    out[rho + d (t M + j)] = sum_xi AT[j, xi] sum_{g, ci} V[rho, xi, t + g, ci] U[xi, g Ci + ci]."""
    l, ci = x.shape
    alpha, nci, co = u.shape
    n = nci // ci
    bt = tr[:alpha * alpha].reshape(alpha, alpha).astype(np.float64)
    at = tr[alpha * alpha:].reshape(tile, alpha).astype(np.float64)
    lo = l + 2 * pad - d * (k - 1)
    out = np.zeros((lo, co))
    for rho in range(d):
        rows = len(range(rho, lo, d))
        tiles = -(-rows // tile)
        v = np.zeros((alpha, tiles + n - 1, ci))
        for r in range(tiles + n - 1):
            for j in range(alpha):
                p = rho + d * (r * tile + j) - pad
                if 0 <= p < l:
                    v[:, r] += bt[:, j, None] * x[p]
        uu = u.astype(np.float64).reshape(alpha, n, ci, co)
        for t in range(tiles):
            m = np.einsum("xgc,xgco->xo", v[:, t:t + n], uu)
            y = at @ m
            for j in range(tile):
                o = rho + d * (t * tile + j)
                if o < lo:
                    out[o] = y[j]
    return out


@pytest.mark.parametrize("k,tile,d,l", [(3, 4, 1, 23), (3, 2, 2, 17), (4, 4, 1, 9), (5, 4, 2, 31), (7, 4, 3, 40),
                                        (11, 4, 5, 61), (12, 4, 1, 13)])
def test_weights_replay_equals_conv1d(k, tile, d, l):
    ci, co = 16, 8
    x = rng.standard_normal((l, ci))
    w = rng.standard_normal((co, ci, k)) / math.sqrt(ci * k)
    pad = d * (k // 2) if k % 2 == 0 else d * (k - 1) // 2
    u, tr = W.wino_weights(w, tile=tile)
    assert u.shape == (W.alpha_of(k, tile), W.variant(k)[1] * ci, co)
    ref = F.conv1d(torch.from_numpy(x).T[None], torch.from_numpy(w), padding=pad, dilation=d)[0].T.numpy()
    np.testing.assert_allclose(_replay(x, u, tr, k, tile, pad, d), ref, atol=2e-5, rtol=0)


def test_row_counts():
    # rmax = ceil(ceil(Lo / d) / 128) * (128 / M) + groups - 1 rows per (residue class, point)
    assert W.tiles_rows(1000, 5, 3, 4, 11) == (2 * 32 + 2) * 5 * 7
    assert W.tiles_rows(300, 1, 1, 4, 3) == (3 * 32) * 6
    assert W.tiles_rows(300, 1, 1, 2, 3) == (3 * 64) * 4
    assert W.stats_chunks(1001, 5) == 2 and W.stats_chunks(128, 1) == 1 and W.stats_chunks(129, 1) == 2


def test_tables_equal_the_committed_values():
    """The exact tables equal tests/golden/winograd_tables.json, the values every Winograd GPU parity case and
    every U / tr operand was built with (F(4, 3), F(4, 4), F(2, 3))."""
    import json
    from pathlib import Path

    gold = json.loads((Path(__file__).resolve().parent / "golden" / "winograd_tables.json").read_text())
    for name, (m, r, pts) in {"F(4,3)": (4, 3, None), "F(4,4)": (4, 4, None), "F(2,3)": (2, 3, W.POINTS_TILE2)}.items():
        got = dict(zip(("AT", "G", "BT"), W.transforms_exact(m, r, pts)))
        for key, mat in gold[name].items():
            assert [[Fraction(v) for v in row] for row in mat] == got[key], (name, key)


def test_wino_weights_sums_in_tap_order():
    """U entries are the tap-order float64 sums of G x w rounded once to f32 (the same bits wherever U is built)."""
    w = rng.standard_normal((8, 16, 7)).astype(np.float32)
    u, _ = W.wino_weights(w)
    r, n = W.variant(7)
    g = W.transforms(4, r)[1]
    for x in range(u.shape[0]):
        for grp in range(n):
            for i in (0, 5, 15):
                for o in (0, 7):
                    acc = 0.0
                    for t in range(r):
                        k = grp * 4 + t
                        acc = acc + g[x, t] * (float(w[o, i, k]) if k < 7 else 0.0)
                    assert u[x, grp * 16 + i, o] == np.float32(acc)
