"""Host side of the reference's Winograd / Toom-Cook 1-D conv op family (python/lokinfer/ops/winograd.py in
lariaus/lokinfer): the exact transform tables and the host weight transform `wino_weights`, which a caller runs
once per conv weight and passes to wino_mm_lc_f32_gpu as operands (U, tr). The tables have to equal the
reference's for the kernels to be a drop-in, so the construction follows the same mathematics:

  correlation F(m, r) with alpha = m + r - 1 points p_0..p_{alpha-2} and infinity:
  y = AT ((G g) * (BT d)) with  G = V_r (Vandermonde rows [p^0 .. p^{r-1}] plus the point at infinity),
  AT = V_m^T,  BT = C^T where C = V_alpha^{-1} (inverted exactly over the rationals),
  and each BT row scaled to max |.| = 1 with G's row scaled up by the same factor.

K = 3 uses F(4, 3) (6 points) or F(2, 3) (4 points, tile = 2); K = 4..12 a nested F(4, 4) (7 points) over
ceil(K / 4) tap groups at offsets 0, 4, 8 that share one transformed input.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np

TILE = 4
MAX_GROUPS = 3
ROWS_TG = 128  # output rows per statistics chunk / GEMM workgroup
POINTS = {3: [0, 1, -1, 2, -2], 4: [0, 1, -1, 2, -2, Fraction(-1, 2)]}
POINTS_TILE2 = [0, 1, -1]


def _vandermonde(points, n):
    """Rows [p^0, ..., p^{n-1}] for each finite point, then the point at infinity (leading coefficient only)."""
    rows = [[Fraction(p) ** j for j in range(n)] for p in points]
    rows.append([Fraction(0)] * (n - 1) + [Fraction(1)])
    return rows


def _inverse(mat):
    """Exact inverse over Fractions (Gauss-Jordan with row pivoting)."""
    n = len(mat)
    aug = [list(row) + [Fraction(int(i == j)) for j in range(n)] for i, row in enumerate(mat)]
    for col in range(n):
        piv = next(r for r in range(col, n) if aug[r][col] != 0)
        aug[col], aug[piv] = aug[piv], aug[col]
        scale = aug[col][col]
        aug[col] = [v / scale for v in aug[col]]
        for r in range(n):
            if r != col and aug[r][col] != 0:
                f = aug[r][col]
                aug[r] = [v - f * w for v, w in zip(aug[r], aug[col])]
    return [row[n:] for row in aug]


def transforms_exact(m: int, r: int, points=None):
    """(AT [m x alpha], G [alpha x r], BT [alpha x alpha]) as Fractions."""
    pts = POINTS[r] if points is None else points
    alpha = m + r - 1
    if len(pts) != alpha - 1:
        raise ValueError(f"F({m},{r}) needs {alpha - 1} finite points")
    va, vb = _vandermonde(pts, m), _vandermonde(pts, r)
    c = _inverse(_vandermonde(pts, alpha))
    bt = [[c[j][i] for j in range(alpha)] for i in range(alpha)]
    g = [list(row) for row in vb]
    at = [[va[j][i] for j in range(alpha)] for i in range(m)]
    for i in range(alpha):
        s = max(abs(v) for v in bt[i])
        bt[i] = [v / s for v in bt[i]]
        g[i] = [v * s for v in g[i]]
    return at, g, bt


def transforms(m: int, r: int, points=None):
    """Float64 (AT, G, BT) of transforms_exact."""
    f = lambda mat: np.array([[float(v) for v in row] for row in mat], dtype=np.float64)  # noqa: E731
    return tuple(f(x) for x in transforms_exact(m, r, points))


def variant(k: int) -> tuple[int, int]:
    """(inner r, tap groups n) for kernel size k: (3, 1) at K = 3, else (4, max(2, ceil(K / 4))) for K <= 12."""
    if k == 3:
        return 3, 1
    if not 4 <= k <= TILE * MAX_GROUPS:
        raise ValueError(f"winograd conv: kernel size {k} unsupported (3..12)")
    return TILE, max(2, -(-k // TILE))


def alpha_of(kernel: int, tile: int = TILE) -> int:
    return 4 if tile == 2 else 6 if kernel == 3 else 7


def wino_weights(w: np.ndarray, tile: int = TILE) -> tuple[np.ndarray, np.ndarray]:
    """torch conv weight f32[Co, Ci, K] -> (U f32[A, n * Ci, Co], tr f32[A * A + m * A] = [BT | AT]), in float64.
    tile = 2 (K = 3 only) selects F(2, 3)."""
    w = np.asarray(w, dtype=np.float64)
    co, ci, k = w.shape
    r, n = variant(k)
    if tile not in (TILE, 2) or (tile == 2 and k != 3):
        raise ValueError("tile 2 is only for K = 3")
    at, g, bt = transforms(tile, r, POINTS_TILE2 if tile == 2 else None)
    alpha = tile + r - 1
    wg = np.zeros((n, r, ci, co))
    for t in range(k):
        wg[t // TILE, t % TILE] = w[:, :, t].T
    u = np.einsum("xk,gkio->xgio", g, wg).reshape(alpha, n * ci, co)
    tr = np.concatenate([bt.reshape(-1), at.reshape(-1)])
    return np.ascontiguousarray(u, dtype=np.float32), tr.astype(np.float32)


def tiles_rows(lo: int, dilation: int, groups: int, tile: int, kernel: int) -> int:
    """Rows of V: d * A * rmax, rmax = ceil(ceil(Lo / d) / 128) * (128 / tile) + groups - 1."""
    rmax = -(-(-(-lo // dilation)) // ROWS_TG) * (ROWS_TG // tile) + (groups - 1)
    return rmax * dilation * alpha_of(kernel, tile)


def stats_chunks(lo: int, dilation: int) -> int:
    """Statistics chunks per residue class: ceil(ceil(Lo / d) / 128)."""
    return -(-(-(-lo // dilation)) // ROWS_TG)
