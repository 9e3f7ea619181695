"""Host side of the Winograd / Toom-Cook 1-D conv op family (the reference's wino_* ops, python/lokinfer/ops/
winograd.py in lariaus/lokinfer): the transform tables and the weight transform a caller runs once per conv weight,
whose results (U, tr) are operands of wino_mm_lc_f32_gpu. U and tr are passed between callers and kernels, so their
values are the reference's; they are derived here from polynomial interpolation.

Toom-Cook correlation F(m, r): y_o = sum_k g_k d_{o+k} for m outputs o and r taps, through alpha = m + r - 1
products y = AT ((G g) * (BT d)). Take alpha - 1 finite points p_i and the point at infinity:
  G   row i = the tap polynomial g(x) = sum_k g_k x^k evaluated at p_i (row [p_i^0 .. p_i^(r-1)]); at infinity its
      leading coefficient (row [0 .. 0, 1]);
  AT  column i = the output polynomial evaluated at p_i (entries p_i^0 .. p_i^(m-1)); at infinity [0 .. 0, 1];
  BT  row i = the coefficients of the interpolation basis polynomial of point i: the Lagrange basis polynomial
      l_i(x) = prod_{j != i} (x - p_j) / (p_i - p_j) of the finite points (degree alpha - 2, so its x^(alpha-1)
      coefficient is 0), and for infinity the node polynomial prod_j (x - p_j) (monic, degree alpha - 1).
Every coefficient is an exact rational; each BT row is then scaled to max |.| = 1 and the matching G row by the
inverse factor (the product (G g)_i (BT d)_i is unchanged).

Variants: K = 3 uses F(4, 3) on 0, +-1, +-2 (6 points) or, with tile = 2, F(2, 3) on 0, +-1 (4 points); K = 4..12
uses F(4, 4) on 0, +-1, +-2, -1/2 (7 points) over ceil(K / 4) >= 2 groups of four taps at offsets 0, 4, 8 that
share one transformed input tile.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np

TILE = 4
MAX_GROUPS = 3
ROWS_TG = 128  # output rows per statistics chunk / GEMM workgroup
POINTS = {3: [0, 1, -1, 2, -2], 4: [0, 1, -1, 2, -2, Fraction(-1, 2)]}
POINTS_TILE2 = [0, 1, -1]


def _times_linear(poly: list, root) -> list:
    """Coefficients (lowest first) of poly(x) * (x - root)."""
    out = [Fraction(0)] * (len(poly) + 1)
    for k, c in enumerate(poly):
        out[k + 1] += c
        out[k] -= c * root
    return out


def _node_poly(points) -> list:
    """prod_j (x - p_j), lowest coefficient first."""
    poly = [Fraction(1)]
    for p in points:
        poly = _times_linear(poly, Fraction(p))
    return poly


def _lagrange(points, i: int) -> list:
    """Coefficients of the Lagrange basis polynomial of points[i] over `points`."""
    pi = Fraction(points[i])
    poly, denom = [Fraction(1)], Fraction(1)
    for j, p in enumerate(points):
        if j != i:
            poly = _times_linear(poly, Fraction(p))
            denom *= pi - Fraction(p)
    return [c / denom for c in poly]


def _powers(p, n: int) -> list:
    return [Fraction(p) ** e for e in range(n)]


def transforms_exact(m: int, r: int, points=None):
    """(AT [m][alpha], G [alpha][r], BT [alpha][alpha]) as Fractions."""
    pts = POINTS[r] if points is None else points
    alpha = m + r - 1
    if len(pts) != alpha - 1:
        raise ValueError(f"F({m},{r}) needs {alpha - 1} finite points")
    at_cols = [_powers(p, m) for p in pts] + [[Fraction(0)] * (m - 1) + [Fraction(1)]]
    at = [[at_cols[i][o] for i in range(alpha)] for o in range(m)]
    g = [_powers(p, r) for p in pts] + [[Fraction(0)] * (r - 1) + [Fraction(1)]]
    bt = [_lagrange(pts, i) + [Fraction(0)] for i in range(alpha - 1)] + [_node_poly(pts)]
    for i, row in enumerate(bt):
        big = max(abs(c) for c in row)
        bt[i] = [c / big for c in row]
        g[i] = [c * big for c in g[i]]
    return at, g, bt


def transforms(m: int, r: int, points=None):
    """(AT, G, BT) of transforms_exact as float64 arrays."""
    return tuple(np.array(mat, dtype=np.float64) for mat in transforms_exact(m, r, points))


def variant(k: int) -> tuple[int, int]:
    """(taps per group r, tap groups n) of kernel size k: (3, 1) for K = 3, else (4, max(2, ceil(K / 4))) up to 12."""
    if k == 3:
        return 3, 1
    if k < 4 or k > TILE * MAX_GROUPS:
        raise ValueError(f"winograd conv: kernel size {k} unsupported (3..12)")
    return TILE, max(2, (k + TILE - 1) // TILE)


def alpha_of(kernel: int, tile: int = TILE) -> int:
    """Transform points of a kernel size and output tile."""
    return 4 if tile == 2 else 6 if kernel == 3 else 7


def wino_weights(w: np.ndarray, tile: int = TILE) -> tuple[np.ndarray, np.ndarray]:
    """torch conv weight f32[Co, Ci, K] -> (U f32[A, n Ci, Co], tr f32[A A + m A] = BT then AT, row-major).
    U[x, g Ci + i, o] = sum_k G[x, k] w[o, i, 4 g + k] (taps past K are zero), the products summed in tap order in
    float64 and rounded once to f32, so U is the same bits wherever it is built. tile = 2 (K = 3 only) selects
    F(2, 3)."""
    w = np.asarray(w, dtype=np.float64)
    co, ci, k = w.shape
    r, n = variant(k)
    if tile not in (TILE, 2) or (tile == 2 and k != 3):
        raise ValueError("tile 2 is only for K = 3")
    at, g, bt = transforms(tile, r, POINTS_TILE2 if tile == 2 else None)
    alpha = tile + r - 1
    taps = np.zeros((co, ci, n * r))
    taps[:, :, :k] = w
    grouped = taps.reshape(co, ci, n, r)  # [o, i, group, tap in group]
    u = np.zeros((alpha, co, ci, n))
    for t in range(r):
        u = u + g[:, t, None, None, None] * grouped[None, :, :, :, t]
    u = u.transpose(0, 3, 2, 1).reshape(alpha, n * ci, co)  # [x, group * Ci + i, o]
    tr = np.concatenate([bt.ravel(), at.ravel()])
    return np.ascontiguousarray(u, dtype=np.float32), tr.astype(np.float32)


def tile_u(u: np.ndarray, groups: int) -> np.ndarray:
    """U f32[A, n Ci, Co] -> the wino_mm ops' tiled form (u_layout = 1) f32[A, Co / 64, n Ci 64]:
    ut[x, cb, (((c n + g) 4 + k4) 64 + j) 4 + q] = U[x, g Ci + 16 c + 4 k4 + q, 64 cb + j] (Ci % 16 == 0,
    Co % 64 == 0): per point, 64-column block, 16-channel chunk and tap group, a k-quad-major 16 x 64 slab."""
    a, nci, co = u.shape
    ci = nci // groups
    t = u.reshape(a, groups, ci // 16, 4, 4, co // 64, 64)  # x, g, c, k4, q, cb, j
    t = t.transpose(0, 5, 2, 1, 3, 6, 4)  # x, cb, c, g, k4, j, q
    return np.ascontiguousarray(t.reshape(a, co // 64, nci * 64))


def wino_weights_t(w: np.ndarray, tile: int = TILE) -> tuple[np.ndarray, np.ndarray]:
    """(Ut, tr): wino_weights' U in the wino_mm ops' tiled form (u_layout = 1, tile_u)."""
    u, tr = wino_weights(w, tile)
    return tile_u(u, variant(w.shape[2])[1]), tr


def tiles_rows(lo: int, dilation: int, groups: int, tile: int, kernel: int) -> int:
    """Rows of V: d * A * rmax, rmax = ceil(ceil(Lo / d) / 128) * (128 / tile) + groups - 1."""
    per_class = (lo + dilation - 1) // dilation
    rmax = (per_class + ROWS_TG - 1) // ROWS_TG * (ROWS_TG // tile) + groups - 1
    return rmax * dilation * alpha_of(kernel, tile)


def stats_chunks(lo: int, dilation: int) -> int:
    """Statistics chunks per residue class: ceil(ceil(Lo / d) / 128)."""
    return ((lo + dilation - 1) // dilation + ROWS_TG - 1) // ROWS_TG
