"""Host neighbour list for the calculator's host-graph route.

The reference calculator builds its host graph with matscipy or ASE
(``neighbor_list("ijS", atoms, cutoff)``, calculator.py:2973-2979) whenever the
device builder does not apply: open or mixed boundaries, fewer than 512 atoms
on a GPU (calculator.py:83-84, 165-173), or an explicit
``SYMMETRIX_NEIGHBOR_BACKEND=host``.  Neither library is a dependency here, so
this module gives the same ``"ijS"`` result from a k-d tree over the periodic
images: for receiver i, source j and integer cell shift S,
``pos[j] - pos[i] + S @ cell`` is shorter than the cutoff, self pairs at zero
shift excluded.  Edges come receiver-major (the order
``_receiver_major_neighbor_arrays`` produces, calculator.py:107-152), then by
source and shift.
"""

from __future__ import annotations

import itertools

import numpy as np
from scipy.spatial import cKDTree


def _image_reach(cell, pbc, cutoff):
    """Cells to search along each periodic axis: the lattice planes of axis a
    are 1/|inv[:, a]| apart."""
    reach = [0, 0, 0]
    if np.any(pbc):
        inv = np.linalg.inv(cell)
        for a in range(3):
            if pbc[a]:
                reach[a] = int(np.ceil(cutoff * np.linalg.norm(inv[:, a])))
    return reach


def neighbor_list_ijS(positions, cell, pbc, cutoff):
    """(receivers i, sources j, shifts S [E,3]) of all pairs closer than cutoff."""
    positions = np.asarray(positions, dtype=np.float64).reshape(-1, 3)
    cell = np.asarray(cell, dtype=np.float64).reshape(3, 3)
    pbc = np.asarray(pbc, dtype=bool).reshape(3)
    n = len(positions)
    if not (np.isfinite(cutoff) and cutoff > 0.0):
        raise ValueError("cutoff must be positive")
    if n == 0:
        return np.zeros(0, np.int32), np.zeros(0, np.int32), np.zeros((0, 3), np.int32)
    if not np.isfinite(positions).all():
        raise ValueError("positions must be finite")
    wrap = np.zeros((n, 3), dtype=np.int64)
    wpos = positions
    if np.any(pbc):
        if not (abs(np.linalg.det(cell)) > 0.0):
            raise ValueError("a periodic cell must be invertible")
        frac = positions @ np.linalg.inv(cell)
        wrap[:, pbc] = np.floor(frac[:, pbc]).astype(np.int64)
        wpos = positions - wrap @ cell
    reach = _image_reach(cell, pbc, cutoff)
    images = np.array(list(itertools.product(*[range(-r, r + 1) for r in reach])), dtype=np.int64)
    points = (wpos[None, :, :] + (images @ cell)[:, None, :]).reshape(-1, 3)
    tree = cKDTree(points)
    hits = tree.query_ball_point(wpos, r=np.nextafter(cutoff, 0.0), return_sorted=True)
    zero = int(np.nonzero(~images.any(axis=1))[0][0])
    rec, src, shf = [], [], []
    for i, found in enumerate(hits):
        if not found:
            continue
        found = np.asarray(found, dtype=np.int64)
        img, j = np.divmod(found, n)
        keep = ~((j == i) & (img == zero))
        img, j = img[keep], j[keep]
        S = images[img] - wrap[j] + wrap[i]
        order = np.lexsort((S[:, 2], S[:, 1], S[:, 0], j))
        rec.append(np.full(len(order), i, dtype=np.int32))
        src.append(j[order].astype(np.int32))
        shf.append(S[order].astype(np.int32))
    if not rec:
        return np.zeros(0, np.int32), np.zeros(0, np.int32), np.zeros((0, 3), np.int32)
    return np.concatenate(rec), np.concatenate(src), np.concatenate(shf)
