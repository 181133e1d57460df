"""Oracle evaluation of one probe atom of a large periodic system on the
subgraph that determines its energy and force (test infrastructure).

With two interactions, atom k's energy reads the atoms within two edges of
k, and its force (the derivative of every energy with respect to k's
position) reads the energies within two edges of k, hence atoms within four
edges.  The subgraph holds the atoms within three edges of k with their full
neighbour lists and the atoms at four edges as nodes without edges; k's
energy and force on it equal the whole system's.
"""

import numpy as np


def probe_subgraph(pos, types, L, probe, cutoff, r_cut, hops=3):
    """The oracle's subgraph around `probe` in a cubic periodic box of side L:
    (node types, num_neigh, neighbour indices, xyz, r, index of the probe)."""
    from scipy.sparse import coo_matrix
    from scipy.sparse.csgraph import shortest_path
    from scipy.spatial import cKDTree

    reach = (hops + 1) * cutoff + 0.5
    if 2 * reach >= L:
        raise ValueError("the box (%.1f A) is too small for a %.1f A probe neighbourhood" % (L, reach))
    d = pos - pos[probe]
    d -= L * np.round(d / L)
    local = np.nonzero(np.einsum("ij,ij->i", d, d) < reach * reach)[0]
    lp = d[local]
    pairs = cKDTree(lp).query_pairs(cutoff, output_type="ndarray")
    m = len(local)
    i = np.concatenate([pairs[:, 0], pairs[:, 1]])
    j = np.concatenate([pairs[:, 1], pairs[:, 0]])
    adj = coo_matrix((np.ones(len(i)), (i, j)), shape=(m, m)).tocsr()
    p = int(np.nonzero(local == probe)[0][0])
    hop = shortest_path(adj, unweighted=True, indices=p)
    keep = np.nonzero(hop <= hops + 1)[0]
    order = keep[np.argsort(hop[keep], kind="stable")]     # probe first, then by hop
    sub = np.full(m, -1, np.int64)
    sub[order] = np.arange(len(order))
    num_neigh = np.zeros(len(order), np.int32)
    neigh, xyz = [], []
    for s, a in enumerate(order):
        if hop[a] > hops:
            continue
        nb = adj.indices[adj.indptr[a]:adj.indptr[a + 1]]
        nb = np.sort(nb)
        assert np.all(sub[nb] >= 0), "a receiver's neighbour is outside the subgraph"
        num_neigh[s] = len(nb)
        neigh.append(sub[nb])
        xyz.append(lp[nb] - lp[a])
    neigh = np.concatenate(neigh).astype(np.int32)
    xyz = np.concatenate(xyz)
    r = np.linalg.norm(xyz, axis=1)
    scale = np.where(r >= r_cut, r_cut / r, 1.0)   # edges past the cutoff are clamped to it
    return types[local[order]], num_neigh, neigh, xyz * scale[:, None], r * scale, 0


def oracle_probe(om, pos, types, L, probe, cutoff, hops=3):
    """(energy, force, receivers of the subgraph) of `probe` from the oracle."""
    from oracle import oracle
    st, nn, neigh, xyz, r, p = probe_subgraph(pos, types, L, probe, cutoff, om.r_cut, hops)
    e, f = om.evaluate(st, nn, neigh, st[neigh], xyz, r)
    receivers = np.repeat(np.arange(len(st), dtype=np.int32), nn)
    F = oracle.reduce_forces(len(st), receivers, neigh, f)
    return e[p], F[p], int(np.count_nonzero(nn))
