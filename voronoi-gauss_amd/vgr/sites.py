"""Site graph of the field: Delaunay (Voronoi-neighbour) adjacency as int32 CSR, and nearest-site queries.

Mirrors sites.py:24-45 of the reference (delaunay_graph, nearest_sites, neighbor_spacing); both use scipy's
Qhull Delaunay and cKDTree, so the scene a caller builds here is the scene the reference would build. On CUDA
tensors nearest_sites runs on the GPU instead (vgr.grid)."""

import numpy as np
from scipy.spatial import Delaunay, cKDTree


def delaunay_graph(points):
	"""-> (points kept, index of the kept points, CSR offsets (N + 1), adjacency (M)), int32. Points left out of
	the triangulation by Qhull (coplanar / nearly coincident) are dropped and the triangulation rebuilt, up to
	three times (sites.py:24-35)."""
	idx = np.arange(len(points))
	for _ in range(3):
		tri = Delaunay(points[idx])
		offsets, adj = tri.vertex_neighbor_vertices
		alone = np.diff(offsets) == 0
		if not alone.any():
			return points[idx], idx, offsets.astype(np.int32), adj.astype(np.int32)
		idx = idx[~alone]
	raise RuntimeError('Delaunay triangulation keeps dropping points')


def nearest_sites(points, queries):
	"""Index of the nearest site of every query point (sites.py:38-39). numpy arrays: scipy's cKDTree, as the
	reference does; CUDA tensors: the GPU grid of vgr.grid.SiteGrid (the same answers up to exact distance ties,
	which go to the smaller index), returned as an int32 CUDA tensor."""
	if getattr(points, 'is_cuda', False):
		from .grid import SiteGrid
		return SiteGrid(points.contiguous()).nearest(queries.contiguous())
	return cKDTree(points).query(queries)[1].astype(np.int32)


def neighbor_spacing(points, k=3):
	"""Mean distance to the k nearest other sites (sites.py:42-45)."""
	d, _ = cKDTree(points).query(points, k + 1)
	return d[:, 1:].mean(1)
