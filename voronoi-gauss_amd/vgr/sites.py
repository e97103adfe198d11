"""Site graph of the field: Delaunay (Voronoi-neighbour) adjacency as int32 CSR, and nearest-site queries.

Mirrors sites.py:24-45 of the reference (delaunay_graph, nearest_sites, neighbor_spacing); both use scipy's
Qhull Delaunay and cKDTree, so the scene a caller builds here is the scene the reference would build. On CUDA
tensors nearest_sites runs on the GPU instead (vgr.grid)."""

import numpy as np
from scipy.spatial import Delaunay, cKDTree


def delaunay_graph(points, attempts=3):
	"""Delaunay neighbours of the points as int32 CSR -> (kept points, their indices into `points`, offsets
	(N + 1), adjacency (M)). Qhull leaves some points out of the triangulation (duplicates, near-coincident
	points); such points have no neighbours, so they are removed and the rest triangulated again, at most
	`attempts` times in all, the rule of the reference's sites.py:24-35."""
	kept = np.arange(len(points))
	for _ in range(attempts):
		offsets, adj = Delaunay(points[kept]).vertex_neighbor_vertices
		isolated = offsets[1:] == offsets[:-1]
		if not isolated.any():
			return points[kept], kept, offsets.astype(np.int32), adj.astype(np.int32)
		kept = kept[~isolated]
	raise RuntimeError(f'Qhull still leaves points without neighbours after {attempts} triangulations')


def nearest_sites(points, queries):
	"""Index of the nearest site of every query point (sites.py:38-39). numpy arrays: scipy's cKDTree, as the
	reference does; CUDA tensors: the GPU grid of vgr.grid.SiteGrid (the same answers up to exact distance ties,
	which go to the smaller index; batches above 65,536 queries answered in their Z-order), returned as an int32 CUDA
	tensor."""
	if getattr(points, 'is_cuda', False):
		from .grid import SiteGrid, query_order
		q = queries.contiguous()
		# large batches (a ray batch's origins) are answered in their Z-order, which lets a wave's lanes share cells
		return SiteGrid(points.contiguous()).nearest(q, order=query_order(q) if len(q) > 65536 else None)
	return cKDTree(points).query(queries, workers=-1)[1].astype(np.int32)


def neighbor_spacing(points, k=3):
	"""Mean distance to the k nearest other sites (sites.py:42-45)."""
	d, _ = cKDTree(points).query(points, k + 1)
	return d[:, 1:].mean(1)
