"""Start-cell locator on the GPU: a uniform grid over the sites and exact nearest-site queries (libvgr's
vgr_grid_build, vgr_grid_cell_points, vgr_grid_nearest_points).

It replaces the host-side cKDTree query of the reference's nearest_sites (sites.py:38-39), which finds the start
site of the traversal per camera centre (bench_infer.py:60, eval_scene.py:69) and per ray origin of a ray batch.
The answer is cKDTree's (float64 distances) up to exact distance ties, which go to the smaller site index."""

import ctypes
import math

import torch

from . import _lib


class SiteGrid:
	"""Sites binned into a uniform grid of about `per_cell` sites per cell (cubic cells over the bounding box).

	points: (N, 3) or (N, 4) float32 CUDA tensor (xyz first), kept by reference; the grid is built on its stream."""

	def __init__(self, points, per_cell=2.0):
		if not (isinstance(points, torch.Tensor) and points.is_cuda):
			raise RuntimeError('points must be a CUDA tensor')
		if points.dtype != torch.float32 or points.dim() != 2 or points.shape[1] < 3 or not points.is_contiguous():
			raise RuntimeError('points must be a contiguous float32 (N, 3) or (N, 4) tensor')
		n = len(points)
		if n == 0:
			raise RuntimeError('SiteGrid needs at least one site')
		self.points, self.stride, self.n = points, points.shape[1], n
		dev = points.device
		lo = points[:, :3].amin(0).double().cpu()
		hi = points[:, :3].amax(0).double().cpu()
		ext = torch.clamp(hi - lo, min=1e-6)
		lo = lo - 1e-6 * ext
		ext = ext * (1 + 2e-6)
		edge = (float(ext.prod()) * per_cell / n) ** (1.0 / 3.0)
		res = [int(min(max(math.ceil(float(e) / edge), 1), 1024)) for e in ext]
		while res[0] * res[1] * res[2] > 4096 * 4096:
			res = [max(r // 2, 1) for r in res]
		self.lo = [float(v) for v in lo]
		self.cell = [float(e) / r for e, r in zip(ext, res)]
		self.res = res
		n_cells = res[0] * res[1] * res[2]
		lib = _lib.load()
		self.cell_start = torch.empty(n_cells + 1, dtype=torch.int32, device=dev)
		self.cell_sites = torch.empty(n, dtype=torch.int32, device=dev)
		work = torch.empty(int(lib.vgr_grid_work_size(n, n_cells)), dtype=torch.int32, device=dev)
		self._geom = (_floats(self.lo), _floats(self.cell), _ints(self.res))
		_lib.call('vgr_grid_build', _lib.ptr(points), n, self.stride, *self._geom, _lib.ptr(self.cell_start),
				  _lib.ptr(self.cell_sites), _lib.ptr(work), _lib.stream_of(dev))
		self._work = work  # released once the asynchronous build has run (caching allocator, same stream)
		# the sites in cell order, (x, y, z, bits of the index) each, which the queries scan (a snapshot of points)
		self.cell_points = torch.empty(n, 4, dtype=torch.float32, device=dev)
		_lib.call('vgr_grid_cell_points', _lib.ptr(points), n, self.stride, _lib.ptr(self.cell_sites),
				  _lib.ptr(self.cell_points), _lib.stream_of(dev))

	def nearest(self, queries, order=None):
		"""Index (int32) of the nearest site of every query point: queries (m, 3) float32 CUDA tensor. order:
		optional int32 (m,) permutation of 0 .. m - 1, the order in which the queries are answered (query_order
		gives a coherent one); the answers do not depend on it."""
		if not (isinstance(queries, torch.Tensor) and queries.is_cuda):
			raise RuntimeError('queries must be a CUDA tensor')
		if queries.dtype != torch.float32 or queries.dim() != 2 or queries.shape[1] != 3 or not queries.is_contiguous():
			raise RuntimeError('queries must be a contiguous float32 (m, 3) tensor')
		if order is not None and not (isinstance(order, torch.Tensor) and order.is_cuda and order.dtype == torch.int32
									  and order.shape == (len(queries),) and order.is_contiguous()):
			raise RuntimeError('order must be a contiguous int32 CUDA tensor of one entry per query')
		out = torch.empty(len(queries), dtype=torch.int32, device=queries.device)
		_lib.call('vgr_grid_nearest_points', _lib.ptr(self.cell_points), self.n, *self._geom, _lib.ptr(self.cell_start),
				  _lib.ptr(queries), len(queries), _lib.ptr(order), _lib.ptr(out), _lib.stream_of(queries.device))
		return out

	def nearest_indexed(self, queries):
		"""nearest() reading the candidate sites through their indices into the point array (vgr_grid_nearest):
		the same answers."""
		if not (isinstance(queries, torch.Tensor) and queries.is_cuda):
			raise RuntimeError('queries must be a CUDA tensor')
		if queries.dtype != torch.float32 or queries.dim() != 2 or queries.shape[1] != 3 or not queries.is_contiguous():
			raise RuntimeError('queries must be a contiguous float32 (m, 3) tensor')
		out = torch.empty(len(queries), dtype=torch.int32, device=queries.device)
		_lib.call('vgr_grid_nearest', _lib.ptr(self.points), self.n, self.stride, *self._geom,
				  _lib.ptr(self.cell_start), _lib.ptr(self.cell_sites), _lib.ptr(queries), len(queries), _lib.ptr(out),
				  _lib.stream_of(queries.device))
		return out


def query_order(queries, pos_bits=8):
	"""A spatially coherent processing order of query points for SiteGrid.nearest: int32 (m,) permutation sorting
	them along the Z-order curve of pos_bits bits per axis over their bounding box (vgr_ray_order with one direction
	bin). The lanes of a wave then scan neighbouring cells."""
	from . import ext
	return ext.ray_order(queries, queries, dir_res=1, pos_bits=pos_bits)


def _floats(v):
	return (ctypes.c_float * 3)(*v)


def _ints(v):
	return (ctypes.c_int32 * 3)(*v)
