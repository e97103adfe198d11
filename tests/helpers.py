"""Shared test inputs: small random fields like the reference tests build (test_foam.py:41-59,
test_march.py:33-53, test_grad.py:52-86) and CPU packing through the oracle's conics."""

import numpy as np
import torch
from scipy.spatial import cKDTree

import oracle
from vgr.render import pack_foam_arrays
from vgr.sites import delaunay_graph


class Field:
	"""Random anisotropic field over a Delaunay graph, numpy float32."""

	def __init__(self, seed=2, n=300, lo=-0.9, hi=0.9, raw_mu=1.0, ls_mu=-1.8, sh_deg=3):
		rng = np.random.default_rng(seed)
		pts, _, offsets, adj = delaunay_graph(rng.uniform(lo, hi, (n, 3)).astype(np.float32).astype(np.float64))
		self.points = pts.astype(np.float32)
		self.offsets, self.adj = offsets, adj
		n = len(pts)
		self.raw = (rng.normal(size=n) * 0.5 + raw_mu).astype(np.float32)
		self.d_log_scale = (rng.normal(size=(n, 3)) * 0.3 + ls_mu).astype(np.float32)
		self.d_quat = rng.normal(size=(n, 4)).astype(np.float32)
		self.c_log_scale = (rng.normal(size=(n, 3)) * 0.3 + ls_mu).astype(np.float32)
		self.c_quat = rng.normal(size=(n, 4)).astype(np.float32)
		sh = (rng.normal(size=(n, 16, 3)) * 0.3).astype(np.float32)
		if sh_deg < 3:
			sh[:, (sh_deg + 1) ** 2:] = 0
		self.sh = sh
		self.sh_deg = sh_deg
		self.tree = cKDTree(self.points)

	@property
	def n(self):
		return len(self.points)

	def conics(self, floor=0.0):
		return oracle.conic(self.d_log_scale, self.d_quat, floor), oracle.conic(self.c_log_scale, self.c_quat, floor)

	def pack(self, floor=0.0, eps_density=0.0, sh_half=False, reorder=False):
		"""render.pack_foam_arrays on CPU tensors with the oracle's conics -> dict of numpy arrays."""
		dA, cA = self.conics(floor)
		t = torch.from_numpy
		p = pack_foam_arrays(t(self.points), t(self.offsets), t(self.adj), t(self.raw), t(self.d_log_scale),
							 t(self.c_log_scale), t(dA), t(cA), t(self.sh), floor, eps_density, sh_half, reorder)
		out = {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
		out['dA'], out['cA'] = dA, cA
		return out

	def rays(self, B=64, seed=2, lo=-0.5, hi=0.5, far_radius=2.0, near=0.02):
		"""o ~ U[lo, hi]^3, d ~ normalised N(0, I), start = nearest site of o, ray_bounds."""
		rng = np.random.default_rng(100 + seed)
		o = rng.uniform(lo, hi, (B, 3)).astype(np.float32)
		d = rng.normal(size=(B, 3))
		d = (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)
		start = self.tree.query(o)[1].astype(np.int32)
		near_t, mid_t, far_t = ray_bounds_np(o, d, near, far_radius)
		return o, d, start, near_t, mid_t, far_t


def ray_bounds_np(o, d, near, far_radius):
	"""render.ray_bounds evaluated with torch on CPU (float32), as numpy."""
	from vgr.render import ray_bounds
	n, m, f = ray_bounds(torch.from_numpy(np.ascontiguousarray(o)), torch.from_numpy(np.ascontiguousarray(d)), near,
						 far_radius)
	return n.numpy(), m.numpy(), f.numpy()


def trace_list(trace_row, n):
	return [int(c) for c in trace_row[:n]]
