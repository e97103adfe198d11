"""GPU start-cell locator (vgr.grid / vgr_grid_build, vgr_grid_cell_points, vgr_grid_nearest_points, and
vgr_grid_nearest) against the exhaustive float64 oracle and scipy's cKDTree (the reference's nearest_sites,
sites.py:38-39): identical site indices, the same from both query kernels and in a coherent query order."""

import numpy as np
import pytest
import torch

import dense
from vgr import grid, render, scenes, sites

pytestmark = pytest.mark.gpu


def T(a, dev):
	return torch.as_tensor(np.ascontiguousarray(a), device=dev)


def gpu_nearest(dev, pts, q, **kw):
	"""Nearest sites through the cell-ordered copy (SiteGrid.nearest), checked equal to the kernel that reads the
	candidates through their indices (SiteGrid.nearest_indexed)."""
	g = grid.SiteGrid(T(pts, dev), **kw)
	qt = T(q, dev)
	out = g.nearest(qt)
	via_index = g.nearest_indexed(qt)
	ordered = g.nearest(qt, order=grid.query_order(qt))
	torch.cuda.synchronize()
	np.testing.assert_array_equal(out.cpu().numpy(), via_index.cpu().numpy())
	np.testing.assert_array_equal(out.cpu().numpy(), ordered.cpu().numpy())
	return out.cpu().numpy(), g


@pytest.mark.parametrize('per_cell', [0.5, 2.0, 16.0])
def test_uniform_sites_inside_and_outside(gpu, per_cell):
	rng = np.random.default_rng(11)
	pts = rng.uniform(-1, 1, (20000, 3)).astype(np.float32)
	q = np.concatenate([rng.uniform(-1, 1, (40000, 3)), rng.uniform(-1.6, 1.6, (20000, 3)),
						rng.normal(0, 3, (500, 3))]).astype(np.float32)
	got, g = gpu_nearest(gpu, pts, q, per_cell=per_cell)
	np.testing.assert_array_equal(got, dense.nearest_brute(pts, q))
	# the grid's CSR covers every site exactly once
	cs = g.cell_start.cpu().numpy()
	assert cs[0] == 0 and cs[-1] == len(pts) and (np.diff(cs) >= 0).all()
	np.testing.assert_array_equal(np.sort(g.cell_sites.cpu().numpy()), np.arange(len(pts)))
	# the cell-ordered copy: slot s holds site cell_sites[s], its position and the bits of its index
	cp, sites_ = g.cell_points.cpu().numpy(), g.cell_sites.cpu().numpy()
	np.testing.assert_array_equal(cp[:, :3], pts[sites_])
	np.testing.assert_array_equal(cp[:, 3].view(np.int32), sites_)


def test_clustered_and_shell_sites_match_ckdtree(gpu):
	"""Config-4-like layout: dense Gaussian clusters plus a 1/U shell out to r = 50 (most cells empty)."""
	from scipy.spatial import cKDTree
	rng = np.random.default_rng(12)
	clusters = rng.uniform(-1, 1, (32, 3))
	dense_pts = clusters[rng.integers(0, 32, 60000)] + rng.normal(0, 0.05, (60000, 3))
	u = rng.normal(size=(20000, 3))
	shell = u / np.linalg.norm(u, axis=1, keepdims=True) / rng.uniform(0.02, 1, (20000, 1))
	pts = np.concatenate([dense_pts, shell]).astype(np.float32)
	q = np.concatenate([rng.uniform(-1, 1, (100000, 3)), rng.uniform(-30, 30, (20000, 3))]).astype(np.float32)
	got, _ = gpu_nearest(gpu, pts, q)
	np.testing.assert_array_equal(got, cKDTree(pts.astype(np.float64)).query(q.astype(np.float64))[1])


def test_pack_points_stride4_lattice_ties_and_degenerate_extent(gpu):
	# stride-4 (pack['points']) input, on a lattice: equidistant queries go to the smaller index
	g3 = np.stack(np.meshgrid(*[np.arange(6.0)] * 3, indexing='ij'), -1).reshape(-1, 3)
	p4 = np.concatenate([g3, np.zeros((len(g3), 1))], 1).astype(np.float32)
	rng = np.random.default_rng(13)
	q = np.concatenate([rng.uniform(-1, 6, (5000, 3)), g3 + 0.5, g3[:50]]).astype(np.float32)
	got, _ = gpu_nearest(gpu, p4, q, per_cell=1.0)
	np.testing.assert_array_equal(got, dense.nearest_brute(g3, q))
	# all sites on one plane (zero extent along z), one site, no queries
	flat = np.concatenate([rng.uniform(-1, 1, (3000, 2)), np.zeros((3000, 1))], 1).astype(np.float32)
	qf = rng.uniform(-1.2, 1.2, (4000, 3)).astype(np.float32)
	np.testing.assert_array_equal(gpu_nearest(gpu, flat, qf)[0], dense.nearest_brute(flat, qf))
	one = np.array([[0.3, -0.2, 0.1]], np.float32)
	assert (gpu_nearest(gpu, one, qf)[0] == 0).all()
	assert len(gpu_nearest(gpu, flat, np.zeros((0, 3), np.float32))[0]) == 0


def test_nearest_sites_dispatch_and_errors(gpu):
	rng = np.random.default_rng(14)
	pts = rng.uniform(-1, 1, (5000, 3)).astype(np.float32)
	q = rng.uniform(-1, 1, (3000, 3)).astype(np.float32)
	host = sites.nearest_sites(pts, q)
	dev = sites.nearest_sites(T(pts, gpu), T(q, gpu))
	assert isinstance(host, np.ndarray) and dev.is_cuda and dev.dtype == torch.int32
	np.testing.assert_array_equal(dev.cpu().numpy(), host)
	# a batch above 65,536 queries is answered in its Z-order: the same answers
	qb = rng.uniform(-1.2, 1.2, (100000, 3)).astype(np.float32)
	np.testing.assert_array_equal(sites.nearest_sites(T(pts, gpu), T(qb, gpu)).cpu().numpy(),
								  sites.nearest_sites(pts, qb))
	with pytest.raises(RuntimeError, match='CUDA tensor'):
		grid.SiteGrid(torch.as_tensor(pts))
	with pytest.raises(RuntimeError, match='float32'):
		grid.SiteGrid(T(pts.astype(np.float64), gpu))
	with pytest.raises(RuntimeError, match='float32'):
		grid.SiteGrid(T(pts, gpu)).nearest(T(q[:, :2], gpu))


def test_camera_and_ray_batch_starts_match_host(gpu):
	"""Starts of a seeded scene: per camera centre (far outside the cloud) and per ray origin of a config-5 batch."""
	sc = scenes.make_scene(5, scale=0.005, n_rays=20000, cache_dir=None, log=None)
	o, _ = sc.ray_batch
	host = sites.nearest_sites(sc.points, o)
	np.testing.assert_array_equal(sites.nearest_sites(T(sc.points, gpu), T(o, gpu)).cpu().numpy(), host)
	c3 = scenes.make_scene(3, scale=0.002, img_scale=0.02, cache_dir=None, log=None)
	centers = np.stack([c.eye for c in c3.cameras]).astype(np.float32)
	np.testing.assert_array_equal(sites.nearest_sites(T(c3.points, gpu), T(centers, gpu)).cpu().numpy(),
								  sites.nearest_sites(c3.points, centers))
