"""Host-side logic on CPU: ray bounds, the inference pack (render.pack_foam_arrays), Morton order, pixel tiles,
seeded scenes and cameras. Closed forms and format invariants; no GPU."""

import math
import os

import numpy as np
import torch

from helpers import Field
from vgr import render, scenes


def test_ray_bounds_closed_form():
	o = torch.tensor([[0.0, 0.0, 3.0], [0.2, -0.1, 0.0], [0.0, 0.0, 0.0]])
	d = torch.nn.functional.normalize(torch.tensor([[0.0, 0.0, -1.0], [1.0, 0.0, 0.0], [0.0, 1.0, 0.0]]), dim=-1)
	near, mid, far = render.ray_bounds(o, d, 0.02, 4.0)
	assert torch.all(near == 0.02)
	# exits of the unit sphere and of the radius-4 sphere, solved by hand
	np.testing.assert_allclose(mid.numpy(), [4.0, -0.2 + math.sqrt(0.04 + 1 - 0.05), 1.0], rtol=1e-6)
	np.testing.assert_allclose(far.numpy(), [7.0, -0.2 + math.sqrt(0.04 + 16 - 0.05), 4.0], rtol=1e-6)
	# a ray that never enters the unit sphere: mid clamped to near + 1e-3, far >= mid + 1e-3
	n2, m2, f2 = render.ray_bounds(torch.tensor([[0.0, 5.0, 0.0]]), torch.tensor([[0.0, 1.0, 0.0]]), 0.02, 4.0)
	assert abs(m2.item() - 0.021) < 1e-7 and abs(f2.item() - 0.022) < 1e-7


def test_cut_bits_round_to_nearest_even_and_order():
	r2 = torch.tensor([float('inf'), 1.0, 0.1, 65504.0])
	lam = torch.tensor([3.0, 0.33333334, 65000.0, 1e-8])
	bits = render.cut_bits(r2, lam).view(torch.int32).numpy().astype(np.uint32)
	lo, hi = (bits & 0xffff).astype(np.uint16), (bits >> 16).astype(np.uint16)
	np.testing.assert_array_equal(lo.view(np.float16), r2.numpy().astype(np.float16))
	np.testing.assert_array_equal(hi.view(np.float16), lam.numpy().astype(np.float16))
	# the safety factors exceed half precision's relative half-ulp (2^-11)
	assert (1 + 2 ** -9) > (1 + 2 ** -11) and (1 - 2 ** -9) < (1 - 2 ** -11)


def test_pack_self_first_csr_and_records():
	f = Field(seed=3, n=200)
	pk = f.pack(eps_density=1e-3)
	n, off, nbr = f.n, pk['offsets'], pk['nbr']
	assert len(off) == n + 1 and off[-1] == len(nbr) == len(f.adj) + n
	for c in range(n):
		row = nbr[off[c]:off[c + 1]]
		assert row[0] == c
		np.testing.assert_array_equal(row[1:], f.adj[f.offsets[c]:f.offsets[c + 1]])
	np.testing.assert_array_equal(pk['edge'][:, :3], f.points[nbr])
	np.testing.assert_array_equal(pk['points'][:, :3], f.points)
	A = pk['attr']
	np.testing.assert_array_equal(A[:, :6], pk['dA'])
	np.testing.assert_array_equal(A[:, 6], np.minimum(f.raw, 30))
	np.testing.assert_array_equal(A[:, 8:14], pk['cA'])
	assert (A[:, [7, 14, 15, 16, 17, 18, 19]] == 0).all()
	# r2 = 2 s_max^2 max(raw - ln eps, 0) (1 + 2^-9), lam = min eigenvalue of the colour conic (1 - 2^-9), as half
	bits = pk['edge'][:, 3].view(np.uint32)
	r2h = (bits & 0xffff).astype(np.uint16).view(np.float16).astype(np.float64)
	lamh = (bits >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
	s_max2 = np.exp(2 * f.d_log_scale.astype(np.float64)).max(1)
	r2 = 2 * s_max2 * np.maximum(f.raw - math.log(1e-3), 0) * (1 + 2 ** -9)
	np.testing.assert_allclose(r2h, r2[nbr], rtol=2 ** -10)
	lam = 1 / np.exp(2 * f.c_log_scale.astype(np.float64)).max(1) * (1 - 2 ** -9)
	np.testing.assert_allclose(lamh, np.minimum(lam, 65000)[nbr], rtol=2 ** -10)
	# eps = 0: every density term is kept
	pk0 = f.pack()
	r2h0 = (pk0['edge'][:, 3].view(np.uint32) & 0xffff).astype(np.uint16).view(np.float16)
	assert np.isinf(r2h0).all()


def test_pack_cut_word_is_per_site():
	"""Every edge record pointing at site k carries k's cut-off word (the self entry's): the premise of the indexed
	records, which store it once per site (attr column 7, zero padding in the reference layout)."""
	f = Field(seed=6, n=250)
	for pk in (f.pack(), f.pack(eps_density=1e-3, reorder=True)):
		cut = pk['edge'][pk['offsets'][:-1], 3].view(np.int32)
		np.testing.assert_array_equal(pk['edge'][:, 3].view(np.int32), cut[pk['nbr']])
		assert (pk['attr'][:, 7] == 0).all()


def test_pack_reorder_keeps_neighbour_order():
	f = Field(seed=4, n=300)
	a, b = f.pack(), f.pack(reorder=True)
	perm, inv = b['perm'], b['inv']
	np.testing.assert_array_equal(inv[perm], np.arange(f.n))
	np.testing.assert_array_equal(b['orig'], perm)
	for c_new in range(f.n):
		c_old = perm[c_new]
		row_new = b['nbr'][b['offsets'][c_new]:b['offsets'][c_new + 1]]
		row_old = a['nbr'][a['offsets'][c_old]:a['offsets'][c_old + 1]]
		np.testing.assert_array_equal(perm[row_new], row_old)  # same neighbours, same order
	np.testing.assert_array_equal(b['attr'], a['attr'][perm])
	np.testing.assert_array_equal(b['sh'], a['sh'][perm])


def test_morton_order_is_a_z_curve():
	pts = torch.tensor([[0.0, 0, 0], [1, 1, 1], [1, 0, 0], [0, 1, 0], [0, 0, 1]])
	order = render.morton_order(pts, bits=1).tolist()
	# codes: x bit 0, y bit 1, z bit 2 -> (0,0,0)=0, (1,0,0)=1, (0,1,0)=2, (0,0,1)=4, (1,1,1)=7
	assert order == [0, 2, 3, 4, 1]


def test_tile_order_groups_8x8_tiles():
	H, W = 20, 30
	perm = scenes.tile_order(H, W)
	assert sorted(perm.tolist()) == list(range(H * W))
	y, x = perm // W, perm % W
	first = perm[:64]
	assert set((first // W).tolist()) == set(range(8)) and set((first % W).tolist()) == set(range(8))
	for t in range(len(perm) // 64):  # every run of 64 lies inside one 8x8 tile
		ys, xs = y[64 * t:64 * t + 64] // 8, x[64 * t:64 * t + 64] // 8
		if len(set(zip(ys.tolist(), xs.tolist()))) != 1:
			break
	else:
		raise AssertionError('expected partial tiles at the image border')


def test_morton_tile_order():
	"""Z-order of the tiles: the same tiles as the row order, each tile's pixels in the same order, and the tiles
	of a 64 x 64 image (8 x 8 tiles) visited along the Z curve: every aligned run of 4 tiles is a 2 x 2 block and
	every run of 16 a 4 x 4 block."""
	H, W = 64, 64
	perm = scenes.tile_order(H, W, curve='morton')
	row = scenes.tile_order(H, W, curve='row')
	assert sorted(perm.tolist()) == list(range(H * W))
	tiles = perm.reshape(-1, 64)
	rows = row.reshape(-1, 64)
	ty, tx = tiles[:, 0] // W // 8, tiles[:, 0] % W // 8
	np.testing.assert_array_equal(tiles, rows[ty * 8 + tx])
	assert scenes.morton2(np.array([0, 0, 1, 1, 2]), np.array([0, 1, 0, 1, 0])).tolist() == [0, 1, 2, 3, 8]
	for n, side in ((4, 2), (16, 4)):
		for s in range(0, 64, n):
			assert len(set(ty[s:s + n].tolist())) == side and len(set(tx[s:s + n].tolist())) == side
	assert ty[:4].tolist() == [0, 0, 1, 1] and tx[:4].tolist() == [0, 1, 0, 1]


def test_camera_rays_convention():
	cam = scenes.Camera(np.array([0.0, 0.0, 3.0]), np.zeros(3), np.array([0.0, 1.0, 0.0]), 64, 48)
	o, d = cam.rays()
	assert o.shape == (64 * 48, 3) and np.allclose(np.linalg.norm(d, axis=1), 1, atol=1e-6)
	# pixel centres: the 4 central pixels straddle the optical axis (looking down -z), +x right, +y (image) down
	c = d.reshape(48, 64, 3)
	centre = c[23:25, 31:33].reshape(-1, 3).mean(0)
	np.testing.assert_allclose(centre / np.linalg.norm(centre), [0, 0, -1], atol=1e-6)
	assert c[24, 63, 0] > 0 and c[47, 32, 1] < 0
	fx, _, cx, _ = cam.intrinsics()
	assert abs(fx - 32 / math.tan(math.radians(30))) < 1e-9 and cx == 32


def test_scene_generation_is_seeded():
	a = scenes.make_scene(3, scale=0.002, img_scale=0.02, cache_dir=None, log=None)
	b = scenes.make_scene(3, scale=0.002, img_scale=0.02, cache_dir=None, log=None)
	for k in ('points', 'offsets', 'adj', 'raw', 'log_scale', 'sh'):
		np.testing.assert_array_equal(getattr(a, k), getattr(b, k))
	assert a.sh_deg == 3 and len(a.cameras) == 4 and a.far_radius == 4.0
	c1 = scenes.make_scene(1, cache_dir=None, log=None)
	assert c1.n_sites <= 16384 and c1.sh_deg == 0 and (c1.sh[:, 1:] == 0).all()
	assert c1.cameras[0].width == 128 and np.allclose(c1.cameras[0].eye, [0, 0, 3])
	c5 = scenes.make_scene(5, scale=0.001, n_rays=1000, cache_dir=None, log=None)
	o, d = c5.ray_batch
	assert o.shape == (1000, 3) and np.abs(o).max() <= 0.9 and np.allclose(np.linalg.norm(d, axis=1), 1, atol=1e-6)
	c4 = scenes.make_scene(4, scale=0.0005, img_scale=0.01, cache_dir=None, log=None)
	assert c4.far_radius == 55.0 and np.linalg.norm(c4.points, axis=1).max() <= 50.0 + 1e-3


def test_delaunay_graph_matches_scipy_and_drops_duplicates():
	from scipy.spatial import Delaunay

	from vgr.sites import delaunay_graph
	rng = np.random.default_rng(0)
	p = rng.uniform(-1, 1, (200, 3))
	pts, idx, off, adj = delaunay_graph(p)
	o2, a2 = Delaunay(p).vertex_neighbor_vertices
	np.testing.assert_array_equal(off, o2)
	np.testing.assert_array_equal(adj, a2)
	assert off.dtype == np.int32 and adj.dtype == np.int32
	q = np.concatenate([p, p[:3]])  # duplicates are left out by Qhull and dropped
	pts, idx, off, adj = delaunay_graph(q)
	assert len(pts) <= 200 and (np.diff(off) > 0).all()


def test_profiles_bind_the_default_workloads_to_these_sources():
	"""The DRAM traffic that bench.py's roofline reads for its two default workloads (config 3 foam_infer, config 5
	march) comes from a committed rocprofv3 profile measured on these kernel sources; a kernel change without a new
	profile would leave the bench's roofline empty."""
	import sys
	root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
	if root not in sys.path:
		sys.path.insert(0, root)
	import bench
	for key, src in (('config3-scale1.0-fused-reorder1-l1-tiles8morton-idx', bench.source_hash('foam_infer.hip')),
					 ('config5-scale1.0-march-l1-order4x8', bench.source_hash('march.hip', 'order.hip'))):
		traffic, where = bench.measured_traffic(key, src)
		assert traffic is not None and traffic > 0, where


def test_bench_refuses_more_than_one_gpu():
	"""bench.py measures one GPU: --gpus N > 1 exits non-zero with a message, before touching a device."""
	import subprocess
	import sys
	root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
	p = subprocess.run([sys.executable, os.path.join(root, 'bench.py'), '--gpus', '2'], capture_output=True, text=True,
					   cwd=root, timeout=120)
	assert p.returncode != 0 and 'one GPU' in (p.stdout + p.stderr)


def test_s_to_t_rounds_like_the_reference():
	"""render.s_to_t bit for bit against render.py:28-33 restated in numpy float32, operation by operation
	(lin = n + (m - n) min(2 s, 1); disparity 1 / (1/m + u (1/f - 1/m)), u = max(2 s - 1, 0)), on 4096 rays x 64
	coordinates including s = 0, 1/2 and 1."""
	from vgr.render import s_to_t
	rng = np.random.default_rng(5)
	B, S = 4096, 64
	n = np.full(B, 0.02, np.float32)
	m = rng.uniform(0.5, 3.0, B).astype(np.float32)
	f = (m + rng.uniform(1e-3, 50.0, B)).astype(np.float32)
	s = np.sort(rng.uniform(0, 1, (B, S)).astype(np.float32), 1)
	s[:, 0], s[:, S // 2], s[:, -1] = 0.0, 0.5, 1.0
	got = s_to_t(torch.from_numpy(s), torch.from_numpy(n), torch.from_numpy(m), torch.from_numpy(f)).numpy()
	one, two = np.float32(1), np.float32(2)
	nn, mm, ff = n[:, None], m[:, None], f[:, None]
	lin = nn + (mm - nn) * np.minimum(two * s, one)
	u = np.maximum(two * s - one, np.float32(0))
	disp = one / (one / mm + u * (one / ff - one / mm))
	want = np.where(s < np.float32(0.5), lin, disp)
	assert got.dtype == np.float32
	np.testing.assert_array_equal(got, want)
	np.testing.assert_allclose(got[:, 0], n, rtol=0)
	np.testing.assert_allclose(got[:, -1], f, rtol=1e-5)  # three reciprocals: a few ulps


def test_sample_pdf_inverts_the_cdf():
	"""render.sample_pdf (render.py:36-50): bit for bit against the reference's sequence of torch operations
	restated here (pdf, cumsum, linspace levels, searchsorted right, clamped gathers, the 1e-5 span guard); and the
	closed form: each sample is the float64 inverse of the piecewise-linear CDF of weights + 1e-5 at its level."""
	from vgr.render import sample_pdf
	rng = np.random.default_rng(6)
	B, S, n = 512, 63, 64
	bins = torch.from_numpy(np.sort(rng.uniform(0, 1, (B, S + 1)).astype(np.float32), 1))
	w = rng.exponential(1.0, (B, S)).astype(np.float32)
	w[::7] = 0.0  # all-zero rows: the 1e-5 floor makes the pdf uniform
	w[1::5, 10:20] = 0.0
	weights = torch.from_numpy(w)
	got = sample_pdf(bins, weights, n, det=True)
	ww = weights + 1e-5
	pdf = ww / ww.sum(-1, keepdim=True)
	cdf = torch.cat([torch.zeros_like(pdf[:, :1]), torch.cumsum(pdf, -1)], -1)
	u = torch.linspace(0.5 / n, 1 - 0.5 / n, n).expand(B, n).contiguous()
	inds = torch.searchsorted(cdf, u, right=True)
	below, above = (inds - 1).clamp_min(0), inds.clamp_max(cdf.shape[-1] - 1)
	cb, ca = cdf.gather(1, below), cdf.gather(1, above)
	bb, ba = bins.gather(1, below), bins.gather(1, above)
	denom = torch.where(ca - cb < 1e-5, torch.ones_like(ca), ca - cb)
	want = bb + (u - cb) / denom * (ba - bb)
	assert torch.equal(got, want)
	# closed form in float64
	c64 = np.concatenate([np.zeros((B, 1)), np.cumsum((w + 1e-5) / (w + 1e-5).sum(1, keepdims=True), 1)], 1)
	lev = (np.arange(n) + 0.5) / n
	b64 = bins.numpy().astype(np.float64)
	for r in range(0, B, 37):
		np.testing.assert_allclose(got[r].numpy(), np.interp(lev, c64[r], b64[r]), atol=2e-5)
