"""GPU parity of march_forward and of the vgf forward operators (walk, density, color, conic) against the CPU
oracle on identical inputs: walked sites bit-exact, values within 1e-4 (fp32)."""

import numpy as np
import pytest
import torch

import oracle
from helpers import Field
from vgr import ext, render, scenes

pytestmark = pytest.mark.gpu


def T(a, dev):
	return torch.as_tensor(np.ascontiguousarray(a), device=dev)


def gpu_march(dev, f, dA, cA, rays, dt, n_bg, t_thresh, w_thresh, trace_cap=0, sh=None, sh_deg=3, lanes=0):
	o, d, start, near, mid, far = rays
	out = ext.march_extension().march_forward(
		T(f.points, dev), T(f.offsets, dev), T(f.adj, dev), T(f.raw, dev), T(dA, dev), T(cA, dev),
		T(f.sh if sh is None else sh, dev), sh_deg, T(o, dev), T(d, dev), T(start, dev), T(near, dev), T(mid, dev),
		T(far, dev), dt, n_bg, t_thresh, w_thresh, trace_cap=trace_cap, lanes=lanes)
	torch.cuda.synchronize()
	return [x.cpu().numpy() for x in out]


@pytest.mark.parametrize('lanes', [1, 16])
@pytest.mark.parametrize('thresholds', [(0.0, -1.0), (1e-4, 1e-4)])
def test_march_vs_oracle(gpu, thresholds, lanes):
	"""test_march.py:33-55 setup (300 sites, B=64 -> 256, dt=0.05, n_bg=8, floor 0.01), in both ray layouts."""
	f = Field(seed=1, n=300)
	rays = f.rays(B=256, seed=1)
	dA, cA = f.conics(0.01)
	rgb, Tt, depth, stats, trace = gpu_march(gpu, f, dA, cA, rays, 0.05, 8, *thresholds, trace_cap=256, lanes=lanes)
	r = oracle.march_forward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, *rays, 0.05, 8, *thresholds,
							 trace_cap=256)
	np.testing.assert_allclose(rgb, r['rgb'], atol=1e-4)
	np.testing.assert_allclose(Tt, r['T'], atol=1e-4)
	assert (stats == r['stats']).all(1).mean() >= 0.98
	n = np.minimum(stats[:, 0], r['stats'][:, 0])
	for i in range(len(n)):
		np.testing.assert_array_equal(trace[i, :n[i]], r['trace'][i, :n[i]])


def test_march_default_step_config1(gpu):
	"""render_rays_uniform defaults (dt = 1/512, n_bg = 64, floor dt/2) on the config-1 scene, one 64x64 view."""
	sc = scenes.make_scene(1, img_scale=0.5, cache_dir=None, log=None)
	from vgr.model import VoronoiGaussField
	model = VoronoiGaussField.from_scene(sc, 'cuda')
	o, d, start, _ = sc.camera_rays(tile=8)
	dev = gpu
	to, tdv, ts = T(o, dev), T(d, dev), T(start, dev)
	out = render.render_rays_uniform(model, to, tdv, ts)
	near, mid, far = render.ray_bounds(to, tdv, 0.02, 4.0)
	dA = oracle.conic(sc.log_scale, sc.quat, 1 / 1024)
	r = oracle.march_forward(sc.points, sc.offsets, sc.adj, sc.raw, dA, dA, sc.sh, 0, o, d, start, near.cpu().numpy(),
							 mid.cpu().numpy(), far.cpu().numpy(), 1 / 512, 64)
	np.testing.assert_allclose(out['rgb'].cpu().numpy(), r['rgb'] + r['T'][:, None] * 0.5, atol=1e-4)
	np.testing.assert_allclose(out['acc'].cpu().numpy(), 1 - r['T'], atol=1e-4)


@pytest.mark.parametrize('sh_deg', [3, 1])
def test_march_layouts_agree(gpu, sh_deg):
	"""One ray per lane and 16 lanes per ray on the same rays (default thresholds, 1/64 steps): the same sites in
	the same order, the same counts, colours within 1e-5 (the sums are added in another order)."""
	f = Field(seed=4, n=400, sh_deg=sh_deg)
	rays = f.rays(B=512, seed=4)
	dA, cA = f.conics(0.01)
	a = gpu_march(gpu, f, dA, cA, rays, 1 / 64, 16, 1e-4, 1e-4, trace_cap=512, sh_deg=sh_deg, lanes=1)
	b = gpu_march(gpu, f, dA, cA, rays, 1 / 64, 16, 1e-4, 1e-4, trace_cap=512, sh_deg=sh_deg, lanes=16)
	assert a[3][:, 0].max() < 512
	np.testing.assert_array_equal(a[4], b[4])
	np.testing.assert_array_equal(a[3], b[3])
	np.testing.assert_allclose(a[0], b[0], atol=1e-5)
	np.testing.assert_allclose(a[1], b[1], atol=1e-5)
	np.testing.assert_allclose(a[2], b[2], atol=1e-4)
	with pytest.raises(RuntimeError, match='lanes_per_ray'):
		gpu_march(gpu, f, dA, cA, rays, 1 / 64, 16, 1e-4, 1e-4, lanes=8)


def test_march_errors(gpu):
	f = Field(seed=1, n=100)
	rays = f.rays(B=8, seed=1)
	dA, cA = f.conics(0.01)
	with pytest.raises(RuntimeError, match='sh must be'):
		gpu_march(gpu, f, dA, cA, rays, 0.05, 8, 0, -1, sh=f.sh.reshape(len(f.sh), 48))
	with pytest.raises(RuntimeError, match='dt'):
		gpu_march(gpu, f, dA, cA, rays, 0.0, 8, 0, -1)
	empty = tuple(a[:0] for a in rays)
	out = gpu_march(gpu, f, dA, cA, empty, 0.05, 8, 0, -1)
	assert out[0].shape == (0, 3)


def test_walk_vs_oracle(gpu):
	f = Field(seed=0, n=400, lo=-1.0, hi=1.0)
	rng = np.random.default_rng(7)
	o = rng.uniform(-1.2, 1.2, (500, 3)).astype(np.float32)
	d = rng.normal(size=(500, 3))
	d = (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)
	z = np.sort(rng.uniform(0, 2.5, (500, 40)), 1).astype(np.float32)
	start = f.tree.query(o)[1].astype(np.int32)
	g = ext.Graph(T(f.points, gpu), T(f.offsets, gpu), T(f.adj, gpu))
	site, steps = g.walk(T(o, gpu), T(d, gpu), T(z, gpu), T(start, gpu))
	rs, rsteps = oracle.walk(f.points, f.offsets, f.adj, o, d, z, start)
	np.testing.assert_array_equal(site.cpu().numpy(), rs)
	np.testing.assert_array_equal(steps.cpu().numpy(), rsteps)


def test_density_color_conic_vs_oracle(gpu):
	f = Field(seed=0, n=400, lo=-1.0, hi=1.0, raw_mu=0.0, ls_mu=-1.2)
	rng = np.random.default_rng(8)
	x = rng.uniform(-1, 1, (3000, 3)).astype(np.float32)
	site = f.tree.query(x)[1].astype(np.int32)
	dirs = rng.normal(size=(3000, 3)).astype(np.float32)
	g = ext.Graph(T(f.points, gpu), T(f.offsets, gpu), T(f.adj, gpu))
	for mult in (1.0, 4.0, 2.0):
		s = ext.density(g, T(f.raw, gpu), T(f.d_log_scale, gpu), T(f.d_quat, gpu), T(x, gpu), T(site, gpu), mult)
		r = oracle.density(f.points, f.offsets, f.adj, f.raw, f.d_log_scale, f.d_quat, x, site, mult)
		np.testing.assert_allclose(s.cpu().numpy(), r, rtol=1e-5, atol=1e-4)
	for deg in (0, 1, 2, 3):
		c = ext.color(g, T(f.c_log_scale, gpu), T(f.c_quat, gpu), T(f.sh, gpu), T(x, gpu), T(dirs, gpu),
					  T(site, gpu), deg)
		r = oracle.color(f.points, f.offsets, f.adj, f.c_log_scale, f.c_quat, f.sh, deg, x, dirs, site)
		np.testing.assert_allclose(c.cpu().numpy(), r, atol=1e-5)
	for floor in (0.0, 0.01):
		A = ext.conic(T(f.d_log_scale, gpu), T(f.d_quat, gpu), floor)
		np.testing.assert_allclose(A.cpu().numpy(), oracle.conic(f.d_log_scale, f.d_quat, floor), rtol=1e-5, atol=1e-3)
	empty = ext.density(g, T(f.raw, gpu), T(f.d_log_scale, gpu), T(f.d_quat, gpu), T(x[:0], gpu), T(site[:0], gpu))
	assert empty.shape == (0,)


def test_color_wide_batches(gpu):
	"""color_forward runs 4 lanes per sample below 2^22 samples and one lane per sample from there: a batch of
	1100 distinct samples repeated past 2^22 gives every copy the same colours (within 1e-6 of the small batch, whose
	lanes add their partial sums in another order) and the oracle's within 1e-5, with records and without."""
	f = Field(seed=6, n=300, lo=-1.0, hi=1.0, raw_mu=0.0, ls_mu=-1.2)
	rng = np.random.default_rng(10)
	n0 = 1100
	x = rng.uniform(-1, 1, (n0, 3)).astype(np.float32)
	site = f.tree.query(x)[1].astype(np.int32)
	dirs = rng.normal(size=(n0, 3)).astype(np.float32)
	reps = (1 << 22) // n0 + 1
	e = ext.extension()
	args = [T(a, gpu) for a in (f.points, f.offsets, f.adj)]
	for deg in (0, 3):
		r = oracle.color(f.points, f.offsets, f.adj, f.c_log_scale, f.c_quat, f.sh, deg, x, dirs, site)
		for rec in (True, False):
			call = lambda xs, ds, ss: e.color_forward(*args, T(f.c_log_scale, gpu), T(f.c_quat, gpu), T(f.sh, gpu),  # noqa: E731
													   deg, xs, ds, ss, records=rec)
			small = call(T(x, gpu), T(dirs, gpu), T(site, gpu)).cpu().numpy()
			big = call(T(x, gpu).repeat(reps, 1), T(dirs, gpu).repeat(reps, 1), T(site, gpu).repeat(reps))
			big = big.view(reps, n0, 3).cpu().numpy()
			assert big.shape[0] * n0 >= 1 << 22
			np.testing.assert_array_equal(big, np.broadcast_to(big[0], big.shape))
			np.testing.assert_allclose(big[0], small, atol=1e-6, rtol=0)
			np.testing.assert_allclose(big[0], r, atol=1e-5)


def test_density_color_records_bit_identical(gpu):
	"""density_forward / color_forward with per-site Gaussian records (a call of m >= N / 8 samples given scratch)
	and without (no scratch, or a call too small for them) give the same bits."""
	f = Field(seed=3, n=500, lo=-1.0, hi=1.0, raw_mu=0.5, ls_mu=-1.5)
	rng = np.random.default_rng(9)
	x = rng.uniform(-1, 1, (2000, 3)).astype(np.float32)
	site = f.tree.query(x)[1].astype(np.int32)
	dirs = rng.normal(size=(2000, 3)).astype(np.float32)
	e = ext.extension()
	args = [T(a, gpu) for a in (f.points, f.offsets, f.adj)]
	for mult in (1.0, 4.0):
		dens = [e.density_forward(*args, T(f.raw, gpu), T(f.d_log_scale, gpu), T(f.d_quat, gpu), T(x, gpu),
								  T(site, gpu), mult, records=rec).cpu().numpy() for rec in (True, False)]
		np.testing.assert_array_equal(dens[0], dens[1])
	for deg in (1, 3):
		col = [e.color_forward(*args, T(f.c_log_scale, gpu), T(f.c_quat, gpu), T(f.sh, gpu), deg, T(x, gpu),
							   T(dirs, gpu), T(site, gpu), records=rec).cpu().numpy() for rec in (True, False)]
		np.testing.assert_array_equal(col[0], col[1])
	# 40 samples over 500 sites: below N / 8, the direct kernel runs with or without scratch
	small = [e.density_forward(*args, T(f.raw, gpu), T(f.d_log_scale, gpu), T(f.d_quat, gpu), T(x[:40], gpu),
							   T(site[:40], gpu), 2.0, records=rec).cpu().numpy() for rec in (True, False)]
	np.testing.assert_array_equal(small[0], small[1])
	np.testing.assert_array_equal(small[0], e.density_forward(*args, T(f.raw, gpu), T(f.d_log_scale, gpu),
															  T(f.d_quat, gpu), T(x, gpu), T(site, gpu),
															  2.0).cpu().numpy()[:40])


def test_render_rays_nerf_path(gpu):
	"""render_rays (NeRF sampling + walk/density/color kernels) on GPU equals the same host code run on CPU with
	the oracle's operators."""
	f = Field(seed=4, n=300, raw_mu=1.0, ls_mu=-1.8)
	o, d, start, *_ = f.rays(B=128, seed=4)
	from types import SimpleNamespace
	import vgr.render as R

	def model_on(dev):
		t = lambda a: torch.as_tensor(a, device=dev)  # noqa: E731
		g = SimpleNamespace(points=t(f.points), offsets=t(f.offsets), adj=t(f.adj))
		return SimpleNamespace(graph=g, raw=t(f.raw), d_log_scale=t(f.d_log_scale), d_quat=t(f.d_quat),
							   c_log_scale=t(f.c_log_scale), c_quat=t(f.c_quat), sh=lambda: t(f.sh), sh_deg=3,
							   bg_logit=torch.zeros(3, device=dev))

	mg = model_on(gpu)
	mg.walk = lambda o_, d_, z, s: ext.Graph(mg.graph.points, mg.graph.offsets, mg.graph.adj).walk(o_, d_, z, s)
	out = R.render_rays(mg, T(o, gpu), T(d, gpu), T(start, gpu), perturb=False)

	mc = model_on('cpu')

	def cwalk(o_, d_, z, s):
		site, steps = oracle.walk(f.points, f.offsets, f.adj, o_.numpy(), d_.numpy(), z.numpy(), s.numpy())
		return torch.from_numpy(site), torch.from_numpy(steps)
	mc.walk = cwalk
	orig_density, orig_color = R.ext.density, R.ext.color
	try:
		R.ext.density = lambda g, raw, ls, q, x, site, mult=1.0: torch.from_numpy(
			oracle.density(f.points, f.offsets, f.adj, f.raw, f.d_log_scale, f.d_quat, x.numpy(), site.numpy(), mult))
		R.ext.color = lambda g, ls, q, sh, x, dirs, site, deg=3: torch.from_numpy(
			oracle.color(f.points, f.offsets, f.adj, f.c_log_scale, f.c_quat, f.sh, deg, x.numpy(), dirs.numpy(),
						 site.numpy()))
		ref = R.render_rays(mc, torch.from_numpy(o), torch.from_numpy(d), torch.from_numpy(start), perturb=False)
	finally:
		R.ext.density, R.ext.color = orig_density, orig_color
	np.testing.assert_allclose(out['rgb'].cpu().numpy(), ref['rgb'].numpy(), atol=1e-4)
	np.testing.assert_allclose(out['acc'].cpu().numpy(), ref['acc'].numpy(), atol=1e-4)
