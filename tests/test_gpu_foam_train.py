"""GPU parity of the training renderer (vgr_foam_forward / vgr_foam_backward through the C ABI, and ext.foam's
autograd) against the C oracle's restatement of foam.cu:160-469 on identical inputs, the oracle being pinned by
the float64 re-trace and float64 autograd. Sites and sample positions are compared exactly; values within 1e-4
(the group sums are added in another order than the oracle's sequential ones); gradients, summed with fp32
atomics, to a relative error (vector norm) of 2e-5."""

import numpy as np
import pytest
import torch

import oracle
from helpers import Field
from test_oracle_grad import rel
from vgr import ext

pytestmark = pytest.mark.gpu


def T(a, dev):
	return torch.as_tensor(np.ascontiguousarray(a), device=dev)


def case(dev, sh_deg=3, B=160, seed=6):
	f = Field(seed=seed, n=300, sh_deg=sh_deg)
	o, d, start, near, _, far = f.rays(B=B, seed=seed)
	dA, cA = f.conics(0.01)
	field = [T(a, dev) for a in (f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh)]
	rays = (o, d, start, near, far)
	return f, dA, cA, field, rays, [T(a, dev) for a in rays]


@pytest.mark.parametrize('t_thresh,w_thresh', [(0.0, -1.0), (1e-4, 1e-4)])
@pytest.mark.parametrize('sh_deg', [3, 1])
def test_foam_forward_matches_oracle(gpu, sh_deg, t_thresh, w_thresh):
	f, dA, cA, field, rays, rt = case(gpu, sh_deg)
	fx = ext.foam_extension()
	rgb, Tt, depth, stats, rec = [x.cpu().numpy() for x in fx.foam_forward(*field, sh_deg, *rt, t_thresh, w_thresh,
																			 512)]
	ref = oracle.foam_forward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, sh_deg, *rays, t_thresh, w_thresh,
							  record_cap=512)
	assert stats[:, 0].max() < 512
	same = (stats == ref['stats']).all(1)
	assert same.mean() >= 0.98
	np.testing.assert_allclose(rgb, ref['rgb'], atol=1e-4)
	np.testing.assert_allclose(Tt, ref['T'], atol=1e-4)
	np.testing.assert_allclose(depth, ref['depth'], atol=1e-3)
	for r in np.nonzero(same)[0]:
		n = stats[r, 0]
		np.testing.assert_array_equal(rec[r, :n, :2], ref['rec'][r, :n, :2])  # t and site bits
		np.testing.assert_allclose(rec[r, :n, 2], ref['rec'][r, :n, 2], rtol=1e-4, atol=1e-5)  # sigma
		# colour, m_min and 1 / A of the samples whose colour was evaluated (the others record 1 / A = 0; their
		# m_min is not part of the record's meaning)
		has_c = ref['rec'][r, :n, 7] > 0
		np.testing.assert_array_equal(rec[r, :n, 7] > 0, has_c)
		np.testing.assert_allclose(rec[r, :n][has_c, 3:], ref['rec'][r, :n][has_c, 3:], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize('record_cap', [512, 4, 0])
@pytest.mark.parametrize('t_thresh,w_thresh', [(0.0, -1.0), (1e-4, 1e-4)])
def test_foam_backward_matches_oracle(gpu, record_cap, t_thresh, w_thresh):
	"""Records replayed (512), replayed for short rays and re-traced for the others (4), re-traced (0)."""
	f, dA, cA, field, rays, rt = case(gpu)
	fx = ext.foam_extension()
	rgb, Tt, _, stats, rec = fx.foam_forward(*field, 3, *rt, t_thresh, w_thresh, record_cap)
	rng = np.random.default_rng(12)
	g_rgb = rng.normal(size=(len(rays[0]), 3)).astype(np.float32)
	g_T = rng.normal(size=len(rays[0])).astype(np.float32)
	got = fx.foam_backward(*field, 3, *rt, t_thresh, w_thresh, rgb, Tt, T(g_rgb, gpu), T(g_T, gpu), rec, stats)
	ref = oracle.foam_backward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, *rays, rgb.cpu().numpy(),
							   Tt.cpu().numpy(), g_rgb, g_T, t_thresh, w_thresh)
	for name, a, r in zip(('raw', 'dA', 'cA', 'sh'), got, ref):
		assert rel(a.cpu().numpy(), r) < 2e-5, name


def test_foam_autograd_matches_oracle(gpu):
	"""ext.foam with gradients on, as train.py calls it through render_rays_foam (ext.py:185-216)."""
	f, dA, cA, field, rays, rt = case(gpu)
	graph = ext.Graph(*field[:3])
	params = [p.clone().requires_grad_() for p in field[3:]]
	rng = np.random.default_rng(13)
	g_rgb = rng.normal(size=(len(rays[0]), 3)).astype(np.float32)
	g_T = rng.normal(size=len(rays[0])).astype(np.float32)
	rgb, Tt, depth, stats = ext.foam(graph, *params, 3, *rt)
	assert not depth.requires_grad and stats.dtype == torch.int32
	((rgb * T(g_rgb, gpu)).sum() + (Tt * T(g_T, gpu)).sum()).backward()
	ref = oracle.foam_backward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, *rays,
							   rgb.detach().cpu().numpy(), Tt.detach().cpu().numpy(), g_rgb, g_T)
	for name, p, r in zip(('raw', 'dA', 'cA', 'sh'), params, ref):
		assert rel(p.grad.cpu().numpy(), r) < 2e-5, name
	with torch.no_grad():
		out = ext.foam(graph, *params, 3, *rt)
	assert torch.equal(out[0], rgb.detach()) and torch.equal(out[1], Tt.detach())


def test_foam_train_edge_cases(gpu):
	f, dA, cA, field, rays, rt = case(gpu, B=16)
	fx = ext.foam_extension()
	start = rt[2].clone()
	start[:4] = -1  # untraced rays: empty foreground, no samples, no gradient
	rays_u = rt[:2] + [start] + rt[3:]
	rgb, Tt, _, stats, rec = fx.foam_forward(*field, 3, *rays_u, 1e-4, 1e-4, 64)
	assert (rgb[:4] == 0).all() and (Tt[:4] == 1).all() and (stats[:4] == 0).all()
	ones3, ones = torch.ones(16, 3, device=gpu), torch.ones(16, device=gpu)
	sel = [x[:4].contiguous() for x in rays_u]
	got = fx.foam_backward(*field, 3, *sel, 1e-4, 1e-4, rgb[:4].contiguous(), Tt[:4].contiguous(), ones3[:4],
						   ones[:4], rec[:4].contiguous(), stats[:4].contiguous())
	assert all(not g.any() for g in got)
	e3, e = torch.empty(0, 3, device=gpu), torch.empty(0, device=gpu)
	ei = torch.empty(0, dtype=torch.int32, device=gpu)
	out = fx.foam_forward(*field, 3, e3, e3, ei, e, e, 1e-4, 1e-4, 8)
	assert out[0].shape == (0, 3) and out[4].shape == (0, 8, 8)
	got = fx.foam_backward(*field, 3, e3, e3, ei, e, e, 1e-4, 1e-4, e3, e, e3, e, torch.empty(0, 8, 8, device=gpu),
						   torch.empty(0, 3, dtype=torch.int32, device=gpu))
	assert all(not g.any() for g in got) and got[3].shape == (f.n, 16, 3)
	with pytest.raises(RuntimeError, match='sh_deg'):
		fx.foam_forward(*field, 4, *rt, 1e-4, 1e-4, 0)
	with pytest.raises(RuntimeError, match='rec must be'):
		fx.foam_backward(*field, 3, *rt, 1e-4, 1e-4, rgb, Tt, ones3, ones, rec[:3], stats)


def test_render_rays_foam_training_step(gpu):
	"""render.render_rays_foam (train.py's renderer, render.py:127-140) under autograd on the config-1 scene: the
	gradients of every field parameter (through ext.conic for the scales and rotations) against the oracle's
	backward chained with its conic backward, and the background's closed form."""
	from vgr import render, scenes
	from vgr.model import VoronoiGaussField
	sc = scenes.make_scene(1, img_scale=0.5, cache_dir=None, log=None)
	o, d, start, _ = sc.camera_rays(tile=8)
	o, d, start = o[::4].copy(), d[::4].copy(), start[::4].copy()
	model = VoronoiGaussField.from_scene(sc, gpu, requires_grad=True)
	W = np.random.default_rng(14).normal(size=(len(o), 3)).astype(np.float32)
	out = render.render_rays_foam(model, T(o, gpu), T(d, gpu), T(start, gpu))
	(out['rgb'] * T(W, gpu)).sum().backward()
	near, _, far = render.ray_bounds(T(o, gpu), T(d, gpu), 0.02, 4.0)
	near, far = near.cpu().numpy(), far.cpu().numpy()
	dA = oracle.conic(sc.log_scale, sc.quat, 0.0)
	fw = oracle.foam_forward(sc.points, sc.offsets, sc.adj, sc.raw, dA, dA, sc.sh, sc.sh_deg, o, d, start, near, far)
	np.testing.assert_allclose(out['rgb'].detach().cpu().numpy(), fw['rgb'] + 0.5 * fw['T'][:, None], atol=1e-4)
	g_T = (0.5 * W).sum(1)
	g_raw, g_dA, g_cA, g_sh = oracle.foam_backward(sc.points, sc.offsets, sc.adj, sc.raw, dA, dA, sc.sh, sc.sh_deg, o,
												   d, start, near, far, fw['rgb'], fw['T'], W, g_T)
	g_dls, g_dq = oracle.conic_backward(sc.log_scale, sc.quat, g_dA, 0.0)
	g_cls, g_cq = oracle.conic_backward(sc.log_scale, sc.quat, g_cA, 0.0)
	for name, p, r in (('raw', model.raw, g_raw), ('d_log_scale', model.d_log_scale, g_dls),
					   ('d_quat', model.d_quat, g_dq), ('c_log_scale', model.c_log_scale, g_cls),
					   ('c_quat', model.c_quat, g_cq), ('sh_dc', model.sh_dc, g_sh[:, :1])):
		assert rel(p.grad.cpu().numpy(), r) < 1e-4, name
	assert not model.sh_rest.grad.any()  # degree 0: no gradient beyond the DC term
	np.testing.assert_allclose(model.bg_logit.grad.cpu().numpy(), 0.25 * (fw['T'][:, None] * W).sum(0), rtol=1e-4,
							   atol=1e-4)


def test_backward_reuses_the_forward_blocks(gpu):
	"""A backward handed the forward's workspace (site blocks already packed: what the autograd Functions do) equals
	one that packs them again, for the training renderer and the march."""
	from vgr import _lib
	f, dA, cA, field, rays, rt = case(gpu)
	rng = np.random.default_rng(15)
	g_rgb = T(rng.normal(size=(len(rays[0]), 3)).astype(np.float32), gpu)
	g_T = T(rng.normal(size=len(rays[0])).astype(np.float32), gpu)
	fx = ext.foam_extension()
	work = torch.empty(int(_lib.load().vgr_foam_work_size(f.n, 3)), dtype=torch.uint8, device=gpu)
	rgb, Tt, _, stats, rec = fx.foam_forward(*field, 3, *rt, 1e-4, 1e-4, 64, work=work)
	a = fx.foam_backward(*field, 3, *rt, 1e-4, 1e-4, rgb, Tt, g_rgb, g_T, rec, stats, work=work)
	b = fx.foam_backward(*field, 3, *rt, 1e-4, 1e-4, rgb, Tt, g_rgb, g_T, rec, stats)
	for x, y in zip(a, b):
		assert rel(x.cpu().numpy(), y.cpu().numpy()) < 1e-6
	mx = ext.march_extension()
	mid = (rt[3] + rt[4]) * 0.5
	mrays = rt[:4] + [mid, rt[4]]
	work = torch.empty(int(_lib.load().vgr_march_backward_work_size(f.n, 3)), dtype=torch.uint8, device=gpu)
	rgb, Tt, _, _ = mx.march_forward(*field, 3, *mrays, 0.05, 8, 1e-4, 1e-4, work=work)
	a = mx.march_backward(*field, 3, *mrays, 0.05, 8, 1e-4, 1e-4, rgb, Tt, g_rgb, g_T, work=work)
	b = mx.march_backward(*field, 3, *mrays, 0.05, 8, 1e-4, 1e-4, rgb, Tt, g_rgb, g_T)
	for x, y in zip(a, b):
		assert rel(x.cpu().numpy(), y.cpu().numpy()) < 1e-6
	with pytest.raises(RuntimeError, match='too small'):
		mx.march_backward(*field, 3, *mrays, 0.05, 8, 1e-4, 1e-4, rgb, Tt, g_rgb, g_T, work=work[:100])
