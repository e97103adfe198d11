"""GPU parity of the march backward (vgr_march_backward through the C ABI, and ext.march's autograd) against the C
oracle's sequential restatement of march.cu:264-345 on identical inputs, the oracle being pinned by float64 autograd
of the dense march. The kernel sums each pass's samples per neighbour in registers and adds them with fp32 atomics,
so the sums agree to rounding, not bitwise: the bar is a relative error (vector norm) of 2e-5 per gradient."""

import numpy as np
import pytest
import torch

import oracle
from helpers import Field
from test_oracle_grad import rel
from vgr import ext

pytestmark = pytest.mark.gpu

DT, NBG = 0.05, 8


def T(a, dev):
	return torch.as_tensor(np.ascontiguousarray(a), device=dev)


def case(dev, sh_deg, t_thresh, w_thresh, B=192, seed=5, lanes=0):
	f = Field(seed=seed, n=300, sh_deg=sh_deg)
	rays = f.rays(B=B, seed=seed)
	dA, cA = f.conics(0.01)
	fx = ext.march_extension()
	field = [T(a, dev) for a in (f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh)]
	rt = [T(a, dev) for a in rays]
	rgb, Tt, _, _ = fx.march_forward(*field, sh_deg, *rt, DT, NBG, t_thresh, w_thresh, lanes=lanes)
	return f, rays, dA, cA, fx, field, rt, rgb, Tt


@pytest.mark.parametrize('lanes', [1, 16])
@pytest.mark.parametrize('t_thresh,w_thresh', [(0.0, -1.0), (1e-4, 1e-4)])
@pytest.mark.parametrize('sh_deg', [3, 2, 0])
def test_march_backward_matches_oracle(gpu, sh_deg, t_thresh, w_thresh, lanes):
	"""Both ray layouts (one ray per lane; 16 lanes per ray, one neighbour per lane), each replaying its own forward."""
	f, rays, dA, cA, fx, field, rt, rgb, Tt = case(gpu, sh_deg, t_thresh, w_thresh, lanes=lanes)
	rng = np.random.default_rng(3)
	g_rgb = rng.normal(size=(len(rays[0]), 3)).astype(np.float32)
	g_T = rng.normal(size=len(rays[0])).astype(np.float32)
	g_rgb[:7] = 0  # rays without an upstream colour gradient still pass dL/dT
	got = fx.march_backward(*field, sh_deg, *rt, DT, NBG, t_thresh, w_thresh, rgb, Tt, T(g_rgb, gpu), T(g_T, gpu),
							lanes=lanes)
	ref = oracle.march_backward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, sh_deg, *rays, DT, NBG,
								rgb.cpu().numpy(), Tt.cpu().numpy(), g_rgb, g_T, t_thresh, w_thresh)
	for name, a, r in zip(('raw', 'dA', 'cA', 'sh'), got, ref):
		assert rel(a.cpu().numpy(), r) < 2e-5, name
	assert (got[3][:, (sh_deg + 1) ** 2:] == 0).all()


def test_march_backward_wave_atomics_match_oracle(gpu):
	"""16,384 rays, where the launch shares each row of atomics across the wave: against the oracle, and against the
	per-lane atomics of the same rays in two launches of 8,192 (whose gradients add)."""
	B = 16384
	f, rays, dA, cA, fx, field, rt, rgb, Tt = case(gpu, 3, 1e-4, 1e-4, B=B, lanes=1)
	rng = np.random.default_rng(8)
	g_rgb = T(rng.normal(size=(B, 3)).astype(np.float32), gpu)
	g_T = T(rng.normal(size=B).astype(np.float32), gpu)
	got = fx.march_backward(*field, 3, *rt, DT, NBG, 1e-4, 1e-4, rgb, Tt, g_rgb, g_T, lanes=1)
	ref = oracle.march_backward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, *rays, DT, NBG, rgb.cpu().numpy(),
								Tt.cpu().numpy(), g_rgb.cpu().numpy(), g_T.cpu().numpy())
	for name, a, r in zip(('raw', 'dA', 'cA', 'sh'), got, ref):
		assert rel(a.cpu().numpy(), r) < 2e-5, name
	halves = [fx.march_backward(*field, 3, *[x[s].contiguous() for x in rt], DT, NBG, 1e-4, 1e-4, rgb[s].contiguous(),
								Tt[s].contiguous(), g_rgb[s].contiguous(), g_T[s].contiguous(), lanes=1)
			  for s in (slice(0, B // 2), slice(B // 2, None))]
	for name, a, h0, h1 in zip(('raw', 'dA', 'cA', 'sh'), got, *halves):
		assert rel((h0 + h1).cpu().numpy(), a.cpu().numpy()) < 1e-5, name


def test_march_autograd_matches_oracle(gpu):
	"""ext.march with gradients on, as training calls it (ext.py:150-182): loss = <rgb, g_rgb> + <T, g_T>."""
	f, rays, dA, cA, fx, field, rt, rgb0, T0 = case(gpu, 3, 1e-4, 1e-4)
	graph = ext.Graph(*field[:3])
	params = [p.clone().requires_grad_() for p in field[3:]]
	rng = np.random.default_rng(4)
	g_rgb = rng.normal(size=(len(rays[0]), 3)).astype(np.float32)
	g_T = rng.normal(size=len(rays[0])).astype(np.float32)
	rgb, Tt, depth, stats = ext.march(graph, *params, 3, *rt, DT, NBG)
	assert torch.equal(rgb.detach(), rgb0) and torch.equal(Tt.detach(), T0)
	assert not depth.requires_grad and stats.dtype == torch.int32
	((rgb * T(g_rgb, gpu)).sum() + (Tt * T(g_T, gpu)).sum()).backward()
	ref = oracle.march_backward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, *rays, DT, NBG,
								rgb0.cpu().numpy(), T0.cpu().numpy(), g_rgb, g_T)
	for name, p, r in zip(('raw', 'dA', 'cA', 'sh'), params, ref):
		assert rel(p.grad.cpu().numpy(), r) < 2e-5, name
	# a loss on T alone: autograd hands no colour gradient, which counts as zero
	params = [p.clone().requires_grad_() for p in field[3:]]
	_, Tt, _, _ = ext.march(graph, *params, 3, *rt, DT, NBG)
	Tt.sum().backward()
	ref = oracle.march_backward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, *rays, DT, NBG,
								rgb0.cpu().numpy(), T0.cpu().numpy(), np.zeros((len(rays[0]), 3), np.float32),
								np.ones(len(rays[0]), np.float32))
	assert rel(params[0].grad.cpu().numpy(), ref[0]) < 2e-5
	assert not params[3].grad.any()


def test_march_backward_edge_cases(gpu):
	f, rays, dA, cA, fx, field, rt, rgb, Tt = case(gpu, 3, 1e-4, 1e-4, B=16)
	ones3, ones = torch.ones(16, 3, device=gpu), torch.ones(16, device=gpu)
	# untraced rays (start -1) have no samples and take no gradient
	start = rt[2].clone().fill_(-1)
	rays_u = rt[:2] + [start] + rt[3:]
	got = fx.march_backward(*field, 3, *rays_u, DT, NBG, 1e-4, 1e-4, rgb, Tt, ones3, ones)
	assert all(not g.any() for g in got)
	# no rays: zeroed gradients of the field's shapes
	e3, e = torch.empty(0, 3, device=gpu), torch.empty(0, device=gpu)
	got = fx.march_backward(*field, 3, e3, e3, torch.empty(0, dtype=torch.int32, device=gpu), e, e, e, DT, NBG, 1e-4,
							1e-4, e3, e, e3, e)
	assert [tuple(g.shape) for g in got] == [(f.n,), (f.n, 6), (f.n, 6), (f.n, 16, 3)]
	assert all(not g.any() for g in got)
	with pytest.raises(RuntimeError, match='sh_deg'):
		fx.march_backward(*field, 4, *rt, DT, NBG, 1e-4, 1e-4, rgb, Tt, ones3, ones)
	with pytest.raises(RuntimeError, match='g_rgb'):
		fx.march_backward(*field, 3, *rt, DT, NBG, 1e-4, 1e-4, rgb, Tt, ones3[:3], ones)
