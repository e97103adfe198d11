"""GPU parity of the backward field operators (vgr_density_backward, vgr_color_backward, vgr_conic_backward through
the C ABI): against the C oracle's sequential sums on identical inputs, and end to end through ext.density /
ext.color / ext.conic autograd against float64 PyTorch autograd of the dense fields, the check of the reference's
test_grad.py:88-114. The kernels scatter with fp32 atomics (and gather dL/dsh per site in another order), so sums
agree to rounding, not bitwise: the bar is a relative error (vector norm) of 1e-5 against the oracle and 1e-4 against
float64."""

import numpy as np
import pytest
import torch

import oracle
from helpers import Field
from test_oracle_grad import mask_of, maha64, quat_rot, rel, sh_basis64
from vgr import ext

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def case(gpu):
	f = Field(seed=3, n=400)
	rng = np.random.default_rng(11)
	m = 3000
	x = rng.uniform(-0.85, 0.85, (m, 3)).astype(np.float32)
	site = f.tree.query(x)[1].astype(np.int32)
	site[:5] = -1  # unresolved samples: no value, no gradient
	dirs = rng.normal(size=(m, 3)).astype(np.float32)
	T = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=gpu)  # noqa: E731
	graph = ext.Graph(T(f.points), T(f.offsets), T(f.adj))
	return f, x, site, dirs, rng, T, graph


@pytest.mark.parametrize('gather', [True, False])
def test_density_backward_matches_oracle(case, gather):
	"""Gradients gathered per site (counting sort of the samples by site) and scattered with atomics."""
	f, x, site, _, rng, T, graph = case
	g_sigma = rng.normal(size=len(x)).astype(np.float32)
	g_sigma[10:20] = 0
	out = ext.extension().density_backward(graph.points, graph.offsets, graph.adj, T(f.raw), T(f.d_log_scale),
										   T(f.d_quat), T(x), T(site), T(g_sigma), gather=gather)
	ok = site >= 0
	ref = oracle.density_backward(f.points, f.offsets, f.adj, f.raw, f.d_log_scale, f.d_quat, x[ok], site[ok],
								  g_sigma[ok])
	for a, r in zip(out, ref):
		assert rel(a.cpu().numpy(), r) < 1e-5


@pytest.mark.parametrize('gather', [True, False])
@pytest.mark.parametrize('sh_deg', [3, 2, 0])
def test_color_backward_matches_oracle(case, sh_deg, gather):
	"""Gradients gathered per site through the workspace (counting sort of the samples by site) and scattered with
	atomics: both against the oracle."""
	f, x, site, dirs, rng, T, graph = case
	sh = f.sh.copy()
	sh[:, (sh_deg + 1) ** 2:] = 0
	g_rgb = rng.normal(size=(len(x), 3)).astype(np.float32)
	fx = ext.extension()
	rgb = fx.color_forward(graph.points, graph.offsets, graph.adj, T(f.c_log_scale), T(f.c_quat), T(sh), sh_deg, T(x),
						   T(dirs), T(site))
	g_rgb[20:40] = 0  # samples without an upstream gradient take no record slot
	out = fx.color_backward(graph.points, graph.offsets, graph.adj, T(f.c_log_scale), T(f.c_quat), T(sh), sh_deg,
							T(x), T(dirs), T(site), rgb, T(g_rgb), gather=gather)
	ok = site >= 0
	ref = oracle.color_backward(f.points, f.offsets, f.adj, f.c_log_scale, f.c_quat, sh, sh_deg, x[ok], dirs[ok],
								site[ok], rgb.cpu().numpy()[ok], g_rgb[ok])
	for a, r in zip(out, ref):
		assert rel(a.cpu().numpy(), r) < 1e-5
	assert (out[2][:, (sh_deg + 1) ** 2:] == 0).all()


@pytest.mark.parametrize('floor', [0.0, 0.05])
def test_conic_backward_matches_oracle(case, floor):
	f, _, _, _, rng, T, _ = case
	gA = rng.normal(size=(f.n, 6)).astype(np.float32)
	g_ls, g_quat = ext.extension().conic_backward(T(f.d_log_scale), T(f.d_quat), floor, T(gA))
	r_ls, r_quat = oracle.conic_backward(f.d_log_scale, f.d_quat, gA, floor)
	assert rel(g_ls.cpu().numpy(), r_ls) < 1e-5
	assert rel(g_quat.cpu().numpy(), r_quat) < 1e-5


def test_autograd_end_to_end_matches_float64(case, gpu):
	"""ext.density and ext.color with gradients on, as training calls them (test_grad.py:84-114)."""
	f, x, site, dirs, rng, T, graph = case
	ok = site >= 0
	x, site, dirs = x[ok], site[ok], dirs[ok]
	params = [T(a).requires_grad_() for a in (f.raw, f.d_log_scale, f.d_quat, f.c_log_scale, f.c_quat, f.sh)]
	raw, ls, q, cls, cq, sh = params
	g_sigma = rng.normal(size=len(x)).astype(np.float32)
	g_rgb = rng.normal(size=(len(x), 3)).astype(np.float32)
	sigma = ext.density(graph, raw, ls, q, T(x), T(site))
	rgb = ext.color(graph, cls, cq, sh, T(x), T(dirs), T(site), 3)
	((sigma * T(g_sigma)).sum() + (rgb * T(g_rgb)).sum()).backward()

	ref = [torch.from_numpy(a).double().requires_grad_() for a in (f.raw, f.d_log_scale, f.d_quat, f.c_log_scale,
																   f.c_quat, f.sh)]
	rraw, rls, rq, rcls, rcq, rsh = ref
	P, X = torch.from_numpy(f.points).double(), torch.from_numpy(x).double()
	mask = mask_of(f, site)
	sigma64 = (torch.exp(rraw)[None] * torch.exp(-0.5 * maha64(P, rls, rq, X)) * mask).sum(1)
	a = torch.softmax(-0.5 * maha64(P, rcls, rcq, X).masked_fill(~mask, float('inf')), 1)
	D = torch.nn.functional.normalize(torch.from_numpy(dirs).double(), dim=-1)
	ck = (torch.einsum('mj,njc->mnc', sh_basis64(D.float()), rsh) + 0.5).clamp_min(0)
	rgb64 = (a[..., None] * ck).sum(1)
	((sigma64 * torch.from_numpy(g_sigma).double()).sum() + (rgb64 * torch.from_numpy(g_rgb).double()).sum()).backward()
	assert rel(sigma.detach().cpu(), sigma64.detach()) < 1e-5
	assert rel(rgb.detach().cpu(), rgb64.detach()) < 1e-5
	for p, r in zip(params, ref):
		assert rel(p.grad.cpu(), r.grad) < 1e-4


def test_conic_autograd_matches_float64(case, gpu):
	f, _, _, _, rng, T, _ = case
	ls, q = T(f.d_log_scale).requires_grad_(), T(f.d_quat).requires_grad_()
	gA = rng.normal(size=(f.n, 6)).astype(np.float32)
	(ext.conic(ls, q, 0.05) * T(gA)).sum().backward()
	rls, rq = (torch.from_numpy(a).double().requires_grad_() for a in (f.d_log_scale, f.d_quat))
	(ext.conic_reference(rls, rq, 0.05) * torch.from_numpy(gA).double()).sum().backward()
	assert rel(ls.grad.cpu(), rls.grad) < 1e-4
	assert rel(q.grad.cpu(), rq.grad) < 1e-4
	assert quat_rot(rq).shape == (f.n, 3, 3)


def test_backward_edge_cases(case, gpu):
	f, x, site, dirs, _, T, graph = case
	fx = ext.extension()
	empty_f, empty_i = torch.empty(0, 3, device=gpu), torch.empty(0, dtype=torch.int32, device=gpu)
	g = fx.density_backward(graph.points, graph.offsets, graph.adj, T(f.raw), T(f.d_log_scale), T(f.d_quat), empty_f,
							empty_i, torch.empty(0, device=gpu))
	assert all((a == 0).all() for a in g)
	# unresolved samples and zero upstream gradients contribute nothing
	g = fx.density_backward(graph.points, graph.offsets, graph.adj, T(f.raw), T(f.d_log_scale), T(f.d_quat),
							T(x[:5]), T(site[:5]), torch.ones(5, device=gpu))
	assert (site[:5] == -1).all() and all((a == 0).all() for a in g)
	g = fx.color_backward(graph.points, graph.offsets, graph.adj, T(f.c_log_scale), T(f.c_quat), T(f.sh), 3, T(x),
						  T(dirs), T(site), torch.zeros(len(x), 3, device=gpu), torch.zeros(len(x), 3, device=gpu))
	assert all((a == 0).all() for a in g)
	with pytest.raises(RuntimeError, match='sh_deg'):
		fx.color_backward(graph.points, graph.offsets, graph.adj, T(f.c_log_scale), T(f.c_quat), T(f.sh), 4, T(x),
						  T(dirs), T(site), torch.zeros(len(x), 3, device=gpu), torch.ones(len(x), 3, device=gpu))
	# no gradient requested: the forward alone, no autograd node
	with torch.no_grad():
		s = ext.density(graph, T(f.raw).requires_grad_(), T(f.d_log_scale), T(f.d_quat), T(x), T(site))
	assert s.grad_fn is None
