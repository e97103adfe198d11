"""The oracle's backward field operators (vgr_oracle.c: oracle_density_backward, oracle_color_backward,
oracle_conic_backward) against float64 PyTorch autograd of the forward fields, the check the reference's own
test_grad.py:88-114 makes for its kernels: sigma = sum over {site} U adj(site) of exp(raw) G, rgb = softmax-weighted
max(SH + 1/2, 0), A = R diag(1 / (s^2 + floor^2)) R^T, each written densely with a neighbourhood mask and
differentiated by autograd -- an independent derivation of the closed forms the oracle restates (vgf.cu:121-148,
179-198, 284-333, 382-424)."""

import numpy as np
import pytest
import torch

import oracle
from helpers import Field

REL = 2e-5  # relative error (norm) of the fp32 oracle gradients against float64 autograd


def quat_rot(q):
	q = q / q.norm(dim=-1, keepdim=True).clamp_min(1e-12)
	w, x, y, z = q.unbind(-1)
	return torch.stack([
		1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
		2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
		2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1).view(*q.shape[:-1], 3, 3)


def sh_basis64(d):
	return torch.from_numpy(np.stack([oracle.sh_basis(v, 3) for v in d.numpy()]).astype(np.float64))


def mask_of(f, site):
	m = torch.zeros(len(site), f.n, dtype=torch.bool)
	for r, i in enumerate(site):
		m[r, i] = True
		m[r, f.adj[f.offsets[i]:f.offsets[i + 1]]] = True
	return m


def maha64(points, log_scale, quat, x):
	y = torch.einsum('nab,mna->mnb', quat_rot(quat), x[:, None] - points[None])
	return (y * y / torch.exp(2 * log_scale.clamp(-20, 20))[None]).sum(-1)


def rel(a, b):
	b = torch.as_tensor(b, dtype=torch.float64)
	return float((torch.as_tensor(a, dtype=torch.float64) - b).norm() / b.norm().clamp_min(1e-30))


@pytest.fixture(scope='module')
def case():
	f = Field(seed=5, n=200)
	rng = np.random.default_rng(7)
	x = rng.uniform(-0.8, 0.8, (500, 3)).astype(np.float32)
	site = f.tree.query(x)[1].astype(np.int32)
	dirs = rng.normal(size=(500, 3)).astype(np.float32)
	return f, x, site, dirs, rng


def test_density_backward_matches_autograd(case):
	f, x, site, _, rng = case
	g_sigma = rng.normal(size=len(x)).astype(np.float32)
	g_raw, g_ls, g_quat = oracle.density_backward(f.points, f.offsets, f.adj, f.raw, f.d_log_scale, f.d_quat, x, site,
												  g_sigma)
	P, X = torch.from_numpy(f.points).double(), torch.from_numpy(x).double()
	raw, ls, q = (torch.from_numpy(a).double().requires_grad_() for a in (f.raw, f.d_log_scale, f.d_quat))
	sigma = (torch.exp(raw)[None] * torch.exp(-0.5 * maha64(P, ls, q, X)) * mask_of(f, site)).sum(1)
	(sigma * torch.from_numpy(g_sigma).double()).sum().backward()
	assert rel(g_raw, raw.grad) < REL
	assert rel(g_ls, ls.grad) < REL
	assert rel(g_quat, q.grad) < REL
	# the gradient only reaches the sites of the sampled neighbourhoods
	touched = mask_of(f, site).any(0).numpy()
	assert (g_raw[~touched] == 0).all() and (g_raw[touched] != 0).any()


@pytest.mark.parametrize('sh_deg', [3, 1])
def test_color_backward_matches_autograd(case, sh_deg):
	f, x, site, dirs, rng = case
	sh = f.sh.copy()
	sh[:, (sh_deg + 1) ** 2:] = 0
	g_rgb = rng.normal(size=(len(x), 3)).astype(np.float32)
	rgb = oracle.color(f.points, f.offsets, f.adj, f.c_log_scale, f.c_quat, sh, sh_deg, x, dirs, site)
	g_ls, g_quat, g_sh = oracle.color_backward(f.points, f.offsets, f.adj, f.c_log_scale, f.c_quat, sh, sh_deg, x,
											   dirs, site, rgb, g_rgb)
	P, X = torch.from_numpy(f.points).double(), torch.from_numpy(x).double()
	ls, q, S = (torch.from_numpy(a).double().requires_grad_() for a in (f.c_log_scale, f.c_quat, sh))
	a = torch.softmax(-0.5 * maha64(P, ls, q, X).masked_fill(~mask_of(f, site), float('inf')), 1)
	D = torch.nn.functional.normalize(torch.from_numpy(dirs).double(), dim=-1)
	B = sh_basis64(D.float())
	B[:, (sh_deg + 1) ** 2:] = 0
	ck = (torch.einsum('mj,njc->mnc', B, S) + 0.5).clamp_min(0)
	rgb64 = (a[..., None] * ck).sum(1)
	assert rel(rgb, rgb64.detach()) < 1e-5
	(rgb64 * torch.from_numpy(g_rgb).double()).sum().backward()
	assert rel(g_ls, ls.grad) < REL
	assert rel(g_quat, q.grad) < REL
	assert rel(g_sh, S.grad) < REL
	assert (g_sh[:, (sh_deg + 1) ** 2:] == 0).all()  # coefficients beyond the degree get nothing


@pytest.mark.parametrize('floor', [0.0, 0.05])
def test_conic_backward_matches_autograd(case, floor):
	f, _, _, _, rng = case
	gA = rng.normal(size=(f.n, 6)).astype(np.float32)
	g_ls, g_quat = oracle.conic_backward(f.d_log_scale, f.d_quat, gA, floor)
	ls, q = (torch.from_numpy(a).double().requires_grad_() for a in (f.d_log_scale, f.d_quat))
	R = quat_rot(q)
	iv = 1.0 / (torch.exp(2 * ls.clamp(-20, 20)) + floor * floor)
	A = torch.einsum('nak,nk,nbk->nab', R, iv, R)
	A6 = torch.stack([A[:, 0, 0], A[:, 0, 1], A[:, 0, 2], A[:, 1, 1], A[:, 1, 2], A[:, 2, 2]], -1)
	assert rel(oracle.conic(f.d_log_scale, f.d_quat, floor), A6.detach()) < 1e-6
	(A6 * torch.from_numpy(gA).double()).sum().backward()
	assert rel(g_ls, ls.grad) < REL
	assert rel(g_quat, q.grad) < REL


def test_gradient_checks_catch_a_planted_error(case):
	"""A mistake of the kind these checks exist for: a quaternion gradient that keeps a radial part (the tangent
	projection left out; a rotation does not depend on |q|, so the true gradient has none). 10 % of the gradient's
	norm along q is far outside the bound, so the autograd comparison pins the projection."""
	f, _, _, _, rng = case
	gA = rng.normal(size=(f.n, 6)).astype(np.float32)
	_, g_quat = oracle.conic_backward(f.d_log_scale, f.d_quat, gA)
	ls, q = (torch.from_numpy(a).double().requires_grad_() for a in (f.d_log_scale, f.d_quat))
	R = quat_rot(q)
	A = torch.einsum('nak,nk,nbk->nab', R, 1.0 / torch.exp(2 * ls), R)
	A6 = torch.stack([A[:, 0, 0], A[:, 0, 1], A[:, 0, 2], A[:, 1, 1], A[:, 1, 2], A[:, 2, 2]], -1)
	(A6 * torch.from_numpy(gA).double()).sum().backward()
	assert rel(g_quat, q.grad) < REL
	g = torch.from_numpy(g_quat).double()
	qn = q.detach() / q.detach().norm(dim=-1, keepdim=True)
	assert (g * qn).sum(-1).abs().max() < 1e-4 * g.norm(dim=-1).max()  # no radial part
	planted = g + 0.1 * g.norm(dim=-1, keepdim=True) * qn
	assert rel(planted, q.grad) > 10 * REL
