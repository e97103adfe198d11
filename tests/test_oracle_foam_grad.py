"""The oracle's restatement of the training renderer (vgr_oracle.c: oracle_foam_forward / oracle_foam_backward,
foam.cu:160-469). The forward is pinned by the float64 bisector-plane re-trace of its cells (test_foam.py:18-37) and
by foam_infer's exact colours on the same rays (the same samples and trapezoid quadrature, restated separately);
the backward by float64 PyTorch autograd of the compositing it differentiates: the samples the oracle's forward
records (t, site), the density sum and softmax-weighted max(SH + 1/2, 0) colour at each, trapezoid segments, the
colour of segments of weight at most w_thresh left out, the ray cut where the forward stopped."""

import numpy as np
import pytest
import torch

import dense
import oracle
from helpers import Field
from test_oracle_grad import rel


def samples_of(rec, n):
	t = rec[:n, 0].astype(np.float64)
	site = rec[:n, 1].copy().view(np.int32)
	return t, site


def foam64(f, o, d, recs, stats, w_thresh, params, sh_deg):
	"""rgb (B, 3) and final T (B,) in float64 from leaf tensors params = (raw, dA, cA, sh)."""
	raw, gdA, gcA, sh = params
	P = torch.from_numpy(f.points).double()
	b = torch.from_numpy(np.stack([oracle.sh_basis(v, sh_deg) for v in d]).astype(np.float64))
	rgb, T_out = [], []
	for r in range(len(o)):
		n = int(stats[r, 0])
		t, site = samples_of(recs[r], n)
		t = torch.from_numpy(t)
		X = torch.from_numpy(o[r]).double()[None] + t[:, None] * torch.from_numpy(d[r]).double()[None]
		ps, pk = [], []
		for s, c in enumerate(site):
			nb = [int(c)] + [int(q) for q in f.adj[f.offsets[c]:f.offsets[c + 1]]]
			ps += [s] * len(nb)
			pk += nb
		ps, pk = torch.tensor(ps), torch.tensor(pk)
		v = X[ps] - P[pk]

		def maha(A):
			a = A[pk]
			return (a[:, 0] * v[:, 0] ** 2 + a[:, 3] * v[:, 1] ** 2 + a[:, 5] * v[:, 2] ** 2 +
					2 * (a[:, 1] * v[:, 0] * v[:, 1] + a[:, 2] * v[:, 0] * v[:, 2] + a[:, 4] * v[:, 1] * v[:, 2]))

		sig = torch.zeros(n, dtype=torch.float64).index_add(0, ps, torch.exp(raw[pk] - 0.5 * maha(gdA)))
		lc = -0.5 * maha(gcA)
		top = torch.full((n,), -np.inf, dtype=torch.float64).scatter_reduce(0, ps, lc.detach(), 'amax')
		a = torch.exp(lc - top[ps])
		A = torch.zeros(n, dtype=torch.float64).index_add(0, ps, a)
		col = (torch.einsum('j,kjc->kc', b[r], sh[pk]) + 0.5).clamp_min(0)
		C = torch.zeros(n, 3, dtype=torch.float64).index_add(0, ps, a[:, None] * col) / A[:, None]
		delta = t[1:] - t[:-1]
		alpha = 1 - torch.exp(-0.5 * (sig[:-1] + sig[1:]) * delta)
		trans = torch.cumprod(torch.cat([torch.ones(1, dtype=torch.float64), 1 - alpha]), 0)
		w = alpha * trans[:-1]
		on = (w > w_thresh).double().detach()
		rgb.append(((w * on)[:, None] * 0.5 * (C[:-1] + C[1:])).sum(0))
		T_out.append(trans[-1])
	return torch.stack(rgb), torch.stack(T_out)


@pytest.fixture(scope='module')
def foam_train_case():
	f = Field(seed=6, n=300)
	rays = f.rays(B=24, seed=6)
	dA, cA = f.conics(0.01)
	return f, rays, dA, cA


def test_foam_forward_cells_and_colours(oracle_lib, foam_train_case):
	"""Cells = the float64 re-trace on (almost) every ray; rgb and T = foam_infer's exact colours."""
	f, rays, dA, cA = foam_train_case
	o, d, start, near, _, far = rays
	fw = oracle.foam_forward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, o, d, start, near, far, 0.0, -1.0,
							 record_cap=4096)
	same = 0
	for r in range(len(o)):
		x0 = o[r].astype(np.float64) + near[r] * d[r].astype(np.float64)
		t64, cells = dense.trace(f.points, f.offsets, f.adj, o[r].astype(np.float64), d[r].astype(np.float64),
								 float(near[r]), float(far[r]), f.tree.query(x0)[1])
		n = fw['stats'][r, 0]
		t, site = samples_of(fw['rec'][r], n)
		# the cell of every sample: x(near), each crossing (the cell entered), x(far) (the last cell again)
		same += list(site) == list(cells) and np.abs(t - t64).max() < 1e-5
	assert same >= 0.95 * len(o), f'{same}/{len(o)}'
	pk = f.pack(floor=0.01)
	ref = oracle.foam_infer(pk, 3, o, d, start, near, far, t_thresh=0.0, w_thresh=-1.0, color_mode=0)
	assert rel(fw['rgb'], ref['rgb']) < 1e-5
	np.testing.assert_allclose(fw['T'], ref['T'], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize('t_thresh,w_thresh', [(0.0, -1.0), (1e-4, 1e-4)])
@pytest.mark.parametrize('sh_deg', [3, 1])
def test_foam_backward_matches_float64_autograd(oracle_lib, t_thresh, w_thresh, sh_deg):
	f = Field(seed=6, n=300, sh_deg=sh_deg)
	o, d, start, near, _, far = f.rays(B=24, seed=6)
	dA, cA = f.conics(0.01)
	fw = oracle.foam_forward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, sh_deg, o, d, start, near, far,
							 t_thresh, w_thresh, record_cap=4096)
	assert fw['stats'][:, 0].max() < 4096
	rng = np.random.default_rng(10)
	g_rgb = rng.normal(size=(len(o), 3)).astype(np.float32)
	g_T = rng.normal(size=len(o)).astype(np.float32)
	got = oracle.foam_backward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, sh_deg, o, d, start, near, far,
							   fw['rgb'], fw['T'], g_rgb, g_T, t_thresh, w_thresh)
	params = [torch.from_numpy(x).double().requires_grad_() for x in (f.raw, dA, cA, f.sh)]
	rgb, T = foam64(f, o, d, fw['rec'], fw['stats'], w_thresh, params, sh_deg)
	assert rel(fw['rgb'], rgb.detach()) < 1e-5 and rel(fw['T'], T.detach()) < 1e-5
	((rgb * torch.from_numpy(g_rgb).double()).sum() + (T * torch.from_numpy(g_T).double()).sum()).backward()
	for name, g, p in zip(('raw', 'dA', 'cA', 'sh'), got, params):
		assert rel(g, p.grad) < 1e-4, name
	assert np.abs(got[0]).max() > 0 and np.abs(got[3]).max() > 0
