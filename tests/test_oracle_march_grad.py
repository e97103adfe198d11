"""The oracle's march backward (vgr_oracle.c: oracle_march_backward, the restatement of march.cu:264-345) against
float64 PyTorch autograd of the march it differentiates: the samples of march_samples, the sites the oracle's own
forward visits (its trace), the density sum, the softmax-weighted max(SH + 1/2, 0) colours and NeRF compositing,
written densely over (sample, neighbour) pairs and differentiated by autograd. With thresholds off every sample is
coloured and none is cut; with the default thresholds the dense march stops where the oracle's forward stopped and
leaves uncoloured the samples whose weight is at most w_thresh, which is the function the reference's backward
differentiates."""

import numpy as np
import pytest
import torch

import dense
import oracle
from helpers import Field
from test_oracle_grad import rel

DT, NBG = 0.05, 8


def march64(f, o, d, bounds, cells, n_samples, w_thresh, params, sh_deg):
	"""rgb (B, 3) and final T (B,) in float64 from leaf tensors params = (raw, dA, cA, sh)."""
	raw, gdA, gcA, sh = params
	P = torch.from_numpy(f.points).double()
	b = torch.from_numpy(np.stack([oracle.sh_basis(v, sh_deg) for v in d]).astype(np.float64))
	rgb, T_out = [], []
	for r in range(len(o)):
		near, mid, far = bounds[r]
		t, delta = dense.march_samples(float(near), float(mid), float(far), DT, NBG)
		n = int(n_samples[r])
		t, delta = torch.from_numpy(t[:n]), torch.from_numpy(delta[:n])
		X = torch.from_numpy(o[r]).double()[None] + t[:, None] * torch.from_numpy(d[r]).double()[None]
		ps, pk = [], []
		for s, c in enumerate(cells[r][:n]):
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
		alpha = 1 - torch.exp(-sig * delta)
		trans = torch.cumprod(torch.cat([torch.ones(1, dtype=torch.float64), 1 - alpha]), 0)
		w = alpha * trans[:-1]
		on = (w > w_thresh).double().detach()
		rgb.append(((w * on)[:, None] * C).sum(0))
		T_out.append(trans[-1])
	return torch.stack(rgb), torch.stack(T_out)


@pytest.mark.parametrize('t_thresh,w_thresh', [(0.0, -1.0), (1e-4, 1e-4)])
@pytest.mark.parametrize('sh_deg', [3, 1])
def test_march_backward_matches_float64_autograd(oracle_lib, t_thresh, w_thresh, sh_deg):
	f = Field(seed=5, n=300, sh_deg=sh_deg)
	o, d, start, near, mid, far = f.rays(B=24, seed=5)
	dA, cA = f.conics(0.01)
	fw = oracle.march_forward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, sh_deg, o, d, start, near, mid, far,
							  DT, NBG, t_thresh, w_thresh, trace_cap=512)
	assert fw['stats'][:, 0].max() < 512
	rng = np.random.default_rng(9)
	g_rgb = rng.normal(size=(len(o), 3)).astype(np.float32)
	g_T = rng.normal(size=len(o)).astype(np.float32)
	got = oracle.march_backward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, sh_deg, o, d, start, near, mid, far,
								DT, NBG, fw['rgb'], fw['T'], g_rgb, g_T, t_thresh, w_thresh)

	params = [torch.from_numpy(x).double().requires_grad_() for x in (f.raw, dA, cA, f.sh)]
	rgb, T = march64(f, o, d, np.stack([near, mid, far], 1), fw['trace'], fw['stats'][:, 0], w_thresh, params,
					 sh_deg)
	assert rel(fw['rgb'], rgb.detach()) < 1e-5 and rel(fw['T'], T.detach()) < 1e-5
	((rgb * torch.from_numpy(g_rgb).double()).sum() + (T * torch.from_numpy(g_T).double()).sum()).backward()
	for name, g, p in zip(('raw', 'dA', 'cA', 'sh'), got, params):
		assert rel(g, p.grad) < 1e-4, name
	if sh_deg < 3:
		assert (got[3][:, (sh_deg + 1) ** 2:] == 0).all()
	assert np.abs(got[0]).max() > 0 and np.abs(got[3]).max() > 0


def test_march_backward_of_nothing_is_zero(oracle_lib):
	"""No upstream gradient, or rays that end before their first sample is coloured: zero gradients."""
	f = Field(seed=5, n=300)
	o, d, start, near, mid, far = f.rays(B=8, seed=5)
	dA, cA = f.conics(0.01)
	fw = oracle.march_forward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, o, d, start, near, mid, far, DT,
							  NBG)
	z3, z = np.zeros((8, 3), np.float32), np.zeros(8, np.float32)
	for g in oracle.march_backward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, o, d, start, near, mid, far,
								   DT, NBG, fw['rgb'], fw['T'], z3, z):
		assert not g.any()
