"""The native pack (vgr_pack_foam, through render.pack_foam) against the torch pack (render.pack_foam_arrays, the
restatement of render.py:179-225 that the host tests pin) on the same device tensors, with and without the Z-order
renumbering, the density cut-off, fp16 SH and a scale floor: every copied field bit for bit; the half2 cut-off
words, which go through exp (the device expf here, torch's exp kernel there; they differ by an ulp on a few
inputs), within one half-ulp on each half and equal on all but a few edges; and the renderer's output from the two
packs identical."""

import math

import numpy as np
import pytest
import torch

from vgr import ext, render, scenes
from vgr.model import VoronoiGaussField

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def model(gpu):
	sc = scenes.make_scene(1, cache_dir=None, log=None)
	return sc, VoronoiGaussField.from_scene(sc, gpu)


def torch_pack(model, scale_floor, eps_density, sh_half, reorder):
	g = model.graph
	dA = ext.conic(model.d_log_scale, model.d_quat, scale_floor)
	cA = ext.conic(model.c_log_scale, model.c_quat, scale_floor)
	return render.pack_foam_arrays(g.points, g.offsets, g.adj, model.raw.detach(), model.d_log_scale.detach(),
								   model.c_log_scale.detach(), dA, cA, model.sh().detach(), scale_floor, eps_density,
								   sh_half, reorder)


@pytest.mark.parametrize('reorder', [False, True])
@pytest.mark.parametrize('scale_floor,eps_density,sh_half', [(0.0, 0.0, False), (0.01, 1e-3, True),
															 (0.0, 1e-4, False)])
def test_native_pack_matches_torch_pack(model, reorder, scale_floor, eps_density, sh_half):
	sc, m = model
	a = render.pack_foam(m, scale_floor, eps_density, sh_half, reorder, index=False)
	b = torch_pack(m, scale_floor, eps_density, sh_half, reorder)
	for k in ('points', 'offsets', 'nbr', 'edge', 'attr', 'sh', 'sh32', 'orig'):
		assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape, k
	for k in ('points', 'offsets', 'nbr', 'attr', 'sh', 'sh32', 'orig'):
		assert torch.equal(a[k].view(torch.uint8) if a[k].dtype == torch.float16 else a[k],
						   b[k].view(torch.uint8) if b[k].dtype == torch.float16 else b[k]), k
	assert torch.equal(a['edge'][:, :3], b['edge'][:, :3])
	wa = a['edge'][:, 3].contiguous().view(torch.int32)
	wb = b['edge'][:, 3].contiguous().view(torch.int32)
	for shift in (0, 16):  # r2 (low half), lam (high half): half bit patterns of positive values, so ulps apart
		ha, hb = (wa >> shift) & 0xffff, (wb >> shift) & 0xffff
		assert (ha - hb).abs().max() <= 1
	assert (wa != wb).double().mean() < 1e-3
	if reorder:
		assert torch.equal(a['perm'], b['perm']) and torch.equal(a['inv'], b['inv'])
	else:
		assert a['perm'] is None and a['inv'] is None
	# the cut-off words are real: finite r2 when eps_density > 0, lam > 0 everywhere
	cut = a['edge'][:, 3].contiguous().view(torch.int32)
	r2 = (cut & 0xffff).to(torch.int16).view(torch.float16).float()
	lam = (cut >> 16).to(torch.int16).view(torch.float16).float()
	assert (lam > 0).all()
	assert torch.isinf(r2).all() if eps_density == 0 else torch.isfinite(r2).any()


def test_native_pack_renders_the_same(model, gpu):
	sc, m = model
	o_np, d_np, start_np, _ = sc.camera_rays(tile=8)
	o, d = torch.from_numpy(o_np).to(gpu), torch.from_numpy(d_np).to(gpu)
	a = render.pack_foam(m, reorder=True)
	b = torch_pack(m, 0.0, 0.0, False, True)
	st = a['inv'][torch.from_numpy(start_np).to(gpu).long()].int()
	near, _, far = render.ray_bounds(o, d, 0.02, sc.far_radius)
	empty = torch.empty(0, dtype=torch.int32, device=gpu)
	fi = ext.foam_infer_extension()
	outs = [fi.foam_infer(p['points'], p['offsets'], p['nbr'], p['edge'], p['attr'], p['sh'], sc.sh_deg, o, d, st,
						  near, far, 1e-4, 1e-4, math.inf, 2, 2, empty, p['orig']) for p in (a, b)]
	for x, y in zip(*outs):
		assert torch.equal(x, y)


@pytest.mark.parametrize('bits', [10, 4])
def test_native_morton_codes_match_torch(model, gpu, bits):
	"""vgr_morton_codes against the torch arithmetic of morton_order on the same device points (and on points
	with a flat axis, where the extent floor applies)."""
	sc, m = model
	for pts in (m.graph.points, torch.cat([m.graph.points[:, :2], torch.zeros_like(m.graph.points[:, :1])], 1)):
		pts = pts.contiguous()
		lo, hi = pts.amin(0), pts.amax(0)
		q = ((pts - lo) / (hi - lo).clamp_min(1e-12) * (2 ** bits - 1)).long()
		code = torch.zeros(len(pts), dtype=torch.long, device=gpu)
		for b in range(bits):
			for a in range(3):
				code |= ((q[:, a] >> b) & 1) << (3 * b + a)
		assert torch.equal(ext.morton_codes(pts, bits), code)
	assert ext.morton_codes(torch.zeros(0, 3, device=gpu)).numel() == 0


@pytest.mark.parametrize('deg', [3, 2, 1, 0])
def test_native_bake_matches_float64(model, gpu, deg):
	"""vgr_bake_colors (the baking step of render.py:228-235) on a packed, renumbered scene against the same colours in
	float64 from the packed positions and SH rows; attr's other columns untouched; a camera centre on a site gives
	that site the degree-0 colour, and degree 0 gives max(Y00 sh_0 + 1/2, 0) everywhere, whatever the view."""
	sc, m = model
	pk = render.pack_foam(m, reorder=True)
	for on_site, center in ((False, torch.tensor(sc.cameras[0].eye, dtype=torch.float32, device=gpu)),
							(True, pk['points'][7, :3].clone())):
		attr = pk['attr'].clone()
		ext.bake_colors(pk['points'], pk['sh32'], deg, center, attr)
		assert torch.equal(attr[:, :16], pk['attr'][:, :16]) and torch.equal(attr[:, 19:], pk['attr'][:, 19:])
		p, sh = pk['points'][:, :3].double(), pk['sh32'].double()
		v = p - center.double()
		dirs = v / v.norm(dim=1, keepdim=True).clamp_min(1e-12)
		ref = (render.sh_basis(dirs, deg)[:, :, None] * sh).sum(1).add(0.5).clamp_min(0)
		assert (attr[:, 16:19].double() - ref).abs().max() < 2e-6
		y00 = (0.28209479177387814 * sh[:, 0] + 0.5).clamp_min(0)
		if on_site:
			assert (attr[7, 16:19].double() - y00[7]).abs().max() < 1e-6
		if deg == 0:
			assert (attr[:, 16:19].double() - y00).abs().max() < 1e-6
	ext.bake_colors(pk['points'][:0], pk['sh32'][:0], deg, center, pk['attr'][:0])


def test_native_pack_errors(gpu):
	pts = torch.zeros(4, 3, device=gpu)
	with pytest.raises(RuntimeError, match='float32|CUDA|sh must'):
		ext.pack_foam(pts, torch.zeros(5, dtype=torch.int32, device=gpu), torch.zeros(0, dtype=torch.int32, device=gpu),
					  torch.zeros(4, device=gpu), torch.zeros(4, 3, device=gpu), torch.zeros(4, 3, device=gpu),
					  torch.zeros(4, 6, device=gpu), torch.zeros(4, 6, device=gpu), torch.zeros(4, 9, 3, device=gpu))
	with pytest.raises(RuntimeError, match='eps_density'):
		ext.pack_foam(pts, torch.zeros(5, dtype=torch.int32, device=gpu), torch.zeros(0, dtype=torch.int32, device=gpu),
					  torch.zeros(4, device=gpu), torch.zeros(4, 3, device=gpu), torch.zeros(4, 3, device=gpu),
					  torch.zeros(4, 6, device=gpu), torch.zeros(4, 6, device=gpu), torch.zeros(4, 16, 3, device=gpu),
					  eps_density=-1.0)
	assert np.isfinite(0.0)
