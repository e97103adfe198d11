"""Coherent ray order (vgr_ray_order) and the renderers' `order` argument: the order is a permutation grouping the
rays by direction bin and origin Z-order, and tracing a batch in it gives every ray bit-identical outputs (each
ray's arithmetic does not depend on the other lanes) in every layout of foam_infer and march_forward."""

import math

import numpy as np
import pytest
import torch

from helpers import Field
from vgr import ext, scenes
from test_gpu_foam import scene_pack
from helpers import ray_bounds_np

pytestmark = pytest.mark.gpu


def T(a, dev):
	return torch.as_tensor(np.ascontiguousarray(a), device=dev)


def octa_bin(d, res):
	"""The octahedral direction bin, restated in numpy float32."""
	d = d.astype(np.float32)
	a = np.abs(d).sum(1)
	u, v = d[:, 0] / a, d[:, 1] / a
	neg = d[:, 2] < 0
	fu = (1 - np.abs(v)) * np.copysign(np.float32(1), u)
	fv = (1 - np.abs(u)) * np.copysign(np.float32(1), v)
	u, v = np.where(neg, fu, u), np.where(neg, fv, v)
	iu = np.clip(((u + 1) * np.float32(0.5) * res).astype(np.int64), 0, res - 1)
	iv = np.clip(((v + 1) * np.float32(0.5) * res).astype(np.int64), 0, res - 1)
	return iu * res + iv


def test_ray_order_is_a_grouping_permutation(gpu):
	sc = scenes.make_scene(5, scale=0.002, n_rays=100000, cache_dir=None, log=None)
	o, d = sc.ray_batch
	order = ext.ray_order(T(o, gpu), T(d, gpu), dir_res=8, pos_bits=7).cpu().numpy()
	np.testing.assert_array_equal(np.sort(order), np.arange(len(o)))
	bins = octa_bin(d[order], 8)
	assert (np.diff(bins) >= 0).all()  # sorted by direction bin first
	# within a bin, consecutive rays are close: the mean origin gap is far below that of the batch order
	same = np.diff(bins) == 0
	gap = np.linalg.norm(np.diff(o[order], axis=0), axis=1)[same].mean()
	assert gap < 0.25 * np.linalg.norm(np.diff(o, axis=0), axis=1).mean()
	assert ext.ray_order(T(o[:0], gpu), T(d[:0], gpu)).numel() == 0


@pytest.mark.parametrize('lanes', [None, 1, 4])
def test_foam_infer_order_gives_identical_rays(gpu, lanes):
	sc = scenes.make_scene(5, scale=0.005, n_rays=20000, cache_dir=None, log=None)
	_, pk = scene_pack(sc, reorder=True)
	o, d, start, _ = sc.camera_rays()
	st = pk['inv'][start].astype(np.int32)
	near, _, far = ray_bounds_np(o, d, 0.02, sc.far_radius)
	p = {k: T(pk[k], gpu) for k in ('points', 'offsets', 'nbr', 'edge', 'attr', 'sh', 'orig')}
	rays = [T(a, gpu) for a in (o, d, st, near, far)]
	order = ext.ray_order(rays[0], rays[1])
	empty = torch.empty(0, dtype=torch.int32, device=gpu)
	fi = ext.foam_infer_extension()
	for mode in (2, 0):
		args = (p['points'], p['offsets'], p['nbr'], p['edge'], p['attr'], p['sh'], sc.sh_deg, *rays, 1e-4, 1e-4,
				math.inf, mode, 2, empty, p['orig'])
		a = fi.foam_infer(*args, trace_cap=64, lanes=lanes)
		b = fi.foam_infer(*args, trace_cap=64, lanes=lanes, order=order)
		for x, y in zip(a, b):
			assert torch.equal(x, y)
	# an order entry outside [0, B) is skipped: that ray's outputs are not written
	bad = order.clone()
	bad[:5] = -1
	out = fi.foam_infer(*args, lanes=lanes, order=bad)
	np.testing.assert_array_equal(out[3][order[5:].long()].cpu().numpy(), a[3][order[5:].long()].cpu().numpy())


@pytest.mark.parametrize('lanes', [1, 16])
def test_march_order_gives_identical_rays(gpu, lanes):
	f = Field(seed=3, n=400)
	o, d, start, near, mid, far = f.rays(B=3000, seed=3)
	dA, cA = f.conics(0.01)
	field = [T(a, gpu) for a in (f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh)]
	rt = [T(a, gpu) for a in (o, d, start, near, mid, far)]
	order = ext.ray_order(rt[0], rt[1], dir_res=2, pos_bits=9)
	mx = ext.march_extension()
	a = mx.march_forward(*field, 3, *rt, 0.05, 8, 1e-4, 1e-4, trace_cap=128, lanes=lanes)
	b = mx.march_forward(*field, 3, *rt, 0.05, 8, 1e-4, 1e-4, trace_cap=128, lanes=lanes, order=order)
	for x, y in zip(a, b):
		assert torch.equal(x, y)
	with pytest.raises(RuntimeError, match='order'):
		mx.march_forward(*field, 3, *rt, 0.05, 8, 1e-4, 1e-4, lanes=lanes, order=order[:10])
