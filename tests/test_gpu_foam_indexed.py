"""GPU tests of the indexed edge records (vgr_foam_index_pack, vgr_foam_infer_indexed): the records' layout, and
the fused rendering through them bit-identical to vgr_foam_infer_lanes with one ray per lane on the reference
records (rgb, T, depth, statistics, traces), which the oracle pins in turn; exact colours through them as the
one-pass blend (with the slot table and the colour cut-off +inf); every other stage, colour mode and ray layout
falls back to the reference records unchanged."""

import math

import numpy as np
import pytest
import torch

from helpers import Field, ray_bounds_np
from test_gpu_foam import compare, ref_foam, scene_pack
from vgr import ext, render, scenes

pytestmark = pytest.mark.gpu

FIELDS = ('rgb', 'T', 'depth', 'stats', 'trace')


def run(dev, pk, sh_deg, o, d, start, near, far, t_thresh=1e-4, w_thresh=1e-4, color_cut=math.inf, color_mode=2,
		stage=2, cap=None, trace_cap=0, lanes=1, indexed=False, slots=False):
	"""One foam_infer launch on numpy inputs -> dict of numpy outputs; indexed: through index_pack's records;
	slots: with the pack's slot table (the reference's cache misses counted once per pass)."""
	t = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=dev)  # noqa: E731
	empty = torch.empty(0, dtype=torch.int32, device=dev)
	orig = pk.get('orig')
	tens = {k: t(pk[k]) for k in ('points', 'offsets', 'nbr', 'edge', 'attr', 'sh')}
	idx = ext.index_pack(tens['offsets'], tens['nbr'], tens['edge'], tens['attr']) if indexed else None
	out = ext.foam_infer_extension().foam_infer(
		tens['points'], tens['offsets'], tens['nbr'], tens['edge'], tens['attr'], tens['sh'], sh_deg, t(o), t(d),
		t(start), t(near), t(far), t_thresh, w_thresh, color_cut, color_mode, stage,
		empty if cap is None else t(cap.astype(np.int32)), t(orig) if orig is not None and len(orig) else empty,
		trace_cap=trace_cap, lanes=lanes, indexed=idx,
		slots=ext.slot_table(tens['offsets'], tens['nbr']) if slots else None)
	torch.cuda.synchronize()
	res = dict(zip(FIELDS, [x.cpu().numpy() for x in out]))
	res.setdefault('trace', None)
	return res


def assert_identical(a, b):
	for k in FIELDS:
		if a[k] is None:
			assert b[k] is None
			continue
		if a[k].dtype == np.float32:  # bit patterns: NaN-safe and sign-of-zero exact
			np.testing.assert_array_equal(a[k].view(np.int32), b[k].view(np.int32), err_msg=k)
		else:
			np.testing.assert_array_equal(a[k], b[k], err_msg=k)


@pytest.fixture(scope='module')
def small(gpu):
	f = Field(seed=5, n=300)
	return f, f.rays(B=256, seed=5)


def test_index_pack_layout(gpu, small):
	"""edge_i = (p_j, bits of nbr[e]); attr_i = attr except column 7, which holds edge[offsets[k], 3] bit for bit;
	and the layout's premise: every record pointing at site k carries that same cut-off word."""
	f, _ = small
	for eps in (0.0, 1e-3):
		pk = f.pack(eps_density=eps, reorder=eps > 0)
		t = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=gpu)  # noqa: E731
		ei, ai = ext.index_pack(t(pk['offsets']), t(pk['nbr']), t(pk['edge']), t(pk['attr']))
		ei, ai = ei.cpu().numpy(), ai.cpu().numpy()
		np.testing.assert_array_equal(ei[:, :3].view(np.int32), pk['edge'][:, :3].view(np.int32))
		np.testing.assert_array_equal(ei[:, 3].view(np.int32), pk['nbr'])
		cut = pk['edge'][pk['offsets'][:-1], 3].view(np.int32)
		np.testing.assert_array_equal(pk['edge'][:, 3].view(np.int32), cut[pk['nbr']])
		np.testing.assert_array_equal(ai[:, 7].view(np.int32), cut)
		keep = [c for c in range(20) if c != 7]
		np.testing.assert_array_equal(ai[:, keep].view(np.int32), pk['attr'][:, keep].view(np.int32))


@pytest.mark.parametrize('sh_deg', [0, 1, 2, 3])
@pytest.mark.parametrize('sh_half', [False, True])
def test_indexed_identical_small_field(gpu, small, sh_deg, sh_half):
	"""Fused colours through the indexed records against the reference records (one ray per lane): every output
	bit-identical, thresholds on and off, with and without a colour cut-off, renumbered or not; and the oracle."""
	f, (o, d, start, near, _, far) = small
	for reorder in (False, True):
		pk = f.pack(sh_half=sh_half, reorder=reorder, eps_density=1e-3 if reorder else 0.0)
		st = pk['inv'][start].astype(np.int32) if reorder else start
		for tt, wt, cut in ((1e-4, 1e-4, math.inf), (0.0, -1.0, math.inf), (1e-4, 1e-4, 2 * math.log(1e3))):
			kw = dict(t_thresh=tt, w_thresh=wt, color_cut=cut, trace_cap=512)
			a = run(gpu, pk, sh_deg, o, d, st, near, far, **kw)
			b = run(gpu, pk, sh_deg, o, d, st, near, far, indexed=True, **kw)
			assert_identical(a, b)
			assert_identical(a, run(gpu, pk, sh_deg, o, d, st, near, far, indexed=True, slots=True, **kw))
			if cut == math.inf and not sh_half:
				r = ref_foam(pk, sh_deg, o, d, st, near, far, tt, wt, color_mode=2, trace_cap=512)
				compare(b, r, exact_trace=tt == 0.0, stats_frac=1.0 if tt == 0.0 else 0.98)


def test_indexed_cap_bad_starts_and_default_layout(gpu, small):
	"""A per-ray sample cap, starts outside the scene, no trace, and the default layout (lanes None)."""
	f, (o, d, start, near, _, far) = small
	pk = f.pack()
	cap = np.full(len(o), 7, np.int32)
	bad = start.copy()
	bad[:4] = [-1, f.n, 2 ** 30, -7]
	for kw in (dict(cap=cap), dict(trace_cap=64), dict(lanes=None), dict(lanes=None, trace_cap=64)):
		a = run(gpu, pk, 3, o, d, bad, near, far, **kw)
		b = run(gpu, pk, 3, o, d, bad, near, far, indexed=True, **kw)
		assert_identical(a, b)
	assert (b['T'][:4] == 1).all() and (b['rgb'][:4] == 0).all() and (b['stats'][:4] == 0).all()


@pytest.mark.parametrize('sh_deg', [0, 3])
@pytest.mark.parametrize('sh_half', [False, True])
def test_exact_colours_by_the_blend(gpu, small, sh_deg, sh_half):
	"""Exact colours with the indexed records, the slot table and the colour cut-off +inf run as the one-pass blend
	(one ray per lane): rgb, T, depth, traces and the first four statistics bit-identical to the fused mode through
	the same records; stats[:, 4] the exact mode's cache misses, every statistic of every ray equal to the two-pass
	kernel's (reference records, same table) with the thresholds off, and rgb within 1e-5 of it; against the oracle
	in exact mode (its cache on) within the parity bar."""
	f, (o, d, start, near, _, far) = small
	for reorder in (False, True):
		pk = f.pack(sh_half=sh_half, reorder=reorder)
		st = pk['inv'][start].astype(np.int32) if reorder else start
		for tt, wt in ((1e-4, 1e-4), (0.0, -1.0)):
			kw = dict(t_thresh=tt, w_thresh=wt, trace_cap=512)
			for lanes in (1, None):
				blend = run(gpu, pk, sh_deg, o, d, st, near, far, color_mode=0, lanes=lanes, indexed=True, slots=True,
							**kw)
				fused = run(gpu, pk, sh_deg, o, d, st, near, far, color_mode=2, lanes=lanes, indexed=True, slots=True,
							**kw)
				for k in ('rgb', 'T', 'depth', 'trace'):
					np.testing.assert_array_equal(blend[k].view(np.int32), fused[k].view(np.int32), err_msg=k)
				np.testing.assert_array_equal(blend['stats'][:, :4], fused['stats'][:, :4])
			two = run(gpu, pk, sh_deg, o, d, st, near, far, color_mode=0, lanes=1, slots=True, **kw)
			np.testing.assert_allclose(blend['rgb'], two['rgb'], atol=1e-5, rtol=0)
			np.testing.assert_array_equal(blend['T'].view(np.int32), two['T'].view(np.int32))
			if tt == 0.0:
				np.testing.assert_array_equal(blend['stats'], two['stats'])
				np.testing.assert_array_equal(blend['trace'], two['trace'])
			if not sh_half:
				r = ref_foam(pk, sh_deg, o, d, st, near, far, tt, wt, color_mode=0, trace_cap=512)
				compare(blend, r, exact_trace=tt == 0.0, stats_frac=1.0 if tt == 0.0 else 0.98)


def test_exact_colours_blend_falls_back(gpu, small):
	"""Exact colours run as two passes without the slot table, with a finite colour cut-off, or with a group of lanes
	per ray, indexed records given or not: the same outputs either way."""
	f, (o, d, start, near, _, far) = small
	pk = f.pack()
	for kw in (dict(slots=False), dict(slots=True, color_cut=2 * math.log(1e3)), dict(slots=True, lanes=4),
			   dict(slots=True, lanes=2)):
		a = run(gpu, pk, 3, o, d, start, near, far, color_mode=0, trace_cap=128, **kw)
		b = run(gpu, pk, 3, o, d, start, near, far, color_mode=0, trace_cap=128, indexed=True, **kw)
		assert_identical(a, b)


def test_indexed_falls_back_outside_fused_one_lane(gpu, small):
	"""Exact colours without the slot table, baked colours, stages 0 and 1, and groups of lanes per ray ignore the
	indexed records: the same outputs as without them."""
	f, (o, d, start, near, _, far) = small
	pk = f.pack()
	pk['attr'][:, 16:19] = 0.25
	for kw in (dict(color_mode=0), dict(color_mode=1, color_cut=2 * math.log(1e3)), dict(stage=0), dict(stage=1),
			   dict(lanes=4), dict(lanes=2, color_mode=2), dict(lanes=None, color_mode=0)):
		a = run(gpu, pk, 3, o, d, start, near, far, trace_cap=128, **kw)
		b = run(gpu, pk, 3, o, d, start, near, far, trace_cap=128, indexed=True, **kw)
		assert_identical(a, b)


@pytest.mark.parametrize('config,scale,img', [(1, 1.0, 1.0), (3, 0.02, 0.08)])
def test_indexed_identical_scenes(gpu, config, scale, img):
	"""Benchmark scenes in the benchmark's ray order (8x8 tiles, Z-order), renumbered pack: bit-identical."""
	sc = scenes.make_scene(config, scale=scale, img_scale=img, cache_dir=None, log=None)
	_, pk = scene_pack(sc, reorder=True)
	o, d, start, _ = sc.camera_rays(tile=8, curve='morton')
	near, _, far = ray_bounds_np(o, d, 0.02, sc.far_radius)
	st = pk['inv'][start].astype(np.int32)
	a = run(gpu, pk, sc.sh_deg, o, d, st, near, far, trace_cap=256)
	b = run(gpu, pk, sc.sh_deg, o, d, st, near, far, trace_cap=256, indexed=True)
	assert_identical(a, b)


def test_render_rays_with_indexed_pack(gpu, small):
	"""render.index_pack + render_rays_foam_infer: the same image as the reference records; errors on records of
	the wrong shape."""
	f, (o, d, start, _, _, _) = small
	from types import SimpleNamespace
	T = lambda a: torch.as_tensor(a, device=gpu)  # noqa: E731
	model = SimpleNamespace(graph=ext.Graph(T(f.points), T(f.offsets), T(f.adj)), raw=T(f.raw),
							d_log_scale=T(f.d_log_scale), d_quat=T(f.d_quat), c_log_scale=T(f.c_log_scale),
							c_quat=T(f.c_quat), sh=lambda: T(f.sh), sh_deg=3, bg_logit=torch.zeros(3, device=gpu))
	pack = render.pack_foam(model, reorder=True, index=False)
	assert 'edge_i' not in pack and 'edge_i' in render.pack_foam(model, reorder=True)  # pack_foam indexes by default
	a = render.render_rays_foam_infer(model, pack, T(o), T(d), T(start), far_radius=2.0, colors='fused',
									  trace_cap=128)
	render.index_pack(pack)
	b = render.render_rays_foam_infer(model, pack, T(o), T(d), T(start), far_radius=2.0, colors='fused',
									  trace_cap=128)
	for k in ('rgb', 'acc', 'depth', 'stats', 'trace'):
		assert torch.equal(a[k], b[k]), k
	fi = ext.foam_infer_extension()
	args = [pack[k] for k in ('points', 'offsets', 'nbr', 'edge', 'attr', 'sh')]
	o_, d_ = T(o).float(), T(d).float()
	near = torch.full((len(o),), 0.02, device=gpu)
	far = torch.full((len(o),), 2.0, device=gpu)
	e = torch.empty(0, dtype=torch.int32, device=gpu)
	with pytest.raises(RuntimeError, match='edge_i and attr_i'):
		fi.foam_infer(*args, 3, o_, d_, pack['inv'][T(start).long()].int(), near, far, 1e-4, 1e-4, math.inf, 2, 2,
					  e, pack['orig'], indexed=(pack['edge_i'][:-1], pack['attr_i']))


@pytest.mark.parametrize('lanes', [2, 4, 8])
def test_site_rows_identical_in_group_layouts(gpu, small, lanes):
	"""The group layouts reading the 64-byte site rows (the first 16 record columns, rows of ext.foam_infer's indexed
	argument), or the 256-byte site blocks that hold the fp32 SH row after them (read in place of sh too), give every
	output bit-identical to the 80-byte attr rows: fused and exact colours, thresholds on and off, renumbered or not,
	with the slot table and without. Site blocks with fp16 SH are refused."""
	f, (o, d, start, near, _, far) = small
	t = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=gpu)  # noqa: E731
	empty = torch.empty(0, dtype=torch.int32, device=gpu)
	for reorder in (False, True):
		pk = f.pack(reorder=reorder)
		st = pk['inv'][start].astype(np.int32) if reorder else start
		tens = {k: t(pk[k]) for k in ('points', 'offsets', 'nbr', 'edge', 'attr', 'sh')}
		ei, ai = ext.index_pack(tens['offsets'], tens['nbr'], tens['edge'], tens['attr'])
		rows = ai[:, :16].contiguous()
		blocks = torch.cat([rows, tens['sh'].reshape(-1, 48)], 1).contiguous()
		assert blocks.data_ptr() % 256 == 0
		slots = ext.slot_table(tens['offsets'], tens['nbr'])
		orig = t(pk['orig']) if pk.get('orig') is not None and len(pk['orig']) else empty
		for mode in (0, 2):
			for tt, wt in ((1e-4, 1e-4), (0.0, -1.0)):
				outs = []
				for idx, sl in (((ei, ai), None), ((ei, ai, rows), None), ((ei, ai, rows), slots),
								((ei, ai, blocks), None), ((ei, ai, blocks), slots)):
					out = ext.foam_infer_extension().foam_infer(
						tens['points'], tens['offsets'], tens['nbr'], tens['edge'], tens['attr'], tens['sh'], 3, t(o),
						t(d), t(st), t(near), t(far), tt, wt, math.inf, mode, 2, empty, orig, trace_cap=256,
						lanes=lanes, indexed=idx, slots=sl)
					torch.cuda.synchronize()
					outs.append(dict(zip(FIELDS, [x.cpu().numpy() for x in out])))
				for other in outs[1:]:
					assert_identical(outs[0], other)
	with pytest.raises(RuntimeError, match='float32'):
		ext.foam_infer_extension().foam_infer(
			tens['points'], tens['offsets'], tens['nbr'], tens['edge'], tens['attr'], tens['sh'].half(), 3, t(o), t(d),
			t(st), t(near), t(far), 1e-4, 1e-4, math.inf, 2, 2, empty, orig, lanes=lanes, indexed=(ei, ai, blocks))
