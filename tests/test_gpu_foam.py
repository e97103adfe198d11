"""GPU parity of foam_infer (libvgr.so through the C ABI) against the CPU oracle on identical seeded inputs:
visited-cell sequences bit-exact, rgb / T / depth within 1e-4 absolute, per-ray statistics equal."""

import math

import numpy as np
import pytest
import torch

import oracle
from helpers import Field, ray_bounds_np
from vgr import ext, render, scenes

pytestmark = pytest.mark.gpu

TOL = 1e-4  # absolute, fp32 rgb / T / depth (north-star parity bar)


def ref_foam(*args, **kw):
	"""The oracle with the reference's per-ray colour cache (foam_infer.cu:151-168), so stats[:, 4] on both sides
	is the number of colour lookups that miss that 8-slot cache; colours are identical with the cache on or off."""
	kw.setdefault('use_cache', True)
	return oracle.foam_infer(*args, **kw)


def gpu_foam(dev, pk, sh_deg, o, d, start, near, far, t_thresh=1e-4, w_thresh=1e-4, color_cut=math.inf,
			 color_mode=0, stage=2, cap=None, trace_cap=0, lanes=None, slots=False):
	t = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=dev)  # noqa: E731
	empty = torch.empty(0, dtype=torch.int32, device=dev)
	orig = pk.get('orig')
	out = ext.foam_infer_extension().foam_infer(
		t(pk['points']), t(pk['offsets']), t(pk['nbr']), t(pk['edge']), t(pk['attr']), t(pk['sh']), sh_deg, t(o),
		t(d), t(start), t(near), t(far), t_thresh, w_thresh, color_cut, color_mode, stage,
		empty if cap is None else t(cap.astype(np.int32)), t(orig) if orig is not None and len(orig) else empty,
		trace_cap=trace_cap, lanes=lanes, slots=ext.slot_table(t(pk['offsets']), t(pk['nbr'])) if slots else None)
	torch.cuda.synchronize()
	res = dict(zip(('rgb', 'T', 'depth', 'stats', 'trace'), [x.cpu().numpy() for x in out]))
	res.setdefault('trace', None)
	return res


def compare(g, r, exact_trace=True, stats_frac=1.0, tol=TOL, w_thresh=1e-4, t_max=4.0):
	"""GPU outputs g against oracle outputs r. rgb and T: within `tol` on every ray. Per-ray statistics equal on
	at least stats_frac of the rays; the others are rays where a threshold test (w > w_thresh or T < t_thresh) saw
	a value within a few ulps of the threshold, since exp differs by ulps between the CPU and the GPU. On those
	rays a segment of weight ~w_thresh at t <= t_max is in or out, so depth may move by w_thresh * t_max."""
	assert np.isfinite(g['rgb']).all() and np.isfinite(g['T']).all()
	np.testing.assert_allclose(g['rgb'], r['rgb'], atol=tol, rtol=0)
	np.testing.assert_allclose(g['T'], r['T'], atol=tol, rtol=0)
	same = (g['stats'] == r['stats']).all(1)
	assert same.mean() >= stats_frac, f'stats equal on {same.mean():.4f} of rays'
	np.testing.assert_allclose(g['depth'][same], r['depth'][same], atol=tol, rtol=tol)
	np.testing.assert_allclose(g['depth'][~same], r['depth'][~same], atol=tol + w_thresh * t_max, rtol=tol)
	if g['trace'] is not None:
		if exact_trace:
			np.testing.assert_array_equal(g['trace'], r['trace'])
		else:  # early termination is coupled to exp: compare the common prefix
			n = np.minimum(g['stats'][:, 0], r['stats'][:, 0])
			cap = g['trace'].shape[1]
			for i in np.nonzero((g['trace'] != r['trace']).any(1))[0]:
				k = min(n[i], cap)
				np.testing.assert_array_equal(g['trace'][i, :k], r['trace'][i, :k])


def psnr(a, b):
	mse = float(((a - b) ** 2).mean())
	return 99.0 if mse == 0 else 10 * math.log10(1.0 / mse)


@pytest.fixture(scope='module')
def small(gpu):
	f = Field(seed=2, n=300)
	return f, f.rays(B=256, seed=2)


@pytest.mark.parametrize('stage', [0, 1, 2])
def test_small_field_stages_thresholds_off(gpu, small, stage):
	"""Thresholds off (every segment counts, t_thresh = 0, w_thresh = -1): full traversals, bit-exact cells."""
	f, (o, d, start, near, _, far) = small
	pk = f.pack()
	g = gpu_foam(gpu, pk, 3, o, d, start, near, far, 0.0, -1.0, stage=stage, trace_cap=512)
	r = ref_foam(pk, 3, o, d, start, near, far, 0.0, -1.0, stage=stage, trace_cap=512)
	compare(g, r)


@pytest.mark.parametrize('color_mode', [0, 2])
@pytest.mark.parametrize('sh_half', [False, True])
@pytest.mark.parametrize('reorder', [False, True])
def test_small_field_modes(gpu, small, color_mode, sh_half, reorder):
	f, (o, d, start, near, _, far) = small
	pk = f.pack(sh_half=sh_half, reorder=reorder)
	st = pk['inv'][start].astype(np.int32) if reorder else start
	g = gpu_foam(gpu, pk, 3, o, d, st, near, far, color_mode=color_mode, trace_cap=512)
	r = ref_foam(pk, 3, o, d, st, near, far, color_mode=color_mode, trace_cap=512)
	compare(g, r, exact_trace=False, stats_frac=0.98)


def test_small_field_baked_eps_and_cap(gpu, small):
	f, (o, d, start, near, _, far) = small
	pk = f.pack(eps_density=1e-3)
	center = np.array([0.1, 0.2, 2.5], np.float32)
	dirs = f.points - center
	dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
	b = render.sh_basis(torch.from_numpy(dirs.astype(np.float32)), 3).numpy()
	pk['attr'][:, 16:19] = np.maximum((b[:, :, None] * f.sh).sum(1) + 0.5, 0)
	cut = 2 * math.log(1 / 1e-3)
	for mode in (1, 2, 0):
		g = gpu_foam(gpu, pk, 3, o, d, start, near, far, color_cut=cut, color_mode=mode, trace_cap=512)
		r = ref_foam(pk, 3, o, d, start, near, far, color_cut=cut, color_mode=mode, trace_cap=512)
		compare(g, r, exact_trace=False, stats_frac=0.98)
	cap = np.maximum(2, r['stats'][:, 0] // 2).astype(np.int32)
	g = gpu_foam(gpu, pk, 3, o, d, start, near, far, stage=0, cap=cap, trace_cap=512)
	r = ref_foam(pk, 3, o, d, start, near, far, stage=0, cap=cap, trace_cap=512)
	compare(g, r)
	np.testing.assert_array_equal(g['stats'][:, 0], cap)


def scene_pack(scene, reorder=False):
	"""Pack a synthetic scene on the GPU (pack_foam with the HIP conic kernel) -> numpy dict for both sides."""
	from vgr.model import VoronoiGaussField
	model = VoronoiGaussField.from_scene(scene, 'cuda')
	pk = render.pack_foam(model, reorder=reorder)
	out = {k: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v) for k, v in pk.items()}
	return model, out


@pytest.mark.parametrize('config,scale,img', [(1, 1.0, 1.0), (2, 0.04, 0.15), (3, 0.02, 0.08), (4, 0.004, 0.06)])
def test_benchmark_scenes_vs_oracle(gpu, config, scale, img):
	"""Seeded benchmark scenes (configs 1-4, reduced site counts beyond config 1), default thresholds, exact
	colours: rgb within 1e-4, PSNR >= 60 dB, cell-sequence prefixes identical."""
	sc = scenes.make_scene(config, scale=scale, img_scale=img, cache_dir=None, log=None)
	model, pk = scene_pack(sc, reorder=config % 2 == 0)
	o, d, start, _ = sc.camera_rays(tile=8)
	near, _, far = ray_bounds_np(o, d, 0.02, sc.far_radius)
	st = pk['inv'][start].astype(np.int32) if pk['inv'] is not None else start
	if len(o) > 60000:  # the oracle checks a deterministic subset; the GPU renders the same subset
		sel = np.arange(0, len(o), len(o) // 60000 + 1)
		o, d, st, near, far = o[sel], d[sel], st[sel], near[sel], far[sel]
	g = gpu_foam(gpu, pk, sc.sh_deg, o, d, st, near, far, trace_cap=256)
	r = ref_foam(pk, sc.sh_deg, o, d, st, near, far, trace_cap=256)
	compare(g, r, exact_trace=False, stats_frac=0.99)
	assert psnr(g['rgb'], r['rgb']) >= 60.0


def test_random_ray_batch_config5(gpu):
	"""Config 5 layout (uniform sites, incoherent rays from inside the cube, low density) at reduced size."""
	sc = scenes.make_scene(5, scale=0.005, n_rays=4096, cache_dir=None, log=None)
	model, pk = scene_pack(sc)
	o, d, start, _ = sc.camera_rays()
	near, _, far = ray_bounds_np(o, d, 0.02, sc.far_radius)
	g = gpu_foam(gpu, pk, 3, o, d, start, near, far, trace_cap=1024)
	r = ref_foam(pk, 3, o, d, start, near, far, trace_cap=1024)
	compare(g, r, exact_trace=False, stats_frac=0.99)
	g0 = gpu_foam(gpu, pk, 3, o, d, start, near, far, stage=0, trace_cap=1024)
	r0 = ref_foam(pk, 3, o, d, start, near, far, stage=0, trace_cap=1024)
	compare(g0, r0)


@pytest.mark.parametrize('lanes', [1, 2, 4, 8])
def test_layouts_small_field(gpu, small, lanes):
	"""Every ray layout of vgr_foam_infer_lanes (one ray per lane, a group of 2, 4 or 8 lanes per ray), whichever
	the default is: every stage and colour mode against the oracle; thresholds off, every statistic equal and the
	cell sequences bit-exact."""
	f, (o, d, start, near, _, far) = small
	pk = f.pack()
	for stage in (0, 1, 2):
		g = gpu_foam(gpu, pk, 3, o, d, start, near, far, 0.0, -1.0, stage=stage, trace_cap=512, lanes=lanes)
		r = ref_foam(pk, 3, o, d, start, near, far, 0.0, -1.0, stage=stage, trace_cap=512)
		compare(g, r)
	for color_mode in (0, 2):
		for sh_half in (False, True):
			pk = f.pack(sh_half=sh_half, reorder=True)
			st = pk['inv'][start].astype(np.int32)
			g = gpu_foam(gpu, pk, 3, o, d, st, near, far, color_mode=color_mode, trace_cap=512, lanes=lanes)
			r = ref_foam(pk, 3, o, d, st, near, far, color_mode=color_mode, trace_cap=512)
			compare(g, r, exact_trace=False, stats_frac=0.98)
	pk = f.pack(eps_density=1e-3)
	center = np.array([0.1, 0.2, 2.5], np.float32)
	dirs = f.points - center
	dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
	b = render.sh_basis(torch.from_numpy(dirs.astype(np.float32)), 3).numpy()
	pk['attr'][:, 16:19] = np.maximum((b[:, :, None] * f.sh).sum(1) + 0.5, 0)
	cut = 2 * math.log(1 / 1e-3)
	for mode in (1, 2, 0):
		g = gpu_foam(gpu, pk, 3, o, d, start, near, far, color_cut=cut, color_mode=mode, trace_cap=512, lanes=lanes)
		r = ref_foam(pk, 3, o, d, start, near, far, color_cut=cut, color_mode=mode, trace_cap=512)
		compare(g, r, exact_trace=False, stats_frac=0.98)
	cap = np.maximum(2, r['stats'][:, 0] // 2).astype(np.int32)
	g = gpu_foam(gpu, pk, 3, o, d, start, near, far, stage=0, cap=cap, trace_cap=512, lanes=lanes)
	np.testing.assert_array_equal(g['stats'][:, 0], cap)
	bad = start.copy()
	bad[:4] = -1
	g = gpu_foam(gpu, pk, 3, o, d, bad, near, far, lanes=lanes)
	assert (g['T'][:4] == 1).all() and (g['rgb'][:4] == 0).all() and (g['stats'][:4] == 0).all()


@pytest.mark.parametrize('lanes', [1, 2, 4, 8])
def test_sh_miss_count_every_layout(gpu, small, lanes):
	"""stats[:, 4] is the reference's count of colour lookups that miss its per-ray 8-slot cache (foam_infer.cu:
	151-168, 359-360), in every ray layout, exact and fused colours, with and without a colour cut-off, with the
	thresholds off (every statistic of every ray equal to the oracle's with its cache on), with the tags per lookup
	in LDS and from the slot table once per pass (colour cut-off +inf). The count is below the number of lookups
	(the oracle without the cache), so the cache is exercised."""
	f, (o, d, start, near, _, far) = small
	pk = f.pack(reorder=True)
	st = pk['inv'][start].astype(np.int32)
	for mode, cut, table in ((0, math.inf, False), (0, math.inf, True), (2, math.inf, False), (2, math.inf, True),
							 (0, 2 * math.log(1e3), False), (2, 2 * math.log(1e3), True)):
		if cut != math.inf and mode == 2 and lanes != 1:
			continue  # a finite cut-off in fused mode always runs one ray per lane
		# (a finite cut-off with the table given keeps per-lookup tags: the table only applies to full passes)
		g = gpu_foam(gpu, pk, 3, o, d, st, near, far, 0.0, -1.0, color_cut=cut, color_mode=mode, trace_cap=512,
					 lanes=lanes, slots=table)
		r = ref_foam(pk, 3, o, d, st, near, far, 0.0, -1.0, color_cut=cut, color_mode=mode, trace_cap=512)
		compare(g, r)
		every = ref_foam(pk, 3, o, d, st, near, far, 0.0, -1.0, color_cut=cut, color_mode=mode, use_cache=False)
		assert (g['stats'][:, 4] <= every['stats'][:, 4]).all()
		assert g['stats'][:, 4].sum() < every['stats'][:, 4].sum()


def test_slot_table_layout(gpu, small):
	"""ext.slot_table (vgr_foam_slot_table) against a restatement on the host: per site and slot s (site & 7) of
	its self-first neighbourhood in CSR order, the first and the last entry at columns 2s and 2s + 1, -2 for an empty
	slot."""
	f, _ = small
	for reorder in (False, True):
		pk = f.pack(reorder=reorder)
		t = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=gpu)  # noqa: E731
		got = ext.slot_table(t(pk['offsets']), t(pk['nbr'])).cpu().numpy()
		want = np.full((f.n, 16), -2, np.int32)
		for k in range(f.n):
			for j in pk['nbr'][pk['offsets'][k]:pk['offsets'][k + 1]]:
				s = int(j) & 7
				if want[k, 2 * s] == -2:
					want[k, 2 * s] = j
				want[k, 2 * s + 1] = j
		np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize('lanes', [1, 2, 4, 8])
@pytest.mark.parametrize('config,scale,img', [(1, 1.0, 1.0), (3, 0.02, 0.08), (5, 0.005, 0.0)])
def test_layouts_scenes(gpu, lanes, config, scale, img):
	"""Every ray layout on benchmark scenes (exact colours and fused colours) against the oracle, and against the
	one-ray-per-lane layout: the same cells (stage 0 statistics bit-equal)."""
	if config == 5:
		sc = scenes.make_scene(5, scale=scale, n_rays=4096, cache_dir=None, log=None)
	else:
		sc = scenes.make_scene(config, scale=scale, img_scale=img, cache_dir=None, log=None)
	model, pk = scene_pack(sc, reorder=config != 5)
	o, d, start, _ = sc.camera_rays(tile=8) if config != 5 else sc.camera_rays()
	near, _, far = ray_bounds_np(o, d, 0.02, sc.far_radius)
	st = pk['inv'][start].astype(np.int32) if pk['inv'] is not None else start
	if len(o) > 60000:
		sel = np.arange(0, len(o), len(o) // 60000 + 1)
		o, d, st, near, far = o[sel], d[sel], st[sel], near[sel], far[sel]
	for mode in (0, 2):
		g = gpu_foam(gpu, pk, sc.sh_deg, o, d, st, near, far, color_mode=mode, trace_cap=256, lanes=lanes)
		r = ref_foam(pk, sc.sh_deg, o, d, st, near, far, color_mode=mode, trace_cap=256)
		compare(g, r, exact_trace=False, stats_frac=0.99)
		assert psnr(g['rgb'], r['rgb']) >= 60.0
	g0 = gpu_foam(gpu, pk, sc.sh_deg, o, d, st, near, far, stage=0, trace_cap=256, lanes=lanes)
	l0 = gpu_foam(gpu, pk, sc.sh_deg, o, d, st, near, far, stage=0, trace_cap=256, lanes=1)
	np.testing.assert_array_equal(g0['stats'], l0['stats'])
	np.testing.assert_array_equal(g0['trace'], l0['trace'])


@pytest.mark.parametrize('config,scale', [(1, 1.0), (3, 0.01)])
def test_lane_per_face_traversal_matches(gpu, config, scale):
	"""The lane-per-face traversal (4, 8 or 16 lanes per ray, group min-reductions) visits the same cells with the
	same sample and walk-step counts as foam_infer's thread-per-ray stage 0, bit for bit, and as the oracle."""
	sc = scenes.make_scene(config, scale=scale, img_scale=0.1, cache_dir=None, log=None)
	_, pk = scene_pack(sc, reorder=True)
	o, d, start, _ = sc.camera_rays(tile=8)
	st = pk['inv'][start].astype(np.int32)
	near, _, far = ray_bounds_np(o, d, 0.02, sc.far_radius)
	g = gpu_foam(gpu, pk, sc.sh_deg, o, d, st, near, far, stage=0, trace_cap=512)
	t = lambda a: torch.as_tensor(np.ascontiguousarray(a), device=gpu)  # noqa: E731
	r = ref_foam(pk, sc.sh_deg, o, d, st, near, far, stage=0, trace_cap=512)
	for lanes in (4, 8, 16):
		stats, trace = ext.traverse_faces(t(pk['points']), t(pk['offsets']), t(pk['nbr']), t(pk['edge']), t(o),
										  t(d), t(st), t(near), t(far), orig=t(pk['orig']), trace_cap=512,
										  lanes=lanes)
		np.testing.assert_array_equal(stats.cpu().numpy(), g['stats'])
		np.testing.assert_array_equal(trace.cpu().numpy(), g['trace'])
		np.testing.assert_array_equal(trace.cpu().numpy(), r['trace'])
	with pytest.raises(RuntimeError, match='lanes_per_ray'):
		ext.traverse_faces(t(pk['points']), t(pk['offsets']), t(pk['nbr']), t(pk['edge']), t(o), t(d), t(st),
						   t(near), t(far), lanes=5)
	# a sample cap, and a start outside the scene
	cap = np.full(len(o), 5, np.int32)
	s5 = ext.traverse_faces(t(pk['points']), t(pk['offsets']), t(pk['nbr']), t(pk['edge']), t(o), t(d), t(st),
							t(near), t(far), cap=t(cap), orig=t(pk['orig']))
	assert (s5.cpu().numpy()[:, 0] <= 5).all()
	bad = st.copy()
	bad[:3] = -1
	sb = ext.traverse_faces(t(pk['points']), t(pk['offsets']), t(pk['nbr']), t(pk['edge']), t(o), t(d), t(bad),
							t(near), t(far), orig=t(pk['orig'])).cpu().numpy()
	assert (sb[:3] == 0).all() and (sb[3:, 0] == g['stats'][3:, 0]).all()


def test_render_rays_foam_infer_api(gpu, small):
	"""render.render_rays_foam_infer end to end (bounds, Morton start remap, background) vs the oracle."""
	f, (o, d, start, near, _, far) = small
	from types import SimpleNamespace
	dev = gpu
	T = lambda a: torch.as_tensor(a, device=dev)  # noqa: E731
	model = SimpleNamespace(graph=ext.Graph(T(f.points), T(f.offsets), T(f.adj)), raw=T(f.raw),
							d_log_scale=T(f.d_log_scale), d_quat=T(f.d_quat), c_log_scale=T(f.c_log_scale),
							c_quat=T(f.c_quat), sh=lambda: T(f.sh), sh_deg=3, bg_logit=torch.zeros(3, device=dev))
	for reorder in (False, True):
		pack = render.pack_foam(model, reorder=reorder)
		out = render.render_rays_foam_infer(model, pack, T(o), T(d), T(start), far_radius=2.0, trace_cap=512)
		pk = {k: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v) for k, v in pack.items()}
		st = pk['inv'][start].astype(np.int32) if reorder else start
		r = ref_foam(pk, 3, o, d, st, near, far, trace_cap=512)
		np.testing.assert_allclose(out['rgb'].cpu().numpy(), r['rgb'] + r['T'][:, None] * 0.5, atol=TOL)
		np.testing.assert_allclose(out['acc'].cpu().numpy(), 1 - r['T'], atol=TOL)


def test_errors_and_empty(gpu, small):
	f, (o, d, start, near, _, far) = small
	pk = f.pack()
	with pytest.raises(RuntimeError, match='color_mode'):
		gpu_foam(gpu, pk, 3, o, d, start, near, far, color_mode=3)
	with pytest.raises(RuntimeError, match='stage'):
		gpu_foam(gpu, pk, 3, o, d, start, near, far, stage=5)
	with pytest.raises(RuntimeError, match='CUDA tensor'):
		e = torch.empty(0, dtype=torch.int32)
		ext.foam_infer_extension().foam_infer(*[torch.as_tensor(pk[k]) for k in ('points', 'offsets', 'nbr', 'edge',
																				 'attr', 'sh')], 3, *[torch.as_tensor(a)
																				 for a in (o, d, start, near, far)],
											  1e-4, 1e-4, math.inf, 0, 2, e, e)
	g = gpu_foam(gpu, pk, 3, o[:0], d[:0], start[:0], near[:0], far[:0])
	assert g['rgb'].shape == (0, 3) and g['stats'].shape == (0, 5)
	bad = start.copy()
	bad[:4] = [-1, f.n, 2 ** 30, -7]
	g = gpu_foam(gpu, pk, 3, o, d, bad, near, far)
	assert (g['T'][:4] == 1).all() and (g['rgb'][:4] == 0).all() and (g['stats'][:4] == 0).all()
	r = ref_foam(pk, 3, o[4:], d[4:], start[4:], near[4:], far[4:])
	np.testing.assert_allclose(g['rgb'][4:], r['rgb'], atol=TOL)
