"""GPU parity at the stated sizes of the benchmark configurations 2-5: each scene is built at its full site count
(500K, 2M, 8M and 4M sites, Delaunay by Qhull in background processes, see conftest.py), the GPU renders the
whole workload (every ray of every camera, or config 5's 16,777,216-ray batch), and the C oracle re-renders a
deterministic subset of those rays (every k-th ray) on the host:

- default thresholds, fused and exact colours: rgb and T within 1e-4 on every checked ray, PSNR >= 60 dB over
  them, per-ray statistics equal on >= 99.5 % of them, and every ray whose statistics differ is a ray that ended
  (or coloured a segment) at a transmittance or weight within ulps of its threshold: its cell sequence is
  identical with the thresholds off;
- cell sequences: bit-exact with the thresholds off (stage 0, the geometric traversal, and stage 2), identical
  common prefixes with them on;
- the safety caps (8192 cells per ray, 4096 walk steps) are counted over the whole workload and printed.

Config 5 also runs march_forward on all 16,777,216 rays in the default layout (one ray per lane at this size),
checked on every k-th ray (values within 1e-4, walked sites bit-exact), and march_backward on 524,288 of its rays
(the smallest batch that takes the one-ray-per-lane layout), with upstream gradients on every 256th ray only, so
that the oracle's backward over those rays gives the same gradients (relative errors: 2e-5 for the density gradients
with the thresholds off, 2e-4 for the colour gradients, whose sample weights 1 - exp(-sigma delta) keep few digits
in fp32 at config 5's densities; see the test).

VGR_STATED_CONFIGS=2,3 (say) restricts the configurations."""

import math

import numpy as np
import pytest
import torch

import oracle
from conftest import progress, stated_configs, wait_for_geometry
from helpers import ray_bounds_np
from test_gpu_foam import compare, psnr, ref_foam
from test_oracle_grad import rel
from vgr import ext, render, scenes
from vgr.model import VoronoiGaussField

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(1200)]

TOL = 1e-4
MAX_CELLS, WALK_CAP = 8192, 4096
SUBSET = {2: 16384, 3: 16384, 4: 8192, 5: 8192}


class Stated:
	"""One full-size configuration: the scene, its GPU pack (Z-order renumbered, as the bench packs it), the host
	copy of the pack for the oracle, and the rays of all cameras (8x8 tiles) or of config 5's batch."""

	def __init__(self, config, dev):
		wait_for_geometry(config)
		self.config = config
		self.sc = sc = scenes.make_scene(config, log=None)
		assert sc.n_sites >= 0.999 * scenes.SITE_COUNTS[config]
		self.model = VoronoiGaussField.from_scene(sc, dev)
		self.pack = render.pack_foam(self.model, reorder=True, index=False)
		self.pk = {k: self.pack[k].cpu().numpy() for k in ('points', 'offsets', 'nbr', 'edge', 'attr', 'sh', 'orig')}
		o, d, start, _ = sc.camera_rays(tile=8)
		self.o, self.d = o, d
		self.start_orig = start
		self.start = self.pk['orig'].argsort()[start].astype(np.int32)  # old -> new numbering
		self.near, self.mid, self.far = ray_bounds_np(o, d, 0.02, sc.far_radius)
		self.dev = dev
		self.B = len(o)

	def t(self, a):
		return torch.as_tensor(np.ascontiguousarray(a), device=self.dev)

	def subset(self, n):
		k = max(1, self.B // n)
		return np.arange(k // 2, self.B, k, dtype=np.int64)[:n]

	def foam(self, sel=None, mode=2, t_thresh=1e-4, w_thresh=1e-4, stage=2, trace_cap=0, indexed=None, lanes=None,
			 order=None, slots=None):
		"""GPU foam_infer over the selected rays (all by default) -> dict of numpy arrays; indexed: the records of
		ext.index_pack, read in place of the reference records; lanes, order: the ray layout and processing order
		(vgr_foam_infer_lanes)."""
		pick = (lambda a: a) if sel is None else (lambda a: a[sel])
		p = self.pack
		empty = torch.empty(0, dtype=torch.int32, device=self.dev)
		out = ext.foam_infer_extension().foam_infer(
			p['points'], p['offsets'], p['nbr'], p['edge'], p['attr'], p['sh'], self.sc.sh_deg, self.t(pick(self.o)),
			self.t(pick(self.d)), self.t(pick(self.start)), self.t(pick(self.near)), self.t(pick(self.far)),
			t_thresh, w_thresh, math.inf, mode, stage, empty, p['orig'], trace_cap=trace_cap, indexed=indexed,
			lanes=lanes, order=order, slots=slots)
		torch.cuda.synchronize()
		res = dict(zip(('rgb', 'T', 'depth', 'stats', 'trace'), [x.cpu().numpy() for x in out]))
		res.setdefault('trace', None)
		return res

	def oracle(self, sel, mode=2, t_thresh=1e-4, w_thresh=1e-4, stage=2, trace_cap=0):
		return ref_foam(self.pk, self.sc.sh_deg, self.o, self.d, self.start, self.near, self.far, t_thresh, w_thresh,
						color_mode=mode, stage=stage, rays=sel, trace_cap=trace_cap)


@pytest.fixture(scope='module', params=stated_configs())
def stated(request, gpu):
	s = Stated(request.param, gpu)
	yield s
	del s
	torch.cuda.empty_cache()


def spread(stats, wave=64):
	"""How uneven the work of the rays is: samples per ray (mean, median, 99th percentile, max) and, for waves of 64
	consecutive rays as the one-ray-per-lane kernel runs them, the mean over waves of mean / max of the samples and
	of the density terms per ray (the share of lane time a wave would keep busy if it could only wait for its
	longest ray)."""
	n = stats[:, 0].astype(np.float64)
	m = (len(stats) // wave) * wave
	w = stats[:m].astype(np.float64).reshape(-1, wave, stats.shape[1])
	use = {name: round(float((w[:, :, col].mean(1) / np.maximum(w[:, :, col].max(1), 1)).mean()), 3)
		   for name, col in (('samples', 0), ('density_terms', 3))}
	return {'samples_mean': round(float(n.mean()), 1), 'p50': float(np.percentile(n, 50)),
			'p99': float(np.percentile(n, 99)), 'max': int(n.max()), 'wave_lane_use_bound': use}


def rows(res, sel):
	return {k: (None if v is None else v[sel]) for k, v in res.items()}


def test_foam_full_workload(stated):
	"""The whole workload in fused colours (the bench's mode) on the GPU; the oracle on every k-th ray."""
	s = stated
	full = s.foam()
	sel = s.subset(SUBSET[s.config])
	r = s.oracle(sel)
	g = rows(full, sel)
	same = (g['stats'] == r['stats']).all(1)
	err = np.abs(g['rgb'] - r['rgb']).max()
	progress(f'[stated sizes] config {s.config}: {s.sc.n_sites} sites, {s.B} rays; oracle on {len(sel)} rays: max '
		  f'|rgb| {err:.2e}, max |T| {np.abs(g["T"] - r["T"]).max():.2e}, stats equal on {same.mean():.5f}, PSNR '
		  f'{psnr(g["rgb"], r["rgb"]):.1f} dB; mean samples {full["stats"][:, 0].mean():.1f}')
	compare(g, r, stats_frac=0.995, t_max=s.sc.far_radius)
	assert psnr(g['rgb'], r['rgb']) >= 60.0
	# rays whose statistics differ: same cells with the thresholds off (the difference is where a threshold fell)
	diff = sel[~same]
	if len(diff):
		go = s.foam(diff, stage=0, t_thresh=0.0, w_thresh=-1.0, trace_cap=MAX_CELLS + 1)
		ro = s.oracle(diff, stage=0, t_thresh=0.0, w_thresh=-1.0, trace_cap=MAX_CELLS + 1)
		np.testing.assert_array_equal(go['trace'], ro['trace'])
	if s.config == 5:  # the bench's layout of this batch
		check_config5_bench_layout(s, sel, r)
	caps = {'rays hitting the 8192-cell cap': int((full['stats'][:, 0] > MAX_CELLS).sum()),
			'rays hitting the 4096-step walk cap': int((full['stats'][:, 2] >= WALK_CAP).sum())}
	progress(f'[stated sizes] config {s.config} safety caps over all {s.B} rays: {caps}')
	progress(f'[stated sizes] config {s.config} ray-length spread: {spread(full["stats"])}')


def test_foam_indexed_records_full_workload(stated):
	"""The bench's default path at the stated size: fused colours through the indexed edge records, with the
	reference's cache misses from the slot table, over the whole workload, bit-identical on every ray to the
	reference records with per-lookup tags (which the oracle checks above)."""
	s = stated
	p = s.pack
	idx = ext.index_pack(p['offsets'], p['nbr'], p['edge'], p['attr'])
	slots = ext.slot_table(p['offsets'], p['nbr'])
	a, b = s.foam(), s.foam(indexed=idx, slots=slots)  # b: the bench's path; a: per-lookup cache tags
	del idx, slots
	for k in ('rgb', 'T', 'depth'):
		np.testing.assert_array_equal(a[k].view(np.int32), b[k].view(np.int32), err_msg=k)
	np.testing.assert_array_equal(a['stats'], b['stats'])
	progress(f'[stated sizes] config {s.config}: indexed records bit-identical to the reference records on all '
			 f'{s.B} rays')


def check_config5_bench_layout(s, sel, r):
	"""Config 5's batch as the bench renders it: 8 lanes per ray in the coherent order of vgr_ray_order (8x8
	direction bins, 7-bit origins), over the whole batch; against the oracle's rays `sel` (results r), and the same
	cells and statistics as the one-ray-per-lane kernel with the thresholds off."""
	order = ext.ray_order(s.t(s.o), s.t(s.d), 8, 7)
	slots = ext.slot_table(s.pack['offsets'], s.pack['nbr'])
	full = s.foam(lanes=8, order=order, slots=slots)
	g = rows(full, sel)
	compare(g, r, stats_frac=0.995, t_max=s.sc.far_radius)
	# the bench's site blocks (record + fp32 SH row in 256 bytes): every output bit-identical
	ei, ai = ext.index_pack(s.pack['offsets'], s.pack['nbr'], s.pack['edge'], s.pack['attr'])
	blocks = torch.cat([ai[:, :16], s.pack['sh'].reshape(-1, 48)], 1).contiguous()
	fb = s.foam(lanes=8, order=order, slots=slots, indexed=(ei, ai, blocks))
	del ei, ai, blocks
	for k in ('rgb', 'T', 'depth', 'stats'):
		np.testing.assert_array_equal(fb[k], full[k], err_msg=k)
	assert psnr(g['rgb'], r['rgb']) >= 60.0
	few = sel[::8]
	g8 = s.foam(few, stage=0, t_thresh=0.0, w_thresh=-1.0, trace_cap=MAX_CELLS + 1, lanes=8)
	g1 = s.foam(few, stage=0, t_thresh=0.0, w_thresh=-1.0, trace_cap=MAX_CELLS + 1, lanes=1)
	np.testing.assert_array_equal(g8['stats'], g1['stats'])
	np.testing.assert_array_equal(g8['trace'], g1['trace'])
	progress(f'[stated sizes] config 5, 8 lanes per ray in coherent order over {s.B} rays: max |rgb| '
			 f'{np.abs(g["rgb"] - r["rgb"]).max():.2e} on {len(sel)} oracle rays; cells identical to one ray per lane')


def test_foam_traces_and_exact_colours(stated):
	"""On the subset: the fused render's cell sequences (common prefixes with the thresholds on), exact colours
	within 1e-4 both as two passes and as the one-pass blend (indexed records with the slot table, the path of
	render_rays_foam_infer on an index_pack'ed pack), and with the thresholds off the stage-0 traversal and the full
	stage-2 render bit-exact in their cells with every statistic equal."""
	s = stated
	sel = s.subset(SUBSET[s.config])
	g = s.foam(sel, trace_cap=2048)
	r = s.oracle(sel, trace_cap=2048)
	compare(g, r, exact_trace=False, stats_frac=0.995, t_max=s.sc.far_radius)
	g = s.foam(sel, mode=0)
	r = s.oracle(sel, mode=0)
	compare(g, r, stats_frac=0.995, t_max=s.sc.far_radius)
	assert psnr(g['rgb'], r['rgb']) >= 60.0
	p = s.pack
	idx = ext.index_pack(p['offsets'], p['nbr'], p['edge'], p['attr'])
	blend = s.foam(sel, mode=0, indexed=idx, slots=ext.slot_table(p['offsets'], p['nbr']))
	del idx
	compare(blend, r, stats_frac=0.995, t_max=s.sc.far_radius)
	assert psnr(blend['rgb'], r['rgb']) >= 60.0
	same = (blend['stats'] == g['stats']).all(1)
	np.testing.assert_allclose(blend['rgb'][same], g['rgb'][same], atol=1e-5, rtol=0)
	progress(f'[stated sizes] config {s.config}: exact colours, two passes / one-pass blend against the oracle on '
			 f'{len(sel)} rays: max |rgb| {np.abs(g["rgb"] - r["rgb"]).max():.2e} / '
			 f'{np.abs(blend["rgb"] - r["rgb"]).max():.2e}')
	few = sel[::8]
	for stage in (0, 2):
		g = s.foam(few, stage=stage, t_thresh=0.0, w_thresh=-1.0, trace_cap=MAX_CELLS + 1)
		r = s.oracle(few, stage=stage, t_thresh=0.0, w_thresh=-1.0, trace_cap=MAX_CELLS + 1)
		compare(g, r, t_max=s.sc.far_radius)
		np.testing.assert_array_equal(g['stats'], r['stats'])
	progress(f'[stated sizes] config {s.config}: thresholds off, {len(few)} rays, mean {g["stats"][:, 0].mean():.0f} '
		  f'cells per ray, cell sequences bit-exact')


@pytest.fixture(scope='module')
def config5_field(gpu):
	if 5 not in stated_configs():
		pytest.skip('config 5 not selected (VGR_STATED_CONFIGS)')
	wait_for_geometry(5)
	sc = scenes.make_scene(5, log=None)
	model = VoronoiGaussField.from_scene(sc, gpu)
	dt, n_bg = 1 / 512, 64
	dA = ext.conic(model.d_log_scale, model.d_quat, 0.5 * dt)
	cA = ext.conic(model.c_log_scale, model.c_quat, 0.5 * dt)
	o, d, start, _ = sc.camera_rays()
	near, mid, far = ray_bounds_np(o, d, 0.02, sc.far_radius)
	host = dict(points=sc.points, offsets=sc.offsets, adj=sc.adj, raw=sc.raw, dA=dA.cpu().numpy(),
				cA=cA.cpu().numpy(), sh=sc.sh)
	yield sc, model, dA, cA, (o, d, start, near, mid, far), host, dt, n_bg
	torch.cuda.empty_cache()


def march_gpu(dev, model, dA, cA, sh_deg, rays, dt, n_bg, t_thresh=1e-4, w_thresh=1e-4, trace_cap=0, lanes=0):
	g = model.graph
	rt = [torch.as_tensor(np.ascontiguousarray(a), device=dev) for a in rays]
	out = ext.march_extension().march_forward(g.points, g.offsets, g.adj, model.raw.detach(), dA, cA,
											  model.sh().detach().contiguous(), sh_deg, *rt, dt, n_bg, t_thresh,
											  w_thresh, trace_cap=trace_cap, lanes=lanes)
	torch.cuda.synchronize()
	return [x.cpu().numpy() for x in out]


def test_march_config5_full_batch(gpu, config5_field):
	"""march_forward over all 16,777,216 rays of config 5 in the default layout, the oracle on every k-th ray; the
	walked sites of that subset bit-exact (one ray per lane forced, the layout of the full batch)."""
	sc, model, dA, cA, rays, host, dt, n_bg = config5_field
	B = len(rays[0])
	rgb, T, depth, stats = march_gpu(gpu, model, dA, cA, sc.sh_deg, rays, dt, n_bg)
	sel = np.arange(511, B, B // 16384, dtype=np.int64)
	r = oracle.march_forward(host['points'], host['offsets'], host['adj'], host['raw'], host['dA'], host['cA'],
							 host['sh'], sc.sh_deg, *rays, dt, n_bg, rays=sel)
	same = (stats[sel] == r['stats']).all(1)
	progress(f'[stated sizes] config 5 march: {B} rays, oracle on {len(sel)}: max |rgb| '
		  f'{np.abs(rgb[sel] - r["rgb"]).max():.2e}, max |T| {np.abs(T[sel] - r["T"]).max():.2e}, stats equal on '
		  f'{same.mean():.5f}, mean samples {stats[:, 0].mean():.1f}')
	np.testing.assert_allclose(rgb[sel], r['rgb'], atol=TOL, rtol=0)
	np.testing.assert_allclose(T[sel], r['T'], atol=TOL, rtol=0)
	assert same.mean() >= 0.995
	few = sel[::16]
	sub = tuple(a[few] for a in rays)
	_, _, _, st, tr = march_gpu(gpu, model, dA, cA, sc.sh_deg, sub, dt, n_bg, trace_cap=2048, lanes=1)
	rt = oracle.march_forward(host['points'], host['offsets'], host['adj'], host['raw'], host['dA'], host['cA'],
							  host['sh'], sc.sh_deg, *sub, dt, n_bg, trace_cap=2048)
	n = np.minimum(np.minimum(st[:, 0], rt['stats'][:, 0]), 2048)
	for i in range(len(few)):
		np.testing.assert_array_equal(tr[i, :n[i]], rt['trace'][i, :n[i]])
	# thresholds off: every sample of every ray, sites and counts identical
	sub = tuple(a[few[:128]] for a in rays)
	_, _, _, st, tr = march_gpu(gpu, model, dA, cA, sc.sh_deg, sub, dt, n_bg, 0.0, -1.0, trace_cap=4096, lanes=1)
	rt = oracle.march_forward(host['points'], host['offsets'], host['adj'], host['raw'], host['dA'], host['cA'],
							  host['sh'], sc.sh_deg, *sub, dt, n_bg, 0.0, -1.0, trace_cap=4096)
	np.testing.assert_array_equal(st, rt['stats'])
	np.testing.assert_array_equal(tr, rt['trace'])


OFF_BARS = {'raw': 2e-5, 'dA': 2e-5, 'cA': 2e-4, 'sh': 2e-4}
ON_BARS = {'raw': 1e-4, 'dA': 1e-4, 'cA': 2e-4, 'sh': 2e-4}


@pytest.mark.parametrize('t_thresh,w_thresh,bars', [(0.0, -1.0, OFF_BARS), (1e-4, 1e-4, ON_BARS)])
def test_march_backward_config5_default_layout(gpu, config5_field, t_thresh, w_thresh, bars):
	"""march_backward over 524,288 rays of config 5 (one ray per lane, the default at this size, forward and
	backward) with upstream gradients on every 256th ray: against the oracle's backward over those rays.

	Bars (relative error, vector norm), thresholds off: density gradients (raw, dA) 2e-5, what fp32 atomics against
	sequential sums leave. Colour gradients (cA, sh) 2e-4: they scale with each sample's weight w = T (1 - exp(-s d)),
	and config 5's sigma delta is about 1e-4, where 1 - exp(-x) (the reference's formula, march.cu:241) keeps only
	about 3 significant digits in fp32, so the ulp by which the device exp and the host's libm exp differ moves w by
	up to 6e-4 relative per sample (measured: about 5e-5 over the batch, the same in both GPU layouts, which agree
	with each other to 1.5e-6). Thresholds on: also a few samples whose weight is within ulps of w_thresh are
	coloured on one side only, 1e-4 for the density gradients."""
	sc, model, dA, cA, rays, host, dt, n_bg = config5_field
	B = 524288
	sub = tuple(np.ascontiguousarray(a[:B]) for a in rays)
	g = model.graph
	rt = [torch.as_tensor(a, device=gpu) for a in sub]
	sh = model.sh().detach().contiguous()
	fx = ext.march_extension()
	rgb, T, _, _ = fx.march_forward(g.points, g.offsets, g.adj, model.raw.detach(), dA, cA, sh, sc.sh_deg, *rt, dt,
									n_bg, t_thresh, w_thresh)
	rng = np.random.default_rng(11)
	g_rgb = np.zeros((B, 3), np.float32)
	g_T = np.zeros(B, np.float32)
	hot = np.arange(0, B, 256)
	g_rgb[hot] = rng.normal(size=(len(hot), 3))
	g_T[hot] = rng.normal(size=len(hot))
	got = fx.march_backward(g.points, g.offsets, g.adj, model.raw.detach(), dA, cA, sh, sc.sh_deg, *rt, dt, n_bg,
							t_thresh, w_thresh, rgb, T, torch.as_tensor(g_rgb, device=gpu),
							torch.as_tensor(g_T, device=gpu))
	torch.cuda.synchronize()
	ref = oracle.march_backward(host['points'], host['offsets'], host['adj'], host['raw'], host['dA'], host['cA'],
								host['sh'], sc.sh_deg, *[a[hot] for a in sub], dt, n_bg, rgb.cpu().numpy()[hot],
								T.cpu().numpy()[hot], g_rgb[hot], g_T[hot], t_thresh, w_thresh)
	errs = {name: rel(a.cpu().numpy(), r) for name, a, r in zip(('raw', 'dA', 'cA', 'sh'), got, ref)}
	progress(f'[stated sizes] config 5 march backward (t_thresh {t_thresh}, w_thresh {w_thresh}), {B} rays, '
		  f'{len(hot)} with gradients: relative errors {errs}')
	for name, e in errs.items():
		assert e < bars[name], name
