"""Pins the CPU oracle (oracle/vgr_oracle.c) against independent checks: float64 dense references restated from
the reference tests, brute-force nearest sites, the segment-in-cell invariant, closed forms and invariances.
No GPU is used here."""

import numpy as np
import pytest

import dense
import oracle
from helpers import Field

INF = float('inf')


@pytest.fixture(scope='module')
def foam_case(oracle_lib):
	"""test_foam.py:41-59 setup: 300 sites in [-0.9, 0.9]^3 (seed 2), 64 rays from [-0.5, 0.5]^3, far_radius 2."""
	f = Field(seed=2, n=300)
	return f, f.pack(), f.rays(B=64, seed=2)


def run_foam(f, pk, rays, trace_cap=4096, **kw):
	o, d, start, near, _, far = rays
	args = dict(t_thresh=0.0, w_thresh=-1.0)
	args.update(kw)
	return oracle.foam_infer(pk, f.sh_deg, o, d, start, near, far, trace_cap=trace_cap, **args)


def test_foam_traversal_matches_float64_retrace(foam_case):
	"""Visited cells = the float64 bisector-plane re-trace (test_foam.py:18-37) on (almost) every ray."""
	f, pk, rays = foam_case
	o, d, start, near, _, far = rays
	out = run_foam(f, pk, rays, stage=0)
	same = 0
	for r in range(len(o)):
		x0 = o[r].astype(np.float64) + near[r] * d[r].astype(np.float64)
		t, cells = dense.trace(f.points, f.offsets, f.adj, o[r].astype(np.float64), d[r].astype(np.float64),
							   float(near[r]), float(far[r]), f.tree.query(x0)[1])
		n = out['stats'][r, 0]
		same += n == len(cells) and list(out['trace'][r, :n]) == list(cells)
	assert same >= 0.95 * len(o), f'{same}/{len(o)} rays with identical cell sequences'


def test_foam_segments_inside_their_cells(foam_case):
	"""Every segment longer than 1e-6 has its midpoint in the attributed cell (test_foam.py:85-88)."""
	f, pk, rays = foam_case
	o, d, start, near, _, far = rays
	out = run_foam(f, pk, rays, stage=0)
	bad = total = 0
	for r in range(len(o)):
		n = out['stats'][r, 0]
		cells = out['trace'][r, :n]
		# re-derive the sample parameters from the cell sequence: the exit of cell i towards cell i + 1
		t = [float(near[r])]
		for a, b in zip(cells[:-1], cells[1:]):
			if a == b:
				t.append(float(far[r]))
				continue
			pa, pb = f.points[a].astype(np.float64), f.points[b].astype(np.float64)
			nrm = pb - pa
			tt = ((0.5 * (pa + pb) - o[r]) @ nrm) / (nrm @ d[r])
			t.append(max(tt, t[-1]))
		t = np.array(t)
		mids = o[r][None] + 0.5 * (t[1:] + t[:-1])[:, None] * d[r][None]
		long_enough = t[1:] - t[:-1] > 1e-6
		bad += int((f.tree.query(mids)[1] != cells[:-1])[long_enough].sum())
		total += int(long_enough.sum())
	assert total > 300
	assert bad <= total * 1e-3, f'{bad} / {total} segments outside their cell'


@pytest.mark.parametrize('mode', [0, 2])
def test_foam_values_match_float64_dense(foam_case, mode):
	"""rgb and T against the float64 dense reference (test_foam.py:76-104), thresholds off, on the rays whose
	traversal agrees with the float64 re-trace."""
	f, pk, rays = foam_case
	o, d, start, near, _, far = rays
	out = run_foam(f, pk, rays, stage=2, color_mode=mode)
	checked = 0
	for r in range(len(o)):
		o64, d64 = o[r].astype(np.float64), d[r].astype(np.float64)
		x0 = o64 + near[r] * d64
		t, cells = dense.trace(f.points, f.offsets, f.adj, o64, d64, float(near[r]), float(far[r]),
							   f.tree.query(x0)[1])
		n = out['stats'][r, 0]
		if n != len(cells) or list(out['trace'][r, :n]) != list(cells):
			continue
		rgb, T = dense.foam_dense(f.points, f.offsets, f.adj, f.raw.astype(np.float64), pk['dA'].astype(np.float64),
								  pk['cA'].astype(np.float64), f.sh.astype(np.float64), f.sh_deg, o64, d64, t, cells)
		np.testing.assert_allclose(out['rgb'][r], rgb, atol=2e-5, rtol=1e-4)
		np.testing.assert_allclose(out['T'][r], T, atol=2e-6, rtol=1e-4)
		checked += 1
	assert checked >= 0.95 * len(o)


def test_foam_lazy_equals_fused_and_cache_is_transparent(foam_case):
	f, pk, rays = foam_case
	lazy = run_foam(f, pk, rays, stage=2, color_mode=0, t_thresh=1e-4, w_thresh=1e-4)
	fused = run_foam(f, pk, rays, stage=2, color_mode=2, t_thresh=1e-4, w_thresh=1e-4)
	np.testing.assert_allclose(lazy['rgb'], fused['rgb'], atol=1e-5)
	np.testing.assert_array_equal(lazy['T'], fused['T'])
	nocache = run_foam(f, pk, rays, stage=2, color_mode=0, t_thresh=1e-4, w_thresh=1e-4, use_cache=False)
	for k in ('rgb', 'T', 'depth'):
		np.testing.assert_array_equal(lazy[k], nocache[k])
	np.testing.assert_array_equal(lazy['stats'][:, :4], nocache['stats'][:, :4])
	assert (nocache['stats'][:, 4] >= lazy['stats'][:, 4]).all()
	assert nocache['stats'][:, 4].sum() > lazy['stats'][:, 4].sum()


def direct_mapped_misses(keys, slots=8):
	"""Misses of a direct-mapped cache of `slots` slots keyed by k mod slots that holds the last key of each slot."""
	held = [-1] * slots
	miss = 0
	for k in keys:
		s = k % slots
		miss += held[s] != k
		held[s] = k
	return miss


@pytest.mark.parametrize('mode', [0, 2])
@pytest.mark.parametrize('reorder', [False, True])
def test_foam_cache_miss_count_is_a_direct_mapped_cache(foam_case, mode, reorder):
	"""stats[:, 4] with the cache on is the miss count of an 8-slot direct-mapped cache keyed by k & 7
	(foam_infer.cu:151-168) over the ray's colour lookups. With the thresholds off and no colour cut-off the
	lookups are, in both colour modes, every neighbourhood entry (self first, CSR order) of every sample's cell in
	sample order, so the count follows from the cell trace alone; without the cache every lookup counts."""
	f, _, rays = foam_case
	pk = f.pack(reorder=reorder)
	o, d, start, near, _, far = rays
	st = pk['inv'][start].astype(np.int32) if reorder else start
	out = oracle.foam_infer(pk, f.sh_deg, o, d, st, near, far, 0.0, -1.0, color_mode=mode, trace_cap=4096)
	every = oracle.foam_infer(pk, f.sh_deg, o, d, st, near, far, 0.0, -1.0, color_mode=mode, use_cache=False)
	inv = pk['inv'] if reorder else np.arange(f.n)
	offsets, nbr = pk['offsets'], pk['nbr']
	for r in range(len(o)):
		n = out['stats'][r, 0]
		cells = inv[out['trace'][r, :n]]  # trace in original numbering -> the pack's numbering
		keys = [int(k) for c in cells for k in nbr[offsets[c]:offsets[c + 1]]]
		assert every['stats'][r, 4] == len(keys)
		assert out['stats'][r, 4] == direct_mapped_misses(keys), f'ray {r}'
	assert out['stats'][:, 4].sum() < every['stats'][:, 4].sum()


def test_foam_morton_reorder_is_invariant(foam_case):
	"""Renumbering the sites (Z-order, render.py:213-222) changes nothing but the cache statistics: same values
	bit for bit and the same cell sequences in original numbering."""
	f, pk, rays = foam_case
	pr = f.pack(reorder=True)
	o, d, start, near, _, far = rays
	base = run_foam(f, pk, rays, stage=2, t_thresh=1e-4, w_thresh=1e-4)
	re = oracle.foam_infer(pr, f.sh_deg, o, d, pr['inv'][start], near, far, 1e-4, 1e-4, trace_cap=4096)
	for k in ('rgb', 'T', 'depth', 'trace'):
		np.testing.assert_array_equal(base[k], re[k])
	np.testing.assert_array_equal(base['stats'][:, :4], re['stats'][:, :4])


def test_foam_stages_and_cap_keep_the_traversal(foam_case):
	"""STAGE 0/1 with cap = the full renderer's sample counts visit the same cells (bench_infer.py:72-79); the
	capped last sample is x(far) in the current cell, where an early-stopped ray's last sample is a crossing."""
	f, pk, rays = foam_case
	full = run_foam(f, pk, rays, stage=2, t_thresh=1e-2, w_thresh=1e-4)
	cap = full['stats'][:, 0].copy()
	for stage in (0, 1):
		s = run_foam(f, pk, rays, stage=stage, t_thresh=1e-2, cap=cap)
		np.testing.assert_array_equal(s['stats'][:, 0], cap)
		for r in range(len(cap)):
			np.testing.assert_array_equal(s['trace'][r, :cap[r] - 1], full['trace'][r, :cap[r] - 1])
		assert (s['rgb'] == 0).all()
		if stage == 0:
			assert (s['T'] == 1).all() and (s['stats'][:, 3] == 0).all()
		else:
			assert (s['T'] < 1).all() and (s['stats'][:, 3] > 0).all()


def test_foam_zero_density_and_opaque_special_cases(oracle_lib):
	f = Field(seed=5, n=200)
	o, d, start, near, _, far = f.rays(B=32, seed=5)
	f.raw[:] = -100.0  # rho = e^-100: no absorption
	pk = f.pack()
	out = oracle.foam_infer(pk, f.sh_deg, o, d, start, near, far, 0.0, -1.0)
	np.testing.assert_allclose(out['T'], 1.0, atol=1e-6)
	np.testing.assert_allclose(out['rgb'], 0.0, atol=1e-6)
	f.raw[:] = 12.0  # extremely dense everywhere: opaque within the first segment
	pk = f.pack()
	out = oracle.foam_infer(pk, f.sh_deg, o, d, start, near, far, 1e-4, 1e-4)
	assert (out['T'] < 1e-4).all()
	assert (out['stats'][:, 0] <= 4).all()


def test_foam_sh_degree0_colour_closed_form(oracle_lib):
	"""Degree 0 and identical sites' colours: every blend is max(1/2 + 0.28209479 sh0, 0) whatever the weights."""
	f = Field(seed=6, n=200, sh_deg=0)
	f.sh[:, 0] = np.array([0.4, -0.2, -3.0], np.float32)
	pk = f.pack()
	o, d, start, near, _, far = f.rays(B=32, seed=6)
	out = oracle.foam_infer(pk, 0, o, d, start, near, far, 0.0, -1.0)
	c = np.maximum(0.5 + 0.28209479177387814 * np.array([0.4, -0.2, -3.0]), 0)
	np.testing.assert_allclose(out['rgb'], (1 - out['T'])[:, None] * c[None], atol=2e-6)


def test_foam_baked_colours_closed_forms(foam_case):
	"""Baked colours (foam_infer.cu:242-244), pinned without the oracle's SH path: (a) one colour c baked into every
	site gives rgb = c (1 - T), blends of equal colours; (b) arbitrary per-site colours against foam_dense blending
	the same colours in float64; (c) colours baked as max(1/2 + 0.28209479 sh0, 0) give what the fused mode
	computes from degree-0 SH, which depends on no direction."""
	f, pk0, rays = foam_case
	o, d, start, near, _, far = rays
	pk = dict(pk0, attr=pk0['attr'].copy())
	c = np.array([0.3, 0.8, 0.05], np.float32)
	pk['attr'][:, 16:19] = c
	out = oracle.foam_infer(pk, 3, o, d, start, near, far, 0.0, -1.0, color_mode=1, trace_cap=4096)
	np.testing.assert_allclose(out['rgb'], (1 - out['T'])[:, None] * c[None], atol=2e-6)
	assert (out['stats'][:, 4] == 0).all()  # no SH evaluation in baked mode
	colours = np.random.default_rng(9).uniform(0, 1, (f.n, 3)).astype(np.float32)
	pk['attr'][:, 16:19] = colours
	out = oracle.foam_infer(pk, 3, o, d, start, near, far, 0.0, -1.0, color_mode=1, trace_cap=4096)
	dense_check(f, pk, rays, out, baked=colours)
	g = Field(seed=7, n=250, sh_deg=0)
	o, d, start, near, _, far = g.rays(B=48, seed=7)
	pk = g.pack()
	pk['attr'][:, 16:19] = np.maximum(0.5 + np.float32(0.28209479177387814) * g.sh[:, 0], 0)
	baked = oracle.foam_infer(pk, 0, o, d, start, near, far, 0.0, -1.0, color_mode=1)
	fused = oracle.foam_infer(pk, 0, o, d, start, near, far, 0.0, -1.0, color_mode=2, use_cache=False)
	np.testing.assert_allclose(baked['rgb'], fused['rgb'], atol=2e-6)
	np.testing.assert_array_equal(baked['T'], fused['T'])
	np.testing.assert_array_equal(baked['stats'][:, :4], fused['stats'][:, :4])


def dense_check(f, pk, rays, out, atol=2e-5, **kw):
	"""The oracle's rgb and T against foam_dense (float64, same mode options) on every ray whose cells agree with
	the float64 re-trace (at least 95 % of them)."""
	o, d, start, near, _, far = rays
	checked = 0
	for r in range(len(o)):
		o64, d64 = o[r].astype(np.float64), d[r].astype(np.float64)
		t, cells = dense.trace(f.points, f.offsets, f.adj, o64, d64, float(near[r]), float(far[r]),
							   f.tree.query(o64 + near[r] * d64)[1])
		n = out['stats'][r, 0]
		if n != len(cells) or list(out['trace'][r, :n]) != list(cells):
			continue
		rgb, T = dense.foam_dense(f.points, f.offsets, f.adj, f.raw.astype(np.float64), pk['dA'].astype(np.float64),
								  pk['cA'].astype(np.float64), f.sh.astype(np.float64), f.sh_deg, o64, d64, t, cells,
								  **kw)
		np.testing.assert_allclose(out['rgb'][r], rgb, atol=atol, rtol=1e-4)
		np.testing.assert_allclose(out['T'][r], T, atol=2e-6, rtol=1e-4)
		checked += 1
	assert checked >= 0.95 * len(o)


@pytest.mark.parametrize('mode', [0, 2])
def test_foam_eps_color_matches_float64_dense(foam_case, mode):
	"""A finite colour cut (foam_infer.cu:236,240,271,276) against foam_dense applying the same rule in float64:
	exact mode keeps m <= m_min + cut, fused mode m <= (running minimum in neighbourhood order) + cut. The cut
	must drop terms (fewer SH evaluations) and change the colours; transmittance and cells stay unchanged."""
	f, pk, rays = foam_case
	cut = 2 * np.log(1 / 1e-2)
	exact = run_foam(f, pk, rays, stage=2, color_mode=mode, use_cache=False)
	out = run_foam(f, pk, rays, stage=2, color_mode=mode, use_cache=False, color_cut=cut)
	np.testing.assert_array_equal(out['T'], exact['T'])
	np.testing.assert_array_equal(out['trace'], exact['trace'])
	assert out['stats'][:, 4].sum() < 0.8 * exact['stats'][:, 4].sum()
	assert np.abs(out['rgb'] - exact['rgb']).max() > 1e-4
	dense_check(f, pk, rays, out, color_cut=cut, fused=mode == 2)


def test_foam_eps_density_matches_float64_dense(oracle_lib):
	"""eps_density (foam_infer.cu:229, render.py:191-197): against foam_dense dropping a term where |x - p_j|^2 >
	r2_j (the half-precision r2 of the pack); and the bound the rule exists for: a dropped term is
	rho_j G_j(x) <= exp(raw_j - |v|^2 / (2 s_max^2)) < eps, so T rises by at most a factor exp(eps E_max (far - near))
	over the exact render's."""
	f = Field(seed=8, n=300, raw_mu=0.5)
	rays = f.rays(B=48, seed=8)
	o, d, start, near, _, far = rays
	eps = 0.05
	exact = oracle.foam_infer(f.pack(), 3, o, d, start, near, far, 0.0, -1.0, trace_cap=4096)
	pk = f.pack(eps_density=eps)
	out = oracle.foam_infer(pk, 3, o, d, start, near, far, 0.0, -1.0, trace_cap=4096)
	np.testing.assert_array_equal(out['trace'], exact['trace'])
	assert out['stats'][:, 3].sum() < 0.9 * exact['stats'][:, 3].sum()  # terms were dropped
	tol = 1e-6 * (1 + exact['T'])
	assert (out['T'] >= exact['T'] - tol).all() and (out['T'] > exact['T'] + 1e-6).any()
	e_max = int(np.diff(pk['offsets']).max())
	assert (out['T'] <= exact['T'] * np.exp(eps * e_max * (far - near)) + tol).all()
	r2 = np.empty(f.n)
	r2[pk['nbr']] = (pk['edge'][:, 3].view(np.uint32) & 0xFFFF).astype(np.uint16).view(np.float16)
	dense_check(f, pk, rays, out, r2=r2)


def test_fp16_sh_oracle_close_to_fp32(foam_case):
	f, pk, rays = foam_case
	ph = f.pack(sh_half=True)
	a = run_foam(f, pk, rays, stage=2)
	b = run_foam(f, ph, rays, stage=2)
	np.testing.assert_allclose(a['rgb'], b['rgb'], atol=2e-3)
	np.testing.assert_array_equal(a['T'], b['T'])


# ------------------------------------------------------------------------------------------- march

def test_march_matches_float64_dense(oracle_lib):
	"""test_march.py:33-79: 300 sites (seed 1), B=64, dt=0.05, n_bg=8, conic floor 0.01, thresholds off."""
	f = Field(seed=1, n=300)
	o, d, start, near, mid, far = f.rays(B=64, seed=1)
	dA, cA = f.conics(0.01)
	out = oracle.march_forward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, o, d, start, near, mid, far, 0.05,
							   8, t_thresh=0.0, w_thresh=-1.0)
	rgb = np.zeros((64, 3))
	T = np.zeros(64)
	for r in range(64):
		rgb[r], T[r] = dense.march_dense(f.points, f.offsets, f.adj, f.raw.astype(np.float64), dA.astype(np.float64),
										 cA.astype(np.float64), f.sh.astype(np.float64), 3, o[r].astype(np.float64),
										 d[r].astype(np.float64), float(near[r]), float(mid[r]), float(far[r]), 0.05, 8,
										 tree=f.tree)
	rel = np.linalg.norm(out['rgb'] - rgb) / np.linalg.norm(rgb)
	assert rel < 1e-4, rel
	np.testing.assert_allclose(out['T'], T, atol=1e-5, rtol=1e-4)
	n_in = np.where(mid > near, np.ceil((mid - near) / 0.05), 0).astype(int)
	np.testing.assert_array_equal(out['stats'][:, 0], n_in + 8)


def test_march_sample_positions_closed_form(oracle_lib):
	for near, mid, far, dt, n_bg in ((0.02, 1.3, 3.5, 0.05, 8), (0.02, 0.021, 2.0, 1 / 512, 64)):
		n_in = int(np.ceil(np.float32(np.float32(mid) - np.float32(near)) / np.float32(dt)))
		t_ref, dl_ref = dense.march_samples(near, mid, far, dt, n_bg)
		for k in range(n_in + n_bg):
			t, dl = oracle.sample_at(near, mid, far, n_in, dt, n_bg, k)
			assert abs(t - t_ref[k]) <= 2e-6 * max(1, t_ref[k]) and abs(dl - dl_ref[k]) <= 2e-6


def test_march_walk_sites_are_nearest(oracle_lib):
	f = Field(seed=3, n=400)
	o, d, start, near, mid, far = f.rays(B=32, seed=3)
	dA, cA = f.conics(0.01)
	out = oracle.march_forward(f.points, f.offsets, f.adj, f.raw, dA, cA, f.sh, 3, o, d, start, near, mid, far, 0.05,
							   8, 0.0, -1.0, trace_cap=512)
	ok = total = 0
	for r in range(32):
		t, _ = dense.march_samples(float(near[r]), float(mid[r]), float(far[r]), 0.05, 8)
		X = o[r][None].astype(np.float64) + t[:, None] * d[r][None]
		nn = f.tree.query(X)[1]
		n = out['stats'][r, 0]
		ok += int((out['trace'][r, :n] == nn[:n]).sum())
		total += n
	assert ok >= 0.999 * total


# ----------------------------------------------------------------------------------- vgf operators

def test_walk_is_exact_nearest_neighbour(oracle_lib):
	"""test_grad.py:61-72: 400 sites in [-1, 1]^3 (seed 0), 500 rays x 40 sorted samples."""
	f = Field(seed=0, n=400, lo=-1.0, hi=1.0)
	rng = np.random.default_rng(7)
	o = rng.uniform(-1.2, 1.2, (500, 3)).astype(np.float32)
	d = rng.normal(size=(500, 3))
	d = (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)
	z = np.sort(rng.uniform(0, 2.5, (500, 40)), 1).astype(np.float32)
	start = f.tree.query(o)[1].astype(np.int32)
	site, steps = oracle.walk(f.points, f.offsets, f.adj, o, d, z, start)
	x = (o[:, None].astype(np.float64) + d[:, None] * z[..., None]).reshape(-1, 3)
	dist_walk = np.linalg.norm(x - f.points[site.ravel()], axis=1)
	dist_nn, _ = f.tree.query(x)
	assert np.mean(dist_walk <= dist_nn + 1e-6) > 0.999
	assert steps.sum() > 0


def test_density_and_color_match_float64_dense(oracle_lib):
	"""test_grad.py:74-109: 3000 random samples with their nearest site."""
	f = Field(seed=0, n=400, lo=-1.0, hi=1.0, raw_mu=0.0, ls_mu=-1.2)
	rng = np.random.default_rng(8)
	x = rng.uniform(-1, 1, (3000, 3)).astype(np.float32)
	site = f.tree.query(x)[1].astype(np.int32)
	dirs = rng.normal(size=(3000, 3)).astype(np.float32)
	for mult in (1.0, 4.0):
		sig = oracle.density(f.points, f.offsets, f.adj, f.raw, f.d_log_scale, f.d_quat, x, site, mult)
		ref = dense.density_dense(f.points, f.offsets, f.adj, f.raw.astype(np.float64), f.d_log_scale, f.d_quat, x,
								  site, mult)
		assert np.linalg.norm(sig - ref) / np.linalg.norm(ref) < 1e-5
	for deg in (0, 3):
		rgb = oracle.color(f.points, f.offsets, f.adj, f.c_log_scale, f.c_quat, f.sh, deg, x, dirs, site)
		ref = dense.color_dense(f.points, f.offsets, f.adj, f.c_log_scale, f.c_quat, f.sh.astype(np.float64), deg, x,
								dirs, site)
		assert np.linalg.norm(rgb - ref) / np.linalg.norm(ref) < 1e-5


def test_conic_closed_form(oracle_lib):
	rng = np.random.default_rng(9)
	ls = rng.normal(-1.5, 0.5, (200, 3)).astype(np.float32)
	q = rng.normal(size=(200, 4)).astype(np.float32)
	for floor in (0.0, 0.01):
		A = oracle.conic(ls, q, floor)
		np.testing.assert_allclose(A, dense.conic_dense(ls, q, floor), rtol=2e-5, atol=1e-4)
	# A Sigma = I with Sigma = R diag(s^2) R^T built independently
	A = oracle.conic(ls, q).astype(np.float64)
	R = dense.quat_rot(q)
	Sig = np.einsum('nak,nk,nbk->nab', R, np.exp(2 * ls.astype(np.float64)), R)
	Af = A[:, [0, 1, 2, 1, 3, 4, 2, 4, 5]].reshape(-1, 3, 3)
	np.testing.assert_allclose(Af @ Sig, np.broadcast_to(np.eye(3), Af.shape), atol=5e-4)
	# identity rotation: diag(1 / (s^2 + floor^2))
	qi = np.tile(np.array([1, 0, 0, 0], np.float32), (200, 1))
	A = oracle.conic(ls, qi, 0.1)
	np.testing.assert_allclose(A[:, [0, 3, 5]], 1 / (np.exp(2 * ls.astype(np.float64)) + 0.01), rtol=1e-5)
	assert np.abs(A[:, [1, 2, 4]]).max() == 0


def test_sh_basis_known_values_and_orthonormality(oracle_lib):
	b = oracle.sh_basis([0.0, 0.0, 1.0], 3)
	expect = np.zeros(16)
	expect[[0, 2, 6, 12]] = [0.28209479, 0.48860251, 0.63078313, 0.74635267]
	np.testing.assert_allclose(b, expect, atol=1e-7)
	for v in ([1, 0, 0], [0.6, -0.8, 0]):
		assert abs(oracle.sh_basis(v, 3)[0] - 0.28209479) < 1e-7
	# orthonormal on the sphere: 4 pi E[b_i b_j] = delta_ij (Fibonacci quadrature)
	m = 20000
	i = np.arange(m) + 0.5
	phi, z = np.pi * (1 + 5 ** 0.5) * i, 1 - 2 * i / m
	r = np.sqrt(1 - z * z)
	dirs = np.stack([r * np.cos(phi), r * np.sin(phi), z], 1)
	B = np.stack([oracle.sh_basis(v, 3) for v in dirs[::4]]).astype(np.float64)
	G = 4 * np.pi * B.T @ B / len(B)
	np.testing.assert_allclose(G, np.eye(16), atol=2e-3)


def test_nearest_brute_matches_ckdtree_and_closed_forms():
	"""nearest_brute (the start-cell oracle) against scipy's cKDTree (the reference's nearest_sites, sites.py:38-39)
	on uniform and clustered sites, queries inside and outside the cloud; closed forms on a lattice."""
	from scipy.spatial import cKDTree
	rng = np.random.default_rng(7)
	uni = rng.uniform(-1, 1, (4000, 3)).astype(np.float32)
	clu = (rng.normal(0, 0.05, (4000, 3)) + rng.uniform(-1, 1, (40, 3))[rng.integers(0, 40, 4000)]).astype(np.float32)
	for pts in (uni, clu):
		q = np.concatenate([rng.uniform(-1.2, 1.2, (3000, 3)), rng.normal(0, 4, (200, 3))]).astype(np.float32)
		got = dense.nearest_brute(pts, q)
		ref = cKDTree(pts.astype(np.float64)).query(q.astype(np.float64))[1]
		np.testing.assert_array_equal(got, ref)
	# lattice: the nearest site of a point in an open Voronoi cell of a unit lattice is its rounding
	g = np.stack(np.meshgrid(*[np.arange(5.0)] * 3, indexing='ij'), -1).reshape(-1, 3).astype(np.float32)
	q = rng.uniform(-0.4, 4.4, (500, 3)).astype(np.float32)
	expect = (np.clip(np.rint(q), 0, 4) @ np.array([25, 5, 1])).astype(np.int32)
	np.testing.assert_array_equal(dense.nearest_brute(g, q), expect)
	# equidistant: ties go to the smaller index
	assert dense.nearest_brute(np.array([[1, 0, 0], [-1, 0, 0]], np.float32), np.zeros((1, 3), np.float32))[0] == 0
