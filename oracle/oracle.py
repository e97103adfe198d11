"""ctypes wrapper of liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU oracle (vgr_oracle.c) restates the reference kernels' semantics in plain C; tests/, smoke() and bench.py's
cpu_baseline leg use it as the checker and the CPU baseline. Nothing in the product (voronoi-gauss_amd/) imports
it. Inputs are numpy arrays (C-contiguous, cast here); outputs are numpy arrays.
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'liboracle.so')
_lib = None

_P, _I32, _I64, _F32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float

_SIGS = {
	'oracle_foam_infer': ([_P, _P, _P, _P, _P, _P, _I32, _I32, _P, _P, _P, _P, _P, _P, _I64, _F32, _F32, _F32, _I32,
						   _I32, _P, _P, _I32, _P, _P, _P, _P, _P, _I32, _I32], ctypes.c_double),
	'oracle_march_forward': ([_P, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _F32, _I32, _F32,
							  _F32, _P, _P, _P, _P, _P, _I32, _I32], ctypes.c_double),
	'oracle_march_backward': ([_P, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _I64, _F32, _I32, _F32,
							   _F32, _P, _P, _P, _P, _P, _P, _P, _P], None),
	'oracle_foam_forward': ([_P, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _I64, _F32, _F32, _P, _P, _P, _P,
							 _P, _I32], None),
	'oracle_foam_backward': ([_P, _P, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _I64, _F32, _F32, _P, _P, _P,
							  _P, _P, _P, _P, _P], None),
	'oracle_walk': ([_P, _P, _P, _P, _P, _P, _P, _I64, _I32, _P, _P, _I32], None),
	'oracle_density': ([_P, _P, _P, _P, _P, _P, _P, _P, _I64, _F32, _P, _I32], None),
	'oracle_color': ([_P, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _I64, _P, _I32], None),
	'oracle_conic': ([_P, _P, _I64, _F32, _P], None),
	'oracle_density_backward': ([_P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P], None),
	'oracle_color_backward': ([_P, _P, _P, _P, _P, _P, _I32, _P, _P, _P, _I64, _P, _P, _P, _P, _P], None),
	'oracle_conic_backward': ([_P, _P, _I64, _F32, _P, _P, _P], None),
	'oracle_sh_basis': ([_F32, _F32, _F32, _I32, _P], None),
	'oracle_sample_at': ([_F32, _F32, _F32, _I32, _F32, _I32, _I32, _P, _P], None),
	'oracle_omp_max_threads': ([], ctypes.c_int),
}


def build(force=False):
	"""Compiles liboracle.so with the Makefile next to this file."""
	cmd = ['make', '-s', '-C', HERE] + (['-B'] if force else [])
	subprocess.run(cmd, check=True)
	return LIB_PATH


def load():
	global _lib
	if _lib is None:
		if not os.path.exists(LIB_PATH):
			build()
		lib = ctypes.CDLL(LIB_PATH)
		for name, (args, res) in _SIGS.items():
			fn = getattr(lib, name)
			fn.argtypes, fn.restype = args, res
		_lib = lib
	return _lib


def _a(x, dtype):
	return None if x is None else np.ascontiguousarray(x, dtype=dtype)


def _p(x):
	return None if x is None else x.ctypes.data


def max_threads():
	return load().oracle_omp_max_threads()


def foam_infer(pack, sh_deg, o, d, start, near, far, t_thresh=1e-4, w_thresh=1e-4, color_cut=float('inf'),
			   color_mode=0, stage=2, cap=None, rays=None, use_cache=True, trace_cap=0, n_threads=0):
	"""pack: dict of numpy arrays as render.pack_foam builds (points, offsets, nbr, edge, attr, sh, orig).
	rays: optional int64 selection of ray indices (outputs follow the selection). -> dict rgb, T, depth, stats,
	trace (or None), seconds (wall time of the parallel loop)."""
	pts = _a(pack['points'], np.float32)
	sh = pack.get('sh')
	half = sh is not None and sh.dtype == np.float16
	sh = _a(sh, np.float16 if half else np.float32)
	orig = pack.get('orig')
	orig = _a(orig, np.int32) if orig is not None and len(orig) == len(pts) else None
	o, d = _a(o, np.float32), _a(d, np.float32)
	start, near, far = _a(start, np.int32), _a(near, np.float32), _a(far, np.float32)
	cap = _a(cap, np.int32)
	rays = _a(rays, np.int64)
	n = len(o) if rays is None else len(rays)
	rgb = np.zeros((n, 3), np.float32)
	T = np.zeros(n, np.float32)
	depth = np.zeros(n, np.float32)
	stats = np.zeros((n, 5), np.int32)
	trace = np.full((n, trace_cap), -1, np.int32) if trace_cap > 0 else None
	keep = [pts, sh, orig, o, d, start, near, far, cap, rays]
	offsets, nbr = _a(pack['offsets'], np.int32), _a(pack['nbr'], np.int32)
	edge, attr = _a(pack['edge'], np.float32), _a(pack['attr'], np.float32)
	keep += [offsets, nbr, edge, attr]
	secs = load().oracle_foam_infer(
		_p(pts), _p(offsets), _p(nbr), _p(edge), _p(attr), _p(sh), int(half), int(sh_deg), _p(o), _p(d), _p(start),
		_p(near), _p(far), _p(rays), n, t_thresh, w_thresh, color_cut, int(color_mode), int(stage), _p(cap), _p(orig),
		int(use_cache), _p(rgb), _p(T), _p(depth), _p(stats), _p(trace), int(trace_cap), int(n_threads))
	del keep
	return {'rgb': rgb, 'T': T, 'depth': depth, 'stats': stats, 'trace': trace, 'seconds': secs}


def march_forward(points, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, start, near, mid, far, dt, n_bg,
				  t_thresh=1e-4, w_thresh=1e-4, rays=None, trace_cap=0, n_threads=0):
	"""-> dict rgb, T, depth, stats (B, 3), trace (sites per sample) or None, seconds."""
	arrs = [_a(points, np.float32), _a(offsets, np.int32), _a(adj, np.int32), _a(raw, np.float32),
			_a(dA, np.float32), _a(cA, np.float32), _a(sh, np.float32)]
	ray_arrs = [_a(o, np.float32), _a(d, np.float32), _a(start, np.int32), _a(near, np.float32),
				_a(mid, np.float32), _a(far, np.float32)]
	rays = _a(rays, np.int64)
	n = len(ray_arrs[0]) if rays is None else len(rays)
	rgb = np.zeros((n, 3), np.float32)
	T = np.zeros(n, np.float32)
	depth = np.zeros(n, np.float32)
	stats = np.zeros((n, 3), np.int32)
	trace = np.full((n, trace_cap), -1, np.int32) if trace_cap > 0 else None
	secs = load().oracle_march_forward(*[_p(a) for a in arrs], int(sh_deg), *[_p(a) for a in ray_arrs], _p(rays), n,
									   float(dt), int(n_bg), t_thresh, w_thresh, _p(rgb), _p(T), _p(depth), _p(stats),
									   _p(trace), int(trace_cap), int(n_threads))
	return {'rgb': rgb, 'T': T, 'depth': depth, 'stats': stats, 'trace': trace, 'seconds': secs}


def march_backward(points, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, start, near, mid, far, dt, n_bg, rgb, T,
				   g_rgb, g_T, t_thresh=1e-4, w_thresh=1e-4):
	"""Gradients of the march's rgb and T: -> g_raw (N,), g_dA (N, 6), g_cA (N, 6), g_sh (N, 16, 3)."""
	arrs = [_a(points, np.float32), _a(offsets, np.int32), _a(adj, np.int32), _a(raw, np.float32),
			_a(dA, np.float32), _a(cA, np.float32), _a(sh, np.float32)]
	ray_arrs = [_a(o, np.float32), _a(d, np.float32), _a(start, np.int32), _a(near, np.float32),
				_a(mid, np.float32), _a(far, np.float32)]
	n, B = len(arrs[0]), len(ray_arrs[0])
	g = [np.zeros(n, np.float32), np.zeros((n, 6), np.float32), np.zeros((n, 6), np.float32),
		 np.zeros((n, 16, 3), np.float32)]
	up = [_a(rgb, np.float32), _a(T, np.float32), _a(g_rgb, np.float32), _a(g_T, np.float32)]
	load().oracle_march_backward(*[_p(a) for a in arrs], int(sh_deg), *[_p(a) for a in ray_arrs], B, float(dt),
								 int(n_bg), t_thresh, w_thresh, *[_p(a) for a in up], *[_p(a) for a in g])
	return tuple(g)


def _foam_args(points, offsets, adj, raw, dA, cA, sh, o, d, start, near, far):
	return ([_a(points, np.float32), _a(offsets, np.int32), _a(adj, np.int32), _a(raw, np.float32),
			 _a(dA, np.float32), _a(cA, np.float32), _a(sh, np.float32)],
			[_a(o, np.float32), _a(d, np.float32), _a(start, np.int32), _a(near, np.float32), _a(far, np.float32)])


def foam_forward(points, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, start, near, far, t_thresh=1e-4,
				 w_thresh=1e-4, record_cap=0):
	"""foam.cu training forward -> dict rgb, T, depth, stats (B, 3) [samples, coloured segments, walk steps], rec
	(B, K, 8) or None."""
	arrs, rays = _foam_args(points, offsets, adj, raw, dA, cA, sh, o, d, start, near, far)
	B = len(rays[0])
	rgb, T, depth = np.zeros((B, 3), np.float32), np.zeros(B, np.float32), np.zeros(B, np.float32)
	stats = np.zeros((B, 3), np.int32)
	rec = np.zeros((B, record_cap, 8), np.float32) if record_cap > 0 else None
	load().oracle_foam_forward(*[_p(x) for x in arrs], int(sh_deg), *[_p(x) for x in rays], B, t_thresh, w_thresh,
							   _p(rgb), _p(T), _p(depth), _p(stats), _p(rec), int(record_cap))
	return {'rgb': rgb, 'T': T, 'depth': depth, 'stats': stats, 'rec': rec}


def foam_backward(points, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, start, near, far, rgb, T, g_rgb, g_T,
				  t_thresh=1e-4, w_thresh=1e-4):
	"""foam.cu training backward -> g_raw (N,), g_dA (N, 6), g_cA (N, 6), g_sh (N, 16, 3)."""
	arrs, rays = _foam_args(points, offsets, adj, raw, dA, cA, sh, o, d, start, near, far)
	n, B = len(arrs[0]), len(rays[0])
	g = [np.zeros(n, np.float32), np.zeros((n, 6), np.float32), np.zeros((n, 6), np.float32),
		 np.zeros((n, 16, 3), np.float32)]
	up = [_a(rgb, np.float32), _a(T, np.float32), _a(g_rgb, np.float32), _a(g_T, np.float32)]
	load().oracle_foam_backward(*[_p(x) for x in arrs], int(sh_deg), *[_p(x) for x in rays], B, t_thresh, w_thresh,
								*[_p(x) for x in up], *[_p(x) for x in g])
	return tuple(g)


def walk(points, offsets, adj, o, d, z, start, n_threads=0):
	arrs = [_a(points, np.float32), _a(offsets, np.int32), _a(adj, np.int32), _a(o, np.float32), _a(d, np.float32),
			_a(z, np.float32), _a(start, np.int32)]
	B, S = arrs[5].shape
	site = np.zeros((B, S), np.int32)
	steps = np.zeros(B, np.int32)
	load().oracle_walk(*[_p(a) for a in arrs], B, S, _p(site), _p(steps), int(n_threads))
	return site, steps


def density(points, offsets, adj, raw, log_scale, quat, x, site, scale_mult=1.0, n_threads=0):
	arrs = [_a(points, np.float32), _a(offsets, np.int32), _a(adj, np.int32), _a(raw, np.float32),
			_a(log_scale, np.float32), _a(quat, np.float32), _a(x, np.float32), _a(site, np.int32)]
	m = len(arrs[6])
	sigma = np.zeros(m, np.float32)
	load().oracle_density(*[_p(a) for a in arrs], m, float(scale_mult), _p(sigma), int(n_threads))
	return sigma


def color(points, offsets, adj, log_scale, quat, sh, sh_deg, x, dirs, site, n_threads=0):
	arrs = [_a(points, np.float32), _a(offsets, np.int32), _a(adj, np.int32), _a(log_scale, np.float32),
			_a(quat, np.float32), _a(sh, np.float32)]
	tail = [_a(x, np.float32), _a(dirs, np.float32), _a(site, np.int32)]
	m = len(tail[0])
	rgb = np.zeros((m, 3), np.float32)
	load().oracle_color(*[_p(a) for a in arrs], int(sh_deg), *[_p(a) for a in tail], m, _p(rgb), int(n_threads))
	return rgb


def conic(log_scale, quat, floor=0.0):
	ls, q = _a(log_scale, np.float32), _a(quat, np.float32)
	A = np.zeros((len(q), 6), np.float32)
	load().oracle_conic(_p(ls), _p(q), len(q), float(np.float32(floor * floor)), _p(A))
	return A


def density_backward(points, offsets, adj, raw, log_scale, quat, x, site, grad_sigma):
	"""-> g_raw (N,), g_ls (N, 3), g_quat (N, 4), accumulated in sample order on one thread."""
	arrs = [_a(points, np.float32), _a(offsets, np.int32), _a(adj, np.int32), _a(raw, np.float32),
			_a(log_scale, np.float32), _a(quat, np.float32), _a(x, np.float32), _a(site, np.int32)]
	n, m = len(arrs[3]), len(arrs[6])
	g_raw, g_ls, g_quat = np.zeros(n, np.float32), np.zeros((n, 3), np.float32), np.zeros((n, 4), np.float32)
	load().oracle_density_backward(*[_p(a) for a in arrs], m, _p(_a(grad_sigma, np.float32)), _p(g_raw), _p(g_ls),
								   _p(g_quat))
	return g_raw, g_ls, g_quat


def color_backward(points, offsets, adj, log_scale, quat, sh, sh_deg, x, dirs, site, rgb, grad_rgb):
	"""-> g_ls (N, 3), g_quat (N, 4), g_sh (N, 16, 3), accumulated in sample order on one thread."""
	arrs = [_a(points, np.float32), _a(offsets, np.int32), _a(adj, np.int32), _a(log_scale, np.float32),
			_a(quat, np.float32), _a(sh, np.float32)]
	tail = [_a(x, np.float32), _a(dirs, np.float32), _a(site, np.int32)]
	n, m = len(arrs[4]), len(tail[0])
	g_ls, g_quat, g_sh = np.zeros((n, 3), np.float32), np.zeros((n, 4), np.float32), np.zeros((n, 16, 3), np.float32)
	load().oracle_color_backward(*[_p(a) for a in arrs], int(sh_deg), *[_p(a) for a in tail], m,
								 _p(_a(rgb, np.float32)), _p(_a(grad_rgb, np.float32)), _p(g_ls), _p(g_quat), _p(g_sh))
	return g_ls, g_quat, g_sh


def conic_backward(log_scale, quat, gA, floor=0.0):
	"""-> g_ls (n, 3), g_quat (n, 4)."""
	ls, q = _a(log_scale, np.float32), _a(quat, np.float32)
	g_ls, g_quat = np.zeros((len(q), 3), np.float32), np.zeros((len(q), 4), np.float32)
	load().oracle_conic_backward(_p(ls), _p(q), len(q), float(np.float32(floor * floor)), _p(_a(gA, np.float32)),
								 _p(g_ls), _p(g_quat))
	return g_ls, g_quat


def sh_basis(d, deg):
	b = np.zeros(16, np.float32)
	load().oracle_sh_basis(float(d[0]), float(d[1]), float(d[2]), int(deg), _p(b))
	return b


def sample_at(near, mid, far, n_in, dt, n_bg, k):
	t, delta = np.zeros(1, np.float32), np.zeros(1, np.float32)
	load().oracle_sample_at(near, mid, far, n_in, dt, n_bg, k, _p(t), _p(delta))
	return float(t[0]), float(delta[0])
