"""Float64 dense references -- TEST INFRASTRUCTURE ONLY.

Independent restatements, in numpy float64, of the reference's own test oracles; they pin the C oracle:
  trace / foam_dense    test_foam.py:18-37 (bisector-plane re-trace) and :76-104 (dense sigma, softmax colour,
                        trapezoid compositing)
  march_samples / march_dense   test_march.py:14-22 and :59-79 (exact nearest site, NeRF compositing)
  density_dense / color_dense   test_grad.py:21-48, :92-104 (quaternion Mahalanobis, softmax blend)
  sh_basis              test_grad.py:21-32
  nearest_brute         sites.py:38-39 (cKDTree nearest site), by exhaustive float64 search
Every neighbourhood is the explicit set {c} U adj(c); nearest sites come from cKDTree, not from a walk.
"""

import numpy as np
from scipy.spatial import cKDTree

SH_C = [0.28209479177387814, 0.4886025119029199, 1.0925484305920792, 0.31539156525252005, 0.5462742152960396,
		0.5900435899266435, 2.890611442640554, 0.4570457994644658, 0.3731763325901154, 1.445305721320277]


def sh_basis(d, deg=3):
	"""(m, 16) real SH basis of unit directions d (m, 3), zero beyond `deg`."""
	d = np.atleast_2d(np.asarray(d, np.float64))
	x, y, z = d[:, 0], d[:, 1], d[:, 2]
	xx, yy, zz = x * x, y * y, z * z
	b = np.zeros((len(d), 16))
	b[:, 0] = SH_C[0]
	if deg >= 1:
		b[:, 1], b[:, 2], b[:, 3] = -SH_C[1] * y, SH_C[1] * z, -SH_C[1] * x
	if deg >= 2:
		b[:, 4], b[:, 5] = SH_C[2] * x * y, -SH_C[2] * y * z
		b[:, 6], b[:, 7] = SH_C[3] * (2 * zz - xx - yy), -SH_C[2] * x * z
		b[:, 8] = SH_C[4] * (xx - yy)
	if deg >= 3:
		b[:, 9], b[:, 10] = -SH_C[5] * y * (3 * xx - yy), SH_C[6] * x * y * z
		b[:, 11] = -SH_C[7] * y * (4 * zz - xx - yy)
		b[:, 12] = SH_C[8] * z * (2 * zz - 3 * xx - 3 * yy)
		b[:, 13] = -SH_C[7] * x * (4 * zz - xx - yy)
		b[:, 14], b[:, 15] = SH_C[9] * z * (xx - yy), -SH_C[5] * x * (xx - 3 * yy)
	return b


def neighborhood(offsets, adj, c):
	return np.concatenate([[c], adj[offsets[c]:offsets[c + 1]]])


def maha6(A, v):
	"""v^T A v for conics A (k, 6) and offsets v (k, 3)."""
	return (A[:, 0] * v[:, 0] ** 2 + A[:, 3] * v[:, 1] ** 2 + A[:, 5] * v[:, 2] ** 2 +
			2 * (A[:, 1] * v[:, 0] * v[:, 1] + A[:, 2] * v[:, 0] * v[:, 2] + A[:, 4] * v[:, 1] * v[:, 2]))


def quat_rot(q):
	q = np.asarray(q, np.float64)
	q = q / np.linalg.norm(q, axis=-1, keepdims=True)
	w, x, y, z = q[..., 0], q[..., 1], q[..., 2], q[..., 3]
	return np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
					 2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
					 2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1).reshape(*q.shape[:-1], 3, 3)


def conic_dense(log_scale, quat, floor=0.0):
	"""A = R diag(1 / (e^{2 s} + floor^2)) R^T, (n, 6), float64."""
	R = quat_rot(quat)
	iv = 1.0 / (np.exp(2 * np.clip(np.asarray(log_scale, np.float64), -20, 20)) + floor * floor)
	A = np.einsum('nak,nk,nbk->nab', R, iv, R)
	return np.stack([A[:, 0, 0], A[:, 0, 1], A[:, 0, 2], A[:, 1, 1], A[:, 1, 2], A[:, 2, 2]], -1)


def trace(pts, offsets, adj, o, d, near, far, cell):
	"""Cell-by-cell traversal through bisector planes in float64 -> sample parameters t (S,) and the cell that
	evaluates each sample (S,); the last sample is x(far) in the last cell."""
	pts = np.asarray(pts, np.float64)
	t, cells = [near], [cell]
	while True:
		js = adj[offsets[cell]:offsets[cell + 1]]
		n = pts[js] - pts[cell]
		dn = n @ d
		ahead = dn > 0
		if not ahead.any():
			break
		tj = ((0.5 * (pts[js] + pts[cell]) - o) * n).sum(1)[ahead] / dn[ahead]
		k = np.argmin(tj)
		if tj[k] >= far:
			break
		cell = js[ahead][k]
		t.append(max(tj[k], t[-1]))
		cells.append(cell)
	t.append(far)
	cells.append(cells[-1])
	return np.array(t), np.array(cells)


def foam_dense(pts, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, t, cells, color_cut=np.inf, fused=False, r2=None,
			   baked=None):
	"""Foreground rgb (3,) and final T of one ray with samples t (S,) evaluated in `cells` (S,), thresholds off:
	sigma = sum over {c} U adj(c) of exp(raw) exp(-m_dA / 2), colour = softmax(-m_cA / 2) blend of
	max(SH + 1/2, 0), trapezoid rule. The approximate modes of foam_infer.cu:229-249,266-276:
	  r2 (N,): a density term counts only where |x - p_j|^2 <= r2_j (eps_density);
	  color_cut: a colour term counts only where m <= m_min + color_cut, m_min the sample's smallest m (exact mode),
	    or, fused, where m <= (the smallest m of the neighbours before it in {c} U adj(c) order) + color_cut;
	  baked (N, 3): site colours used instead of the SH colours."""
	pts = np.asarray(pts, np.float64)
	X = o[None] + t[:, None] * d[None]
	b = sh_basis(d[None], sh_deg)[0]
	sig = np.zeros(len(t))
	C = np.zeros((len(t), 3))
	for s, (x, c) in enumerate(zip(X, cells)):
		nb = neighborhood(offsets, adj, c)
		v = x[None] - pts[nb]
		dens = np.exp(raw[nb]) * np.exp(-0.5 * maha6(dA[nb], v))
		if r2 is not None:
			dens = np.where((v * v).sum(1) <= r2[nb], dens, 0.0)
		sig[s] = dens.sum()
		m = maha6(cA[nb], v)
		if fused:
			run = np.minimum.accumulate(np.concatenate([[np.inf], m[:-1]]))
			keep = m <= run + color_cut
		else:
			keep = m <= m.min() + color_cut
		lw = np.where(keep, -0.5 * m, -np.inf)
		a = np.exp(lw - lw.max())
		a /= a.sum()
		ck = np.asarray(baked, np.float64)[nb] if baked is not None else \
			np.maximum(np.einsum('j,njc->nc', b, sh[nb]) + 0.5, 0)
		C[s] = a @ ck
	delta = t[1:] - t[:-1]
	alpha = 1 - np.exp(-0.5 * (sig[1:] + sig[:-1]) * delta)
	trans = np.cumprod(np.concatenate([[1.0], 1 - alpha]))
	w = alpha * trans[:-1]
	return (w[:, None] * 0.5 * (C[1:] + C[:-1])).sum(0), trans[-1]


def march_samples(near, mid, far, dt, n_bg):
	"""Midpoints and lengths of the march steps of one ray."""
	n_in = int(np.ceil((mid - near) / dt)) if mid > near else 0
	t0 = near + dt * np.arange(n_in)
	t1 = np.minimum(t0 + dt, mid)
	u = np.arange(n_bg + 1) / n_bg
	tb = 1.0 / (1.0 / mid + u * (1.0 / far - 1.0 / mid))
	t = np.concatenate([0.5 * (t0 + t1), 1.0 / (1.0 / mid + 0.5 * (u[:-1] + u[1:]) * (1.0 / far - 1.0 / mid))])
	return t, np.concatenate([t1 - t0, tb[1:] - tb[:-1]])


def march_dense(pts, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, near, mid, far, dt, n_bg, tree=None):
	"""Foreground rgb (3,) and final T of one marched ray, thresholds off, exact nearest sites."""
	pts = np.asarray(pts, np.float64)
	tree = tree or cKDTree(pts)
	t, delta = march_samples(near, mid, far, dt, n_bg)
	X = o[None] + t[:, None] * d[None]
	site = tree.query(X)[1]
	b = sh_basis(d[None], sh_deg)[0]
	sig = np.zeros(len(t))
	C = np.zeros((len(t), 3))
	for s, (x, c) in enumerate(zip(X, site)):
		nb = neighborhood(offsets, adj, c)
		v = x[None] - pts[nb]
		sig[s] = (np.exp(raw[nb]) * np.exp(-0.5 * maha6(dA[nb], v))).sum()
		lw = -0.5 * maha6(cA[nb], v)
		a = np.exp(lw - lw.max())
		a /= a.sum()
		C[s] = a @ np.maximum(np.einsum('j,njc->nc', b, sh[nb]) + 0.5, 0)
	alpha = 1 - np.exp(-sig * delta)
	trans = np.cumprod(np.concatenate([[1.0], 1 - alpha]))
	w = alpha * trans[:-1]
	return (w[:, None] * C).sum(0), trans[-1]


def gauss_m(pts, log_scale, quat, k, x, inv_mult2=1.0):
	"""Mahalanobis distances of x (3,) to Gaussians k (n,) from (log_scale, quat)."""
	R = quat_rot(quat[k])
	v = x[None] - np.asarray(pts, np.float64)[k]
	y = np.einsum('nab,na->nb', R, v)
	return (y * y * inv_mult2 / np.exp(2 * np.asarray(log_scale, np.float64)[k])).sum(-1)


def density_dense(pts, offsets, adj, raw, log_scale, quat, x, site, scale_mult=1.0):
	out = np.zeros(len(x))
	for i, (xi, c) in enumerate(zip(np.asarray(x, np.float64), site)):
		nb = neighborhood(offsets, adj, c)
		out[i] = (np.exp(raw[nb]) * np.exp(-0.5 * gauss_m(pts, log_scale, quat, nb, xi, 1 / scale_mult ** 2))).sum()
	return out


def color_dense(pts, offsets, adj, log_scale, quat, sh, sh_deg, x, dirs, site):
	dirs = np.asarray(dirs, np.float64)
	dirs = dirs / np.linalg.norm(dirs, axis=1, keepdims=True)
	B = sh_basis(dirs, sh_deg)
	out = np.zeros((len(x), 3))
	for i, (xi, c) in enumerate(zip(np.asarray(x, np.float64), site)):
		nb = neighborhood(offsets, adj, c)
		lw = -0.5 * gauss_m(pts, log_scale, quat, nb, xi)
		a = np.exp(lw - lw.max())
		a /= a.sum()
		out[i] = a @ np.maximum(np.einsum('j,njc->nc', B[i], sh[nb]) + 0.5, 0)
	return out


def nearest_brute(points, queries):
	"""Nearest site of every query point by exhaustive search: the lexicographic argmin of (float64 squared
	distance (dx^2 + dy^2) + dz^2, site index). Restates nearest_sites (sites.py:38-39, scipy cKDTree in float64)
	up to exact distance ties, which cKDTree leaves unspecified."""
	p = np.asarray(points, np.float64)[:, :3]
	q = np.asarray(queries, np.float64)
	out = np.empty(len(q), np.int32)
	chunk = max(1, int(2e7 // max(len(p), 1)))
	for s in range(0, len(q), chunk):
		v = q[s:s + chunk, None, :] - p[None]
		d2 = (v[..., 0] * v[..., 0] + v[..., 1] * v[..., 1]) + v[..., 2] * v[..., 2]
		out[s:s + chunk] = d2.argmin(1)  # first index among equal minima
	return out
