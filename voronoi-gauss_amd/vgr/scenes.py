"""Seeded synthetic scenes and cameras of the five benchmark configurations.

Every scene is a fixed point cloud with its Delaunay CSR adjacency (sites.delaunay_graph), per-site density
raw = ln(rho), isotropic Gaussian log-scales shared by the density and colour Gaussians, identity rotations and
SH coefficients (N, 16, 3), plus pinhole cameras (or a raw ray batch for config 5). The mapping to the
reference's model (model.py:19-46) is: raw -> rho = exp(raw), log_scale -> conic diag(e^{-2s}), sh = (N, 16, 3).

`scale` < 1 shrinks the site count (tests); the distributions are unchanged. Geometry (points + CSR) is the
expensive part (Qhull); it is cached as .npy files under `cache_dir` keyed by config, seed and site count.
"""

import math
import os
import time
from dataclasses import dataclass, field

import numpy as np

from .sites import delaunay_graph, nearest_sites

DEFAULT_CACHE = os.environ.get('VGR_SCENE_CACHE',
							   os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))),
											'.scene_cache'))

SITE_COUNTS = {1: 16_384, 2: 500_000, 3: 2_000_000, 4: 8_000_000, 5: 4_000_000}
SEEDS = {1: 0, 2: 1, 3: 2, 4: 3, 5: 4}


@dataclass
class Camera:
	"""Pinhole camera, OpenCV axes (x right, y down, z forward), horizontal field of view in degrees."""
	eye: np.ndarray
	target: np.ndarray
	up: np.ndarray
	width: int
	height: int
	fov_deg: float = 60.0

	def c2w(self):
		f = self.target - self.eye
		f = f / np.linalg.norm(f)
		r = np.cross(f, self.up)
		r = r / np.linalg.norm(r)
		down = np.cross(f, r)
		return np.stack([r, down, f], 1)  # columns = camera axes in world coordinates

	def intrinsics(self):
		fx = 0.5 * self.width / math.tan(math.radians(self.fov_deg) / 2)
		return fx, fx, 0.5 * self.width, 0.5 * self.height

	def rays(self):
		"""-> o, d (H * W, 3) float32, row-major pixels: d = normalise(R K^-1 (px + 0.5, py + 0.5, 1)), the
		convention of colmap.py:129-134."""
		fx, fy, cx, cy = self.intrinsics()
		py, px = np.meshgrid(np.arange(self.height, dtype=np.float64), np.arange(self.width, dtype=np.float64),
							 indexing='ij')
		cam = np.stack([(px + 0.5 - cx) / fx, (py + 0.5 - cy) / fy, np.ones_like(px)], -1).reshape(-1, 3)
		d = cam @ self.c2w().T
		d /= np.linalg.norm(d, axis=1, keepdims=True)
		o = np.broadcast_to(self.eye, d.shape)
		return np.ascontiguousarray(o, dtype=np.float32), np.ascontiguousarray(d, dtype=np.float32)


@dataclass
class Scene:
	config: int
	seed: int
	points: np.ndarray       # (N, 3) f32
	offsets: np.ndarray      # (N + 1) i32
	adj: np.ndarray          # (M) i32
	raw: np.ndarray          # (N) f32, ln(density)
	log_scale: np.ndarray    # (N, 3) f32
	quat: np.ndarray         # (N, 4) f32, w x y z
	sh: np.ndarray           # (N, 16, 3) f32
	sh_deg: int
	far_radius: float
	cameras: list = field(default_factory=list)
	ray_batch: tuple = None  # (o, d) for ray-batch configs
	near: float = 0.02

	@property
	def n_sites(self):
		return len(self.points)

	def camera_rays(self, tile=8, curve='row'):
		"""-> o, d (B, 3) f32 of all cameras (tile order when tile > 0, the tiles in `curve` order: 'row' or
		'morton'), start (B,) i32 = the site nearest to each camera centre, and the pixel permutation (None for ray
		batches)."""
		if self.ray_batch is not None:
			o, d = self.ray_batch
			return o, d, nearest_sites(self.points, o), None
		os_, ds, starts, perms = [], [], [], []
		centers = np.stack([c.eye for c in self.cameras]).astype(np.float32)
		cstart = nearest_sites(self.points, centers)
		base = 0
		for c, s in zip(self.cameras, cstart):
			o, d = c.rays()
			perm = tile_order(c.height, c.width, tile, tile, curve) if tile else np.arange(len(o))
			os_.append(o[perm])
			ds.append(d[perm])
			starts.append(np.full(len(o), s, dtype=np.int32))
			perms.append(perm + base)
			base += len(o)
		return (np.concatenate(os_), np.concatenate(ds), np.concatenate(starts), np.concatenate(perms))


def morton2(y, x):
	"""Z-order key of non-negative integer coordinates below 2^16 (bits of y and x interleaved, y above x)."""
	def spread(v):
		v = v.astype(np.int64) & 0xFFFF
		v = (v | (v << 8)) & 0x00FF00FF
		v = (v | (v << 4)) & 0x0F0F0F0F
		v = (v | (v << 2)) & 0x33333333
		return (v | (v << 1)) & 0x55555555
	return (spread(y) << 1) | spread(x)


def tile_order(H, W, th=8, tw=8, curve='row'):
	"""Pixel permutation grouping th * tw consecutive rays into th x tw tiles (bench_infer.py:37-41 uses 4 x 8
	for 32-lane warps; 8 x 8 fills a 64-lane wavefront). The tiles follow each other in row-major order ('row') or
	along the Z-order curve of their tile coordinates ('morton'), which keeps any run of consecutive tiles (the
	tiles a GPU renders at one time) compact in the image."""
	y, x = np.meshgrid(np.arange(H), np.arange(W), indexing='ij')
	ty, tx = y // th, x // tw
	if curve == 'row':
		tkey = ty.astype(np.int64) * ((W + tw - 1) // tw) + tx
	elif curve == 'morton':
		tkey = morton2(ty, tx)
	else:
		raise ValueError(f'unknown tile curve {curve!r}')
	key = tkey * (th * tw) + (y % th) * tw + x % tw
	return np.argsort(key.ravel(), kind='stable')


def softplus(x):
	return np.logaddexp(0.0, x)


def _unit(rng, n):
	u = rng.normal(size=(n, 3))
	return u / np.linalg.norm(u, axis=1, keepdims=True)


def _clusters(rng, n, lo=-1.0, hi=1.0, k=64):
	"""n points from a mixture of k isotropic Gaussians, centres U[lo, hi]^3, sigma ~ U(0.05, 0.2), redrawn
	until inside [lo, hi]^3."""
	centres = rng.uniform(lo, hi, (k, 3))
	sig = rng.uniform(0.05, 0.2, k)
	out = np.empty((0, 3))
	while len(out) < n:
		m = n - len(out)
		c = rng.integers(0, k, m)
		p = centres[c] + sig[c, None] * rng.normal(size=(m, 3))
		out = np.concatenate([out, p[np.all((p >= lo) & (p <= hi), axis=1)]])
	return out[:n]


def _surface(rng, n, jitter=0.005):
	"""n points on the unit sphere and two tori (R = 0.6, r = 0.15, in the xy and xz planes), one third each,
	moved along the surface normal by N(0, jitter)."""
	kind = rng.integers(0, 3, n)
	p = np.empty((n, 3))
	nrm = np.empty((n, 3))
	s = kind == 0
	u = _unit(rng, int(s.sum()))
	p[s], nrm[s] = u, u
	R, r = 0.6, 0.15
	for t, plane in ((1, 'xy'), (2, 'xz')):
		s = kind == t
		m = int(s.sum())
		a, b = rng.uniform(0, 2 * np.pi, m), rng.uniform(0, 2 * np.pi, m)
		ring = np.stack([np.cos(a), np.sin(a)], 1)
		q = np.empty((m, 3))
		nq = np.empty((m, 3))
		q[:, 0], nq[:, 0] = (R + r * np.cos(b)) * ring[:, 0], np.cos(b) * ring[:, 0]
		if plane == 'xy':
			q[:, 1], q[:, 2] = (R + r * np.cos(b)) * ring[:, 1], r * np.sin(b)
			nq[:, 1], nq[:, 2] = np.cos(b) * ring[:, 1], np.sin(b)
		else:
			q[:, 2], q[:, 1] = (R + r * np.cos(b)) * ring[:, 1], r * np.sin(b)
			nq[:, 2], nq[:, 1] = np.cos(b) * ring[:, 1], np.sin(b)
		p[s], nrm[s] = q, nq
	return p + rng.normal(scale=jitter, size=(n, 1)) * nrm, kind


def _geometry(config, n, rng):
	"""-> raw points (n, 3) float64 and a per-point class used by the attribute draw (0 volume, 1 surface)."""
	cls = np.zeros(n, dtype=np.int8)
	if config in (1, 5):
		p = rng.uniform(-1, 1, (n, 3))
	elif config == 2:
		p = _clusters(rng, n)
	elif config == 3:
		ns = int(round(0.7 * n))
		ps, _ = _surface(rng, ns)
		p = np.concatenate([ps, rng.uniform(-1.5, 1.5, (n - ns, 3))])
		cls[:ns] = 1
	elif config == 4:
		nd = int(round(0.75 * n))
		r = 1.0 / rng.uniform(0.02, 1.0, n - nd)
		p = np.concatenate([_clusters(rng, nd), _unit(rng, n - nd) * r[:, None]])
	else:
		raise ValueError(f'unknown config {config}')
	return p, cls


def _orbit(n, radius, width, height, elev=0.0):
	cams = []
	for k in range(n):
		th = 2 * np.pi * k / n
		eye = np.array([radius * np.sin(th), elev, radius * np.cos(th)])
		cams.append(Camera(eye, np.zeros(3), np.array([0.0, 1.0, 0.0]), width, height))
	return cams


def _cameras(config, img_scale):
	def px(v):
		return max(8, int(round(v * img_scale)))
	if config == 1:
		return [Camera(np.array([0.0, 0.0, 3.0]), np.zeros(3), np.array([0.0, 1.0, 0.0]), px(128), px(128))]
	if config == 2:
		return _orbit(8, 3.0, px(800), px(800))
	if config == 3:
		return _orbit(4, 3.0, px(1920), px(1080))
	if config == 4:
		cams = []
		for k in range(4):
			th = 2 * np.pi * k / 4 + np.pi / 4
			eye = np.array([0.6 * np.cos(th), 0.1, 0.6 * np.sin(th)])
			cams.append(Camera(eye, 3.0 * eye, np.array([0.0, 1.0, 0.0]), px(1920), px(1080)))
		return cams
	return []


def load_geometry(config, n_sites=None, cache_dir=DEFAULT_CACHE, log=print):
	"""-> points (N, 3) f32, offsets (N + 1) i32, adj (M) i32, point class (N,) i8, for the seeded config."""
	seed = SEEDS[config]
	n = SITE_COUNTS[config] if n_sites is None else int(n_sites)
	path = None
	if cache_dir:
		path = os.path.join(cache_dir, f'c{config}_s{seed}_n{n}')
		if os.path.exists(path + '_adj.npy'):
			return (np.load(path + '_pts.npy'), np.load(path + '_off.npy'), np.load(path + '_adj.npy'),
					np.load(path + '_cls.npy'))
	rng = np.random.default_rng(seed)
	p, cls = _geometry(config, n, rng)
	p32 = p.astype(np.float32)
	t0 = time.time()
	if log:
		log(f'[scene] config {config}: Delaunay of {n} sites (Qhull) ...')
	pts, idx, offsets, adj = delaunay_graph(p32.astype(np.float64))
	if log:
		log(f'[scene] config {config}: Delaunay of {n} sites in {time.time() - t0:.1f} s, mean degree '
			f'{len(adj) / len(pts):.2f}, max {int(np.diff(offsets).max())}')
	pts = pts.astype(np.float32)
	cls = cls[idx]
	if path:
		os.makedirs(cache_dir, exist_ok=True)
		for suffix, arr in (('_pts', pts), ('_off', offsets), ('_cls', cls), ('_adj', adj)):
			np.save(path + suffix + '.tmp.npy', arr)
			os.replace(path + suffix + '.tmp.npy', path + suffix + '.npy')
	return pts, offsets, adj, cls


def make_scene(config, scale=1.0, img_scale=1.0, n_rays=None, cache_dir=DEFAULT_CACHE, log=print):
	"""Seeded synthetic scene of benchmark configuration `config` (1..5) with round(scale * N) sites."""
	n = max(64, int(round(SITE_COUNTS[config] * scale)))
	pts, offsets, adj, cls = load_geometry(config, n, cache_dir, log)
	N = len(pts)
	rng = np.random.default_rng(1000 + SEEDS[config])  # attribute stream, independent of the geometry draw
	if config == 1:
		dens = softplus(rng.normal(0.0, 1.0, N))
		ls = rng.normal(-3.0, 0.3, N)
		sh_deg = 0
	else:
		if config == 2:
			dens = softplus(rng.normal(1.0, 1.0, N))
		elif config == 3:
			dens = np.where(cls == 1, softplus(rng.normal(4.0, 0.5, N)), softplus(rng.normal(-3.0, 0.5, N)))
		elif config == 4:
			dens = softplus(rng.normal(0.0, 1.5, N))
		else:
			dens = softplus(rng.normal(-4.0, 0.5, N))
		ls = rng.normal(-4.0, 0.3, N)
		sh_deg = 3
	sh = np.zeros((N, 16, 3))
	sh[:, 0] = rng.normal(0.0, 0.5, (N, 3))
	if sh_deg > 0:
		sh[:, 1:] = rng.normal(0.0, 0.05, (N, 15, 3))
	quat = np.zeros((N, 4), dtype=np.float32)
	quat[:, 0] = 1.0
	scene = Scene(config=config, seed=SEEDS[config], points=pts, offsets=offsets, adj=adj,
				  raw=np.log(dens).astype(np.float32), log_scale=np.repeat(ls[:, None], 3, 1).astype(np.float32),
				  quat=quat, sh=sh.astype(np.float32), sh_deg=sh_deg, far_radius=55.0 if config == 4 else 4.0,
				  cameras=_cameras(config, img_scale))
	if config == 5:
		scene.ray_batch = ray_batch(config, n_rays)
	return scene


def ray_batch(config=5, n_rays=None):
	"""The seeded ray batch of config 5: origins uniform in [-0.9, 0.9]^3, directions uniform on S^2 ->
	(o, d) float32 (B, 3), B = 16,777,216 unless n_rays is given."""
	B = 16_777_216 if n_rays is None else int(n_rays)
	rr = np.random.default_rng(2000 + SEEDS[config])
	o = rr.uniform(-0.9, 0.9, (B, 3)).astype(np.float32)
	return o, _unit(rr, B).astype(np.float32)


def site_points(config, scale=1.0):
	"""The seeded site draw of a config before triangulation (float32 (n, 3)): what the start-cell locator needs,
	without the Qhull step (which only drops coincident points)."""
	n = max(64, int(round(SITE_COUNTS[config] * scale)))
	p, _ = _geometry(config, n, np.random.default_rng(SEEDS[config]))
	return p.astype(np.float32)


def _main(argv=None):
	"""`python -m vgr.scenes --geometry C [C ...] [--cache DIR]`: triangulates the seeded site clouds of the given
	configurations at their full site counts and stores them in the geometry cache (what make_scene then loads)."""
	import argparse
	ap = argparse.ArgumentParser(description=_main.__doc__)
	ap.add_argument('--geometry', type=int, nargs='+', required=True, choices=sorted(SITE_COUNTS))
	ap.add_argument('--cache', default=DEFAULT_CACHE)
	a = ap.parse_args(argv)
	for c in a.geometry:
		t0 = time.time()
		pts, _, adj, _ = load_geometry(c, cache_dir=a.cache, log=lambda *m: print(*m, flush=True))
		print(f'[scene] config {c}: {len(pts)} sites, {len(adj)} adjacency entries, cached in {time.time() - t0:.1f} s',
			  flush=True)


if __name__ == '__main__':
	_main()
