"""Cameras of trained scenes: the binary COLMAP sparse model (sparse/0/cameras.bin, images.bin, points3D.bin) of the
Mip-NeRF 360 / Deep Blending layout, normalised into the unit ball the way the reference's colmap.py:1-134 does, so
that a model trained by the reference renders through its own test views here.

The readers follow COLMAP's documented binary format (little-endian; counts as uint64). Only what rendering needs is
kept: intrinsics, world-to-camera rotations and translations, image names, and the sparse points that define the
normalisation. Images are read only on request (they are the ground truth, not an input of the renderer)."""

import os
import struct

import numpy as np
import torch

# parameters per COLMAP camera model: SIMPLE_PINHOLE, PINHOLE, SIMPLE_RADIAL, RADIAL, OPENCV, OPENCV_FISHEYE,
# FULL_OPENCV (colmap.py:10)
CAMERA_PARAMS = {0: 3, 1: 4, 2: 4, 3: 5, 4: 8, 5: 8, 6: 12}


def qvec_to_rot(q):
	"""Rotation matrix of the unit quaternion (w, x, y, z) (colmap.py:13-19)."""
	w, x, y, z = q
	return np.array([
		[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
		[2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
		[2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)],
	])


def _unpack(fh, fmt):
	size = struct.calcsize(fmt)
	raw = fh.read(size)
	if len(raw) != size:
		raise ValueError(f'{fh.name}: truncated COLMAP file')
	return struct.unpack(fmt, raw)


def read_cameras(path):
	"""{camera id: (model, width, height, params)} (colmap.py:22-29)."""
	cams = {}
	with open(path, 'rb') as fh:
		for _ in range(_unpack(fh, '<Q')[0]):
			cid, model, w, h = _unpack(fh, '<iiQQ')
			if model not in CAMERA_PARAMS:
				raise ValueError(f'{path}: camera model {model} is not supported')
			cams[cid] = (model, w, h, _unpack(fh, f'<{CAMERA_PARAMS[model]}d'))
	return cams


def read_images(path):
	"""{image id: (name, R world->camera (3, 3), t (3,), camera id)} (colmap.py:32-45)."""
	images = {}
	with open(path, 'rb') as fh:
		for _ in range(_unpack(fh, '<Q')[0]):
			iid = _unpack(fh, '<i')[0]
			q = _unpack(fh, '<4d')
			t = _unpack(fh, '<3d')
			cid = _unpack(fh, '<i')[0]
			name = bytearray()
			while (ch := fh.read(1)) not in (b'\0', b''):
				name += ch
			n2d = _unpack(fh, '<Q')[0]
			fh.seek(24 * n2d, 1)  # the 2D observations (x, y, point id) are not needed
			images[iid] = (name.decode(), qvec_to_rot(q), np.array(t), cid)
	return images


def read_points(path):
	"""-> xyz (P, 3) float64, rgb (P, 3) float32 in [0, 1], reprojection error (P,), tracks (list of image-id
	arrays) (colmap.py:48-58)."""
	xyz, rgb, err, tracks = [], [], [], []
	with open(path, 'rb') as fh:
		for _ in range(_unpack(fh, '<Q')[0]):
			_unpack(fh, '<Q')  # point id
			xyz.append(_unpack(fh, '<3d'))
			rgb.append(_unpack(fh, '<3B'))
			err.append(_unpack(fh, '<d')[0])
			n = _unpack(fh, '<Q')[0]
			tracks.append(np.frombuffer(fh.read(8 * n), dtype=np.int32)[0::2].copy())
	return (np.array(xyz, np.float64).reshape(-1, 3), np.array(rgb, np.float32).reshape(-1, 3) / 255.0,
			np.array(err, np.float64), tracks)


def intrinsics(model, params):
	"""(fx, fy, cx, cy); radial terms are ignored, the images being undistorted (colmap.py:61-65)."""
	if model in (0, 2, 3):
		f, cx, cy = params[:3]
		return f, f, cx, cy
	return tuple(params[:4])


def normalization_of(xyz, radius=0.95, keep_quantile=0.98):
	"""(center, scale) with x_n = (x - center) / scale putting `keep_quantile` of the sparse points within
	`radius` (colmap.py:94-97)."""
	center = np.median(xyz, 0)
	scale = np.quantile(np.linalg.norm(xyz - center, axis=1), keep_quantile) / radius
	return center, scale


class ColmapCameras:
	"""The views of one split (every `test_every`-th image by name is a test view, colmap.py:84-89) in normalised
	coordinates: K (n, 3, 3) at the downsampled resolution, c2w (n, 4, 4) camera-to-world with OpenCV axes,
	centers (n, 3). `normalization` = (center, scale) as stored in a trained model's checkpoint; without it, it is
	derived from the sparse points."""

	def __init__(self, root, split='test', downsample=4, device='cuda', test_every=8, radius=0.95,
				 keep_quantile=0.98, normalization=None, load_images=False):
		if split not in ('train', 'test'):
			raise ValueError(f"split must be 'train' or 'test' (got {split!r})")
		self.root, self.device = root, torch.device(device)
		sparse = os.path.join(root, 'sparse', '0')
		cams = read_cameras(os.path.join(sparse, 'cameras.bin'))
		images = read_images(os.path.join(sparse, 'images.bin'))
		order = sorted(images, key=lambda i: images[i][0])
		idx = np.arange(len(order))
		keep = idx % test_every != 0 if split == 'train' else idx % test_every == 0
		self.image_ids = [order[i] for i in idx[keep]]
		self.names = [images[i][0] for i in self.image_ids]
		self.n = len(self.names)
		if self.n == 0:
			raise ValueError(f'{root}: no {split} images')

		img_dir = os.path.join(root, 'images' if downsample == 1 else f'images_{downsample}')
		first = os.path.join(img_dir, self.names[0])
		if os.path.exists(first):
			from PIL import Image
			with Image.open(first) as im:
				self.W, self.H = im.size
		else:  # no image files: the resolution the downsampled images would have
			_, w, h, _ = cams[images[self.image_ids[0]][3]]
			self.W, self.H = int(round(w / downsample)), int(round(h / downsample))
		self.images = None
		if load_images:
			from PIL import Image
			rgb = [np.asarray(Image.open(os.path.join(img_dir, n)).convert('RGB')) for n in self.names]
			self.images = torch.from_numpy(np.stack(rgb)).to(self.device)

		if normalization is None:
			xyz = read_points(os.path.join(sparse, 'points3D.bin'))[0]
			normalization = normalization_of(xyz, radius, keep_quantile)
		center, scale = normalization
		center, scale = np.asarray(center, np.float64).reshape(3), float(scale)
		self.normalization = (center, scale)

		Ks, c2ws = [], []
		for iid in self.image_ids:
			_, R, t, cid = images[iid]
			model, w, h, params = cams[cid]
			fx, fy, cx, cy = intrinsics(model, params)
			sx, sy = self.W / w, self.H / h
			Ks.append(np.array([[fx * sx, 0, cx * sx], [0, fy * sy, cy * sy], [0, 0, 1]]))
			c2w = np.eye(4)
			c2w[:3, :3] = R.T
			c2w[:3, 3] = (-R.T @ t - center) / scale
			c2ws.append(c2w)
		self.K = torch.tensor(np.stack(Ks), dtype=torch.float32, device=self.device)
		self.K_inv = torch.linalg.inv(self.K)
		self.c2w = torch.tensor(np.stack(c2ws), dtype=torch.float32, device=self.device)
		self.centers = self.c2w[:, :3, 3].contiguous()

	def rays(self, img, px, py):
		"""Rays through pixel centres (px + 0.5, py + 0.5) of views `img` (colmap.py:126-131) -> o, d (m, 3)."""
		p = torch.stack([px + 0.5, py + 0.5, torch.ones_like(px)], -1).float()
		d = torch.bmm(self.K_inv[img], p[:, :, None])
		d = torch.bmm(self.c2w[img, :3, :3].contiguous(), d)[:, :, 0]
		d = d / d.norm(dim=-1, keepdim=True)
		return self.centers[img], d

	def image_rays(self, i):
		"""-> o, d (H * W, 3) of view i in row-major pixel order, and its image (H * W, 3) in [0, 1] or None."""
		py, px = torch.meshgrid(torch.arange(self.H, device=self.device), torch.arange(self.W, device=self.device),
								indexing='ij')
		img = torch.full((self.H * self.W,), i, dtype=torch.long, device=self.device)
		o, d = self.rays(img, px.reshape(-1), py.reshape(-1))
		gt = None if self.images is None else self.images[i].reshape(-1, 3).float() / 255.0
		return o.contiguous(), d.contiguous(), gt
