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


def split_views(images, split, test_every):
	"""Image ids of one split, in name order: the test split is every `test_every`-th image by name starting with the
	first, the train split the others (colmap.py:84-89)."""
	if split not in ('train', 'test'):
		raise ValueError(f"split must be 'train' or 'test' (got {split!r})")
	by_name = sorted(images, key=lambda iid: images[iid][0])
	is_test = [rank % test_every == 0 for rank in range(len(by_name))]
	return [iid for iid, t in zip(by_name, is_test) if t == (split == 'test')]


def image_size(root, downsample, first_name, camera):
	"""(W, H) of the split's images: read from the first downsampled image file when present, else the camera's
	resolution divided by `downsample` (the size the downsampled images have)."""
	img_dir = os.path.join(root, 'images' if downsample == 1 else f'images_{downsample}')
	path = os.path.join(img_dir, first_name)
	if os.path.exists(path):
		from PIL import Image
		with Image.open(path) as im:
			return im.size
	_, w, h, _ = camera
	return int(round(w / downsample)), int(round(h / downsample))


def view_matrices(cams, images, ids, width, height, center, scale):
	"""Per view: K (n, 3, 3) scaled from the camera's resolution to width x height, and camera-to-world c2w (n, 4, 4)
	in normalised coordinates (rotation R^T of the world-to-camera rotation R, camera centre (-R^T t - center) /
	scale), as colmap.py:100-118 defines them; all views at once."""
	R = np.stack([images[i][1] for i in ids])                  # (n, 3, 3) world -> camera
	t = np.stack([images[i][2] for i in ids])                  # (n, 3)
	cam = [cams[images[i][3]] for i in ids]
	fxfycxcy = np.array([intrinsics(c[0], c[3]) for c in cam], np.float64)  # (n, 4)
	res = np.array([(c[1], c[2]) for c in cam], np.float64)    # (n, 2) native width, height
	sx, sy = width / res[:, 0], height / res[:, 1]
	n = len(ids)
	K = np.zeros((n, 3, 3))
	K[:, 0, 0], K[:, 1, 1] = fxfycxcy[:, 0] * sx, fxfycxcy[:, 1] * sy
	K[:, 0, 2], K[:, 1, 2] = fxfycxcy[:, 2] * sx, fxfycxcy[:, 3] * sy
	K[:, 2, 2] = 1.0
	Rt = np.transpose(R, (0, 2, 1))
	c2w = np.tile(np.eye(4), (n, 1, 1))
	c2w[:, :3, :3] = Rt
	c2w[:, :3, 3] = (-np.einsum('nij,nj->ni', Rt, t) - center) / scale
	return K, c2w


class ColmapCameras:
	"""The views of one split (every `test_every`-th image by name is a test view, colmap.py:84-89) in normalised
	coordinates: K (n, 3, 3) at the downsampled resolution, c2w (n, 4, 4) camera-to-world with OpenCV axes,
	centers (n, 3). `normalization` = (center, scale) as stored in a trained model's checkpoint; without it, it is
	derived from the sparse points."""

	def __init__(self, root, split='test', downsample=4, device='cuda', test_every=8, radius=0.95,
				 keep_quantile=0.98, normalization=None, load_images=False):
		self.root, self.device = root, torch.device(device)
		sparse = os.path.join(root, 'sparse', '0')
		cams = read_cameras(os.path.join(sparse, 'cameras.bin'))
		images = read_images(os.path.join(sparse, 'images.bin'))
		self.image_ids = split_views(images, split, test_every)
		if not self.image_ids:
			raise ValueError(f'{root}: no {split} images')
		self.names = [images[i][0] for i in self.image_ids]
		self.n = len(self.names)
		self.W, self.H = image_size(root, downsample, self.names[0], cams[images[self.image_ids[0]][3]])
		self.images = self._read_images(downsample) if load_images else None

		if normalization is None:
			normalization = normalization_of(read_points(os.path.join(sparse, 'points3D.bin'))[0], radius,
											 keep_quantile)
		center = np.asarray(normalization[0], np.float64).reshape(3)
		scale = float(normalization[1])
		self.normalization = (center, scale)

		K, c2w = view_matrices(cams, images, self.image_ids, self.W, self.H, center, scale)
		self.K = torch.tensor(K, dtype=torch.float32, device=self.device)
		self.K_inv = torch.linalg.inv(self.K)
		self.c2w = torch.tensor(c2w, dtype=torch.float32, device=self.device)
		self.centers = self.c2w[:, :3, 3].contiguous()

	def _read_images(self, downsample):
		from PIL import Image
		img_dir = os.path.join(self.root, 'images' if downsample == 1 else f'images_{downsample}')
		rgb = [np.asarray(Image.open(os.path.join(img_dir, n)).convert('RGB')) for n in self.names]
		return torch.from_numpy(np.stack(rgb)).to(self.device)

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
