"""Trained-scene inputs (CPU): the reference's model.pth checkpoint (train.py:168-170, loaded as bench_fps.py:19-28)
and its COLMAP cameras (colmap.py:1-134), on synthetic files written here in the same binary formats. Checked
against closed forms: intrinsics scaled to the image size, camera centres and principal rays from the poses, the
unit-ball normalisation of the sparse points, the test/train split by name order."""

import os
import pickle
import struct

import numpy as np
import pytest
import torch

from vgr import colmap
from vgr.model import VoronoiGaussField, load_checkpoint, load_model


# ------------------------------------------------------------------ COLMAP binary writers (the documented format)

def write_cameras(path, cams):
	with open(path, 'wb') as fh:
		fh.write(struct.pack('<Q', len(cams)))
		for cid, (model, w, h, params) in cams.items():
			fh.write(struct.pack('<iiQQ', cid, model, w, h))
			fh.write(struct.pack(f'<{len(params)}d', *params))


def write_images(path, images):
	with open(path, 'wb') as fh:
		fh.write(struct.pack('<Q', len(images)))
		for iid, (name, q, t, cid, n2d) in images.items():
			fh.write(struct.pack('<i', iid) + struct.pack('<4d', *q) + struct.pack('<3d', *t) + struct.pack('<i', cid))
			fh.write(name.encode() + b'\0')
			fh.write(struct.pack('<Q', n2d))
			for j in range(n2d):
				fh.write(struct.pack('<ddq', 1.0 * j, 2.0 * j, -1))


def write_points(path, xyz, rgb):
	with open(path, 'wb') as fh:
		fh.write(struct.pack('<Q', len(xyz)))
		for i, (p, c) in enumerate(zip(xyz, rgb)):
			fh.write(struct.pack('<Q', i) + struct.pack('<3d', *p) + struct.pack('<3B', *c) + struct.pack('<d', 0.5))
			track = [(1, 0), (2, 3)]
			fh.write(struct.pack('<Q', len(track)))
			for image_id, point2d in track:
				fh.write(struct.pack('<ii', image_id, point2d))


def quat_of(R):
	"""Unit quaternion (w, x, y, z) of a rotation matrix (Shepperd's method: the largest of 4w², 4x², 4y², 4z²
	sets the divisor, so half turns are exact too)."""
	t = np.trace(R)
	c = np.argmax([t, R[0, 0], R[1, 1], R[2, 2]])
	if c == 0:
		w = np.sqrt(1 + t) / 2
		q = [w, (R[2, 1] - R[1, 2]) / (4 * w), (R[0, 2] - R[2, 0]) / (4 * w), (R[1, 0] - R[0, 1]) / (4 * w)]
	elif c == 1:
		x = np.sqrt(1 + 2 * R[0, 0] - t) / 2
		q = [(R[2, 1] - R[1, 2]) / (4 * x), x, (R[0, 1] + R[1, 0]) / (4 * x), (R[0, 2] + R[2, 0]) / (4 * x)]
	elif c == 2:
		y = np.sqrt(1 + 2 * R[1, 1] - t) / 2
		q = [(R[0, 2] - R[2, 0]) / (4 * y), (R[0, 1] + R[1, 0]) / (4 * y), y, (R[1, 2] + R[2, 1]) / (4 * y)]
	else:
		z = np.sqrt(1 + 2 * R[2, 2] - t) / 2
		q = [(R[1, 0] - R[0, 1]) / (4 * z), (R[0, 2] + R[2, 0]) / (4 * z), (R[1, 2] + R[2, 1]) / (4 * z), z]
	return np.array(q)


def test_quat_of_inverts_qvec_to_rot():
	rng = np.random.default_rng(9)
	mats = [random_rotation(rng) for _ in range(20)] + [np.diag([1.0, -1.0, -1.0]), np.diag([-1.0, 1.0, -1.0]),
														 np.diag([-1.0, -1.0, 1.0]), np.eye(3)]
	for R in mats:
		np.testing.assert_allclose(colmap.qvec_to_rot(quat_of(R)), R, atol=1e-12)


def random_rotation(rng):
	q = rng.normal(size=4)
	q /= np.linalg.norm(q)
	if q[0] < 0.2:
		q[0] = 0.2 + abs(q[0])
		q /= np.linalg.norm(q)
	return colmap.qvec_to_rot(q)


@pytest.fixture()
def sparse_model(tmp_path):
	rng = np.random.default_rng(5)
	cams = {1: (1, 800, 600, (700.0, 690.0, 401.0, 299.0)),  # PINHOLE fx fy cx cy
			2: (2, 640, 480, (500.0, 320.0, 240.0, 0.01))}  # SIMPLE_RADIAL f cx cy k
	images, poses = {}, {}
	for iid in range(1, 17):
		R = random_rotation(rng)
		centre = rng.uniform(-3, 3, 3)
		t = -R @ centre
		name = f'img_{(17 - iid):03d}.png'  # name order differs from id order
		images[iid] = (name, quat_of(R), t, 1 if iid % 2 else 2, iid % 3)
		poses[name] = (R, t, centre, 1 if iid % 2 else 2)
	xyz = rng.normal(0.5, 2.0, (400, 3))
	sparse = tmp_path / 'sparse' / '0'
	sparse.mkdir(parents=True)
	write_cameras(sparse / 'cameras.bin', cams)
	write_images(sparse / 'images.bin', images)
	write_points(sparse / 'points3D.bin', xyz, rng.integers(0, 256, (400, 3)))
	return tmp_path, cams, poses, xyz


def test_readers_roundtrip(sparse_model):
	root, cams, poses, xyz = sparse_model
	sparse = os.path.join(root, 'sparse', '0')
	got = colmap.read_cameras(os.path.join(sparse, 'cameras.bin'))
	assert got == cams
	imgs = colmap.read_images(os.path.join(sparse, 'images.bin'))
	assert len(imgs) == 16
	for name, R, t, cid in imgs.values():
		np.testing.assert_allclose(R, poses[name][0], atol=1e-12)
		np.testing.assert_allclose(t, poses[name][1], atol=1e-12)
		assert cid == poses[name][3]
	pts, rgb, err, tracks = colmap.read_points(os.path.join(sparse, 'points3D.bin'))
	np.testing.assert_array_equal(pts, xyz)
	assert rgb.shape == (400, 3) and (rgb >= 0).all() and (rgb <= 1).all() and (err == 0.5).all()
	assert all(list(tr) == [1, 2] for tr in tracks)
	# quaternion convention: identity, and a quarter turn about z
	np.testing.assert_allclose(colmap.qvec_to_rot((1, 0, 0, 0)), np.eye(3))
	s = np.sqrt(0.5)
	np.testing.assert_allclose(colmap.qvec_to_rot((s, 0, 0, s)), [[0, -1, 0], [1, 0, 0], [0, 0, 1]], atol=1e-12)
	assert colmap.intrinsics(2, (500.0, 320.0, 240.0, 0.01)) == (500.0, 500.0, 320.0, 240.0)


@pytest.mark.parametrize('split', ['test', 'train'])
def test_cameras_normalised_split_and_rays(sparse_model, split):
	root, cams, poses, xyz = sparse_model
	sc = colmap.ColmapCameras(str(root), split, downsample=2, device='cpu')
	names = sorted(poses)
	want = [n for i, n in enumerate(names) if (i % 8 == 0) == (split == 'test')]
	assert sc.names == want and sc.n == len(want)
	# no image files: the resolution of the first view's camera, downsampled
	cid0 = poses[want[0]][3]
	assert (sc.W, sc.H) == (round(cams[cid0][1] / 2), round(cams[cid0][2] / 2))
	center = np.median(xyz, 0)
	scale = np.quantile(np.linalg.norm(xyz - center, axis=1), 0.98) / 0.95
	np.testing.assert_allclose(sc.normalization[0], center)
	assert sc.normalization[1] == pytest.approx(scale)
	for i, name in enumerate(sc.names):
		R, t, centre, cid = poses[name]
		fx, fy, cx, cy = colmap.intrinsics(cams[cid][0], cams[cid][3])
		sx, sy = sc.W / cams[cid][1], sc.H / cams[cid][2]
		np.testing.assert_allclose(sc.K[i].numpy(), [[fx * sx, 0, cx * sx], [0, fy * sy, cy * sy], [0, 0, 1]],
								   rtol=1e-6)
		np.testing.assert_allclose(sc.centers[i].numpy(), (centre - center) / scale, atol=1e-5)
		# the ray through the principal point is the camera's forward axis, R^T (0, 0, 1)
		px = torch.tensor([cx * sx - 0.5]); py = torch.tensor([cy * sy - 0.5])
		o, d = sc.rays(torch.tensor([i]), px, py)
		np.testing.assert_allclose(d[0].numpy(), R.T @ [0, 0, 1], atol=1e-5)
		np.testing.assert_allclose(o[0].numpy(), (centre - center) / scale, atol=1e-5)
	o, d, gt = sc.image_rays(0)
	assert o.shape == d.shape == (sc.H * sc.W, 3) and gt is None
	np.testing.assert_allclose(d.norm(dim=1).numpy(), 1.0, atol=1e-6)
	# pixel (px, py) of row-major order: the first ray of the second row is pixel (0, 1)
	_, d01 = sc.rays(torch.tensor([0]), torch.tensor([0.0]), torch.tensor([1.0]))
	np.testing.assert_allclose(d[sc.W].numpy(), d01[0].numpy(), atol=1e-6)


def test_cameras_given_normalisation_and_images(sparse_model):
	from PIL import Image
	root, cams, poses, xyz = sparse_model
	img_dir = root / 'images_4'
	img_dir.mkdir()
	names = sorted(poses)
	for k, name in enumerate(names):
		Image.fromarray(np.full((150, 200, 3), k, np.uint8)).save(img_dir / name)
	sc = colmap.ColmapCameras(str(root), 'test', downsample=4, device='cpu', load_images=True,
							  normalization=(np.zeros(3), 2.0))
	assert (sc.W, sc.H) == (200, 150)
	assert sc.images.shape == (2, 150, 200, 3) and int(sc.images[1, 0, 0, 0]) == 8
	R, t, centre, _ = poses[sc.names[1]]
	np.testing.assert_allclose(sc.centers[1].numpy(), centre / 2.0, atol=1e-5)
	_, _, gt = sc.image_rays(1)
	assert gt.shape == (150 * 200, 3) and float(gt.max()) == pytest.approx(8 / 255)
	with pytest.raises(ValueError, match='split'):
		colmap.ColmapCameras(str(root), 'val', device='cpu')


def test_truncated_file_is_an_error(tmp_path):
	p = tmp_path / 'cameras.bin'
	p.write_bytes(struct.pack('<Q', 2) + struct.pack('<iiQQ', 1, 1, 10, 10))
	with pytest.raises(ValueError, match='truncated'):
		colmap.read_cameras(str(p))


# ------------------------------------------------------------------ checkpoints

def small_field(n=60, seed=0):
	g = torch.Generator().manual_seed(seed)
	pts = torch.rand(n, 3, generator=g)
	offsets = torch.zeros(n + 1, dtype=torch.int32)
	adj = torch.zeros(0, dtype=torch.int32)
	m = VoronoiGaussField(pts, offsets, adj, torch.rand(n, 3, generator=g), torch.rand(n, generator=g) + 0.1)
	with torch.no_grad():
		for p in m.parameters():
			p.add_(torch.randn(p.shape, generator=g) * 0.1)
	m.sh_deg = 3
	return m


def reference_checkpoint(m, **extra):
	ck = {'state': m.state_dict(), 'points': m.graph.points, 'offsets': m.graph.offsets, 'adj': m.graph.adj,
		  'sh_deg': m.sh_deg, 'normalization': (np.array([0.25, -1.0, 3.5]), np.float64(4.75)),
		  'args': {'data': '/data/bonsai', 'downsample': 4, 'iters': 30000, 'lr': 0.01, 'fused': True, 'ckpt': None}}
	ck.update(extra)
	return ck


def test_checkpoint_roundtrip(tmp_path):
	m = small_field()
	path = tmp_path / 'model.pth'
	torch.save(reference_checkpoint(m), path)
	m2, ck = load_model(str(path), 'cpu')
	for (k, a), (k2, b) in zip(m.state_dict().items(), m2.state_dict().items()):
		assert k == k2 and torch.equal(a, b)
	assert m2.sh_deg == 3 and not any(p.requires_grad for p in m2.parameters())
	assert torch.equal(m2.graph.points, m.graph.points)
	center, scale = ck['normalization']
	np.testing.assert_array_equal(center, [0.25, -1.0, 3.5])
	assert float(scale) == 4.75 and ck['args']['downsample'] == 4


class Opaque:
	"""An object a checkpoint must not be allowed to construct."""


def test_checkpoint_refuses_foreign_objects_and_missing_keys(tmp_path):
	m = small_field()
	bad = tmp_path / 'bad.pth'
	torch.save(reference_checkpoint(m, args=Opaque()), bad)
	with pytest.raises(pickle.UnpicklingError):
		load_checkpoint(str(bad), 'cpu')
	partial = tmp_path / 'partial.pth'
	torch.save({'state': m.state_dict(), 'points': m.graph.points}, partial)
	with pytest.raises(KeyError, match='offsets'):
		load_checkpoint(str(partial), 'cpu')
