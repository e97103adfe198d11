"""A trained scene end to end on the GPU: a reference-format model.pth (train.py:168-170) and a COLMAP sparse model,
written here from a seeded scene, are loaded (vgr.model.load_model, vgr.colmap.ColmapCameras), packed and rendered
through a test view with render_rays_foam_infer; the foreground and transmittance match the CPU oracle on the same
rays within the parity bar, and the view matches the same camera built directly."""

import numpy as np
import pytest
import torch

import oracle
from test_trained import quat_of, write_cameras, write_images, write_points
from vgr import colmap, render, scenes, sites
from vgr.model import VoronoiGaussField, load_model

pytestmark = pytest.mark.gpu

TOL = 1e-4


def write_sparse_model(root, eyes, width, height, fov_deg=60.0):
	"""PINHOLE views looking at the origin from `eyes`, in COLMAP's world-to-camera form."""
	fx = 0.5 * width / np.tan(np.radians(fov_deg) / 2)
	cams = {1: (1, width, height, (fx, fx, 0.5 * width, 0.5 * height))}
	images = {}
	for i, eye in enumerate(eyes):
		cam = scenes.Camera(np.asarray(eye, np.float64), np.zeros(3), np.array([0.0, 1.0, 0.0]), width, height, fov_deg)
		R = cam.c2w().T  # world -> camera
		images[i + 1] = (f'view_{i:02d}.png', quat_of(R), -R @ cam.eye, 1, 0)
	sparse = root / 'sparse' / '0'
	sparse.mkdir(parents=True)
	write_cameras(sparse / 'cameras.bin', cams)
	write_images(sparse / 'images.bin', images)
	write_points(sparse / 'points3D.bin', np.random.default_rng(0).uniform(-1, 1, (64, 3)), np.zeros((64, 3), int))


def test_trained_checkpoint_and_colmap_view(gpu, tmp_path):
	sc = scenes.make_scene(1, img_scale=0.25, cache_dir=None, log=None)
	field = VoronoiGaussField.from_scene(sc, gpu)
	ck = {'state': field.state_dict(), 'points': field.graph.points, 'offsets': field.graph.offsets,
		  'adj': field.graph.adj, 'sh_deg': field.sh_deg, 'normalization': (np.zeros(3), np.float64(1.0)),
		  'args': {'data': str(tmp_path), 'downsample': 1}}
	torch.save(ck, tmp_path / 'model.pth')
	eyes = [(0.0, 0.0, 3.0)] + [(3 * np.cos(a), 0.4, 3 * np.sin(a)) for a in np.linspace(0.3, 5.9, 15)]
	write_sparse_model(tmp_path, eyes, 64, 48)

	model, ck2 = load_model(str(tmp_path / 'model.pth'), gpu)
	cams = colmap.ColmapCameras(str(tmp_path), 'test', downsample=1, device=gpu, normalization=ck2['normalization'])
	assert cams.n == 2 and (cams.W, cams.H) == (64, 48)
	o, d, _ = cams.image_rays(0)
	# the first test view is the camera at (0, 0, 3): its rays are those of the same camera built directly
	o_ref, d_ref = scenes.Camera(np.array([0.0, 0.0, 3.0]), np.zeros(3), np.array([0.0, 1.0, 0.0]), 64, 48).rays()
	np.testing.assert_allclose(d.cpu().numpy(), d_ref, atol=2e-6)
	np.testing.assert_allclose(o.cpu().numpy(), o_ref, atol=1e-6)

	start = sites.nearest_sites(model.graph.points, cams.centers[:1]).expand(len(o)).contiguous()
	pack = render.pack_foam(model, reorder=True)
	for colors, mode in (('exact', 0), ('fused', 2)):
		out = render.render_rays_foam_infer(model, pack, o, d, start, colors=colors)
		pk = {k: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v) for k, v in pack.items()}
		o_np, d_np = o.cpu().numpy(), d.cpu().numpy()
		near, _, far = render.ray_bounds(o, d, 0.02, 4.0)
		st = pk['inv'][start.cpu().numpy()].astype(np.int32)
		r = oracle.foam_infer(pk, model.sh_deg, o_np, d_np, st, near.cpu().numpy(), far.cpu().numpy(),
							  color_mode=mode)
		bg = torch.sigmoid(model.bg_logit).cpu().numpy()
		np.testing.assert_allclose(out['rgb'].cpu().numpy(), r['rgb'] + r['T'][:, None] * bg, atol=TOL)
		np.testing.assert_allclose(out['acc'].cpu().numpy(), 1 - r['T'], atol=TOL)
		assert (r['T'] < 0.999).mean() > 0.2  # the view sees the scene, not only background
