"""The field's per-site parameters as a torch module, and the loader of trained checkpoints.

VoronoiGaussField keeps the reference's class name, constructor arguments, parameter names (so a model.pth
state_dict loads into it) and methods (model.py:19-59): a density Gaussian per site (rho = exp(raw), log-scales,
rotation quaternion), a colour Gaussian (log-scales, quaternion), SH colour coefficients split into the DC term and
the rest, and a background logit. The renderers' autograd Functions (ext.foam, ext.march, ext.density, ext.color,
ext.conic) give the parameters their gradients; the optimiser and the training loop stay the reference's train.py."""

import math

import torch
import torch.nn as nn

from .ext import Graph

# SH degree-0 basis value: a site's base colour is 1/2 + SH_DC0 * sh_dc.
SH_DC0 = 0.28209479177387814
C0 = SH_DC0  # the reference's name for it (model.py:10)

# state_dict names of the per-site parameters, in the reference's order
_SITE_PARAMS = ('raw', 'd_log_scale', 'd_quat', 'c_log_scale', 'c_quat', 'sh_dc', 'sh_rest')


def identity_quat(n, device):
	"""(n, 4) unit quaternions w x y z of the identity rotation."""
	return torch.tensor([1.0, 0.0, 0.0, 0.0], device=device).repeat(n, 1)


def _opacity_density(spacing, alpha):
	"""Density rho of a Gaussian of scale `spacing` whose line integral through its centre, rho * s * sqrt(2 pi),
	is the optical depth -ln(1 - alpha) of opacity alpha."""
	return -math.log1p(-alpha) / (spacing * math.sqrt(2.0 * math.pi))


class VoronoiGaussField(nn.Module):
	"""Field over the fixed sites `points` (N, 3) with Delaunay adjacency (offsets, adj). colors (N, 3) in [0, 1]
	set the initial DC colours; spacing (N,) the initial isotropic scale of both Gaussians (clamped to >= 1e-4), and
	each density starts at the value that gives a lone Gaussian opacity init_alpha along a ray through its centre.
	sh_deg is the highest SH degree the coefficients hold; the degree in use (sh_deg attribute) starts at 0."""

	def __init__(self, points, offsets, adj, colors, spacing, init_alpha=0.1, sh_deg=3):
		super().__init__()
		n, dev = points.shape[0], points.device
		self.graph = Graph(points, offsets, adj)
		self.max_sh_deg, self.sh_deg = sh_deg, 0
		scale = spacing.clamp_min(1e-4)
		log_scale = scale.log().unsqueeze(1).expand(n, 3)
		init = {
			'raw': _opacity_density(scale, init_alpha).log(),
			'd_log_scale': log_scale, 'd_quat': identity_quat(n, dev),
			'c_log_scale': log_scale, 'c_quat': identity_quat(n, dev),
			'sh_dc': ((colors.clamp(0, 1) - 0.5) / SH_DC0).unsqueeze(1),
			'sh_rest': torch.zeros(n, 15, 3, device=dev),
		}
		for name in _SITE_PARAMS:
			self.register_parameter(name, nn.Parameter(init[name].contiguous().clone()))
		self.bg_logit = nn.Parameter(torch.zeros(3, device=dev))

	@classmethod
	def from_scene(cls, scene, device='cuda', requires_grad=False):
		"""Field holding the parameters of a synthetic scene (scenes.Scene) on `device`."""
		def on(a):
			return torch.as_tensor(a, device=device)
		n = scene.n_sites
		m = cls(on(scene.points), on(scene.offsets), on(scene.adj), torch.zeros(n, 3, device=device),
				torch.ones(n, device=device), sh_deg=max(scene.sh_deg, 0))
		sh = on(scene.sh)
		values = {'raw': on(scene.raw), 'd_log_scale': on(scene.log_scale), 'c_log_scale': on(scene.log_scale),
				  'd_quat': on(scene.quat), 'c_quat': on(scene.quat), 'sh_dc': sh[:, :1], 'sh_rest': sh[:, 1:]}
		with torch.no_grad():
			for name, v in values.items():
				getattr(m, name).copy_(v)
		m.sh_deg = scene.sh_deg
		m.requires_grad_(requires_grad)
		return m

	@property
	def n_sites(self):
		return self.raw.shape[0]

	def sh(self):
		"""(N, 16, 3) SH coefficients, DC first."""
		return torch.cat([self.sh_dc, self.sh_rest], 1)

	def walk(self, o, d, z, start):
		"""Nearest site of each sample o + z d (z sorted along each ray) by the greedy Delaunay walk."""
		return self.graph.walk(o, d, z, start)

	def param_groups(self, lr):
		"""Optimiser groups keyed like the reference's (model.py:51-59): lr is a dict with 'raw', 'scale', 'quat',
		'sh_dc', 'sh_rest' and 'bg'."""
		groups = {'raw': ['raw'], 'scale': ['d_log_scale', 'c_log_scale'], 'quat': ['d_quat', 'c_quat'],
				  'sh_dc': ['sh_dc'], 'sh_rest': ['sh_rest'], 'bg': ['bg_logit']}
		return [{'params': [getattr(self, p) for p in names], 'lr': lr[key], 'name': key}
				for key, names in groups.items()]


# numpy types a reference checkpoint's `normalization` (center array, scale scalar) is made of: the only globals the
# checkpoint loader lets the unpickler build, so loading executes nothing from the file
def _numpy_safe_globals():
	import numpy as np
	names = [np.ndarray, np.dtype, np.float64, np.float32, type(np.dtype(np.float64)), type(np.dtype(np.float32))]
	try:
		from numpy._core.multiarray import _reconstruct, scalar
	except ImportError:  # numpy < 2
		from numpy.core.multiarray import _reconstruct, scalar
	return names + [_reconstruct, scalar]


def load_checkpoint(path, device='cuda'):
	"""The dict a reference training run saves as model.pth (train.py:168-170): 'state' (the field's state_dict),
	'points', 'offsets', 'adj', 'sh_deg', 'normalization' ((center, scale) of the COLMAP scene) and 'args'. Loaded
	with torch.load(weights_only=True), numpy's array and scalar types allowed for the normalization; any other
	object in the file is refused."""
	with torch.serialization.safe_globals(_numpy_safe_globals()):
		ck = torch.load(path, map_location=device, weights_only=True)
	missing = [k for k in ('state', 'points', 'offsets', 'adj', 'sh_deg') if k not in ck]
	if missing:
		raise KeyError(f'{path}: not a voronoi-gauss checkpoint (missing {", ".join(missing)})')
	return ck


def load_model(path, device='cuda'):
	"""-> (VoronoiGaussField, checkpoint dict): the trained field of a reference model.pth, frozen for rendering
	(bench_fps.py:19-28)."""
	ck = load_checkpoint(path, device)
	pts = ck['points']
	n = len(pts)
	model = VoronoiGaussField(pts, ck['offsets'], ck['adj'], torch.zeros(n, 3, device=device),
							  torch.ones(n, device=device))
	model.load_state_dict(ck['state'])
	model.sh_deg = int(ck['sh_deg'])
	model.requires_grad_(False)
	return model, ck
