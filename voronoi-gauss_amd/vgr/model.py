"""Per-site parameters of the field (model.py:19-59 of the reference): density Gaussian (rho = exp(raw), scale,
rotation), colour Gaussian (scale, rotation), SH colour (sh_dc + sh_rest) and a background logit.

They are nn.Parameters: the renderers' autograd Functions (ext.foam, ext.march, ext.density, ext.color, ext.conic)
give them gradients; the optimiser and the training loop are the reference's own train.py."""

import math

import torch
import torch.nn as nn

from .ext import Graph

C0 = 0.28209479177387814


def identity_quat(n, device):
	q = torch.zeros(n, 4, device=device)
	q[:, 0] = 1.0
	return q


class VoronoiGaussField(nn.Module):
	"""points (N, 3) fixed sites; offsets/adj their Delaunay adjacency; colors (N, 3) in [0, 1]; spacing (N,)
	mean distance to the nearest sites, used as the initial isotropic scale of both Gaussians."""

	def __init__(self, points, offsets, adj, colors, spacing, init_alpha=0.1, sh_deg=3):
		super().__init__()
		device = points.device
		n = len(points)
		self.graph = Graph(points, offsets, adj)
		self.max_sh_deg, self.sh_deg = sh_deg, 0
		s = spacing.clamp_min(1e-4)
		# a ray through the centre of a lone Gaussian has opacity init_alpha: rho s sqrt(2 pi) = -ln(1 - a)
		rho = -math.log(1.0 - init_alpha) / (s * math.sqrt(2.0 * math.pi))
		self.raw = nn.Parameter(rho.log())
		self.d_log_scale = nn.Parameter(s.log()[:, None].repeat(1, 3))
		self.d_quat = nn.Parameter(identity_quat(n, device))
		self.c_log_scale = nn.Parameter(s.log()[:, None].repeat(1, 3))
		self.c_quat = nn.Parameter(identity_quat(n, device))
		self.sh_dc = nn.Parameter(((colors.clamp(0, 1) - 0.5) / C0)[:, None])
		self.sh_rest = nn.Parameter(torch.zeros(n, 15, 3, device=device))
		self.bg_logit = nn.Parameter(torch.zeros(3, device=device))

	@classmethod
	def from_scene(cls, scene, device='cuda', requires_grad=False):
		"""Field holding a synthetic scene's parameters (scenes.Scene) on `device`."""
		t = lambda a: torch.as_tensor(a, device=device)  # noqa: E731
		n = scene.n_sites
		m = cls(t(scene.points), t(scene.offsets), t(scene.adj), torch.zeros(n, 3, device=device),
				torch.ones(n, device=device), sh_deg=max(scene.sh_deg, 0))
		with torch.no_grad():
			m.raw.copy_(t(scene.raw))
			m.d_log_scale.copy_(t(scene.log_scale))
			m.c_log_scale.copy_(t(scene.log_scale))
			m.d_quat.copy_(t(scene.quat))
			m.c_quat.copy_(t(scene.quat))
			sh = t(scene.sh)
			m.sh_dc.copy_(sh[:, :1])
			m.sh_rest.copy_(sh[:, 1:])
		m.sh_deg = scene.sh_deg
		m.requires_grad_(requires_grad)
		return m

	@property
	def n_sites(self):
		return len(self.raw)

	def sh(self):
		return torch.cat([self.sh_dc, self.sh_rest], 1)

	def walk(self, o, d, z, start):
		return self.graph.walk(o, d, z, start)


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
