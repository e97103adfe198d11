"""Host side of the renderers: ray bounds, the packed records of the inference renderer, a NeRF-style sampler over
the field operators, and the wrappers that add the background colour.

The public functions keep the names, arguments and outputs of the reference's render.py (cited per function), so
code written against it runs unchanged; the bodies are this package's own, written around the gfx950 operators of
ext.py (libvgr.so). render_rays_foam_infer is the north-star path: one vgr_foam_infer launch per call."""

import math

import torch
import torch.nn.functional as F

from . import ext

# ---------------------------------------------------------------------------------------------------- ray bounds


def sphere_exit(o, d, radius):
	"""Ray parameter at which o + t d (unit d) leaves the sphere of `radius` about the origin: the larger root of
	t^2 + 2 (o.d) t + |o|^2 - radius^2 = 0, with a negative discriminant taken as 0 (render.py:16-19)."""
	od = (o * d).sum(-1)
	disc = od * od - ((o * o).sum(-1) - radius * radius)
	return disc.clamp_min(0).sqrt() - od


def _exit_after(o, d, radius, earliest):
	return torch.maximum(sphere_exit(o, d, radius), torch.as_tensor(earliest, dtype=o.dtype, device=o.device))


def ray_bounds(o, d, near, far_radius):
	"""(near, mid, far) per ray: near is the constant `near`; mid the exit of the unit sphere, at least near + 1e-3;
	far the exit of the sphere of radius far_radius, at least mid + 1e-3 (render.py:22-25)."""
	t_mid = _exit_after(o, d, 1.0, near + 1e-3)
	t_far = _exit_after(o, d, far_radius, t_mid + 1e-3)
	return torch.full_like(t_mid, near), t_mid, t_far


# ---------------------------------------------------------------------------------------- NeRF-style sampling


def s_to_t(s, t_near, t_mid, t_far):
	"""Ray parameter of the normalised coordinate s in [0, 1]: s in [0, 1/2] maps linearly onto [near, mid], s in
	[1/2, 1] linearly in disparity 1/t onto [mid, far] (render.py:28-33)."""
	n, m, f = t_near.unsqueeze(-1), t_mid.unsqueeze(-1), t_far.unsqueeze(-1)
	# the reference's operation order (a + (b - a) w, not torch.lerp, which rounds differently for w >= 1/2)
	inside = n + (m - n) * (2 * s).clamp(max=1.0)
	inv_m = 1.0 / m
	beyond = 1.0 / (inv_m + (2 * s - 1).clamp(min=0.0) * (1.0 / f - inv_m))
	return torch.where(s < 0.5, inside, beyond)


def sample_pdf(bins, weights, n, det=True):
	"""n samples per ray from the piecewise-constant density `weights` (+1e-5 each) over the intervals of `bins`
	(B, S + 1), by inverting its CDF at n evenly spaced (det) or uniform random levels (render.py:36-50)."""
	w = weights + 1e-5
	cdf = F.pad(torch.cumsum(w / w.sum(-1, keepdim=True), -1), (1, 0), value=0.0)
	B = bins.shape[0]
	if det:
		levels = torch.linspace(0.5 / n, 1 - 0.5 / n, n, device=bins.device, dtype=bins.dtype).expand(B, n).contiguous()
	else:
		levels = torch.rand(B, n, device=bins.device, dtype=bins.dtype)
	hi = torch.searchsorted(cdf, levels, right=True)
	i0, i1 = (hi - 1).clamp_min(0), hi.clamp_max(cdf.shape[-1] - 1)
	c0, c1 = cdf.gather(1, i0), cdf.gather(1, i1)
	span = c1 - c0
	frac = (levels - c0) / torch.where(span < 1e-5, torch.ones_like(span), span)
	b0, b1 = bins.gather(1, i0), bins.gather(1, i1)
	return b0 + frac * (b1 - b0)


def composite(sigma, t, t_far):
	"""NeRF alpha compositing of samples at t (B, S) with densities sigma: the last sample's interval reaches t_far
	(empty when t_far is before it) -> weights (B, S), final transmittance (B,) (render.py:53-57)."""
	ends = torch.cat([t, torch.maximum(t_far.unsqueeze(-1), t[:, -1:])], 1)
	alpha = 1.0 - torch.exp(-sigma * torch.diff(ends, dim=1))
	trans = torch.cumprod(F.pad(1.0 - alpha + 1e-10, (1, 0), value=1.0), 1)
	return alpha * trans[:, :-1], trans[:, -1]


def _points(o, d, t):
	"""(B * S, 3) sample points o + t d for t (B, S)."""
	return (o.unsqueeze(1) + d.unsqueeze(1) * t.unsqueeze(-1)).reshape(-1, 3)


def proposal_weights(model, o, d, s, bounds, start, scale_mult):
	"""Compositing weights at the normalised coordinates s of the density with every Gaussian widened by
	scale_mult, as a proposal for the next sampling round (render.py:60-68)."""
	t = s_to_t(s, *bounds)
	site, _ = model.walk(o, d, t, start)
	with torch.no_grad():
		sigma = ext.density(model.graph, model.raw, model.d_log_scale, model.d_quat, _points(o, d, t),
							site.reshape(-1), scale_mult)
	return composite(sigma.view_as(t), t, bounds[2])[0]


def resample(s, w, n, det):
	"""n new coordinates drawn from weights w at s, over intervals bounded by the midpoints of s and by 0 and 1."""
	edges = F.pad(F.pad(0.5 * (s[:, :-1] + s[:, 1:]), (1, 0), value=0.0), (0, 1), value=1.0)
	return sample_pdf(edges, w, n, det)


def render_rays(model, o, d, start, n_coarse=64, n_fine=(64, 64), proposal_mult=(4.0, 2.0), near=0.02,
				far_radius=4.0, perturb=True, min_weight=1e-4):
	"""NeRF-style rendering through the field operators (render.py:77-106): n_coarse stratified coordinates, then one
	proposal round per entry of n_fine (Gaussians widened by proposal_mult) each adding that many coordinates; the
	merged, sorted samples are walked to their sites, their density and (where the compositing weight exceeds
	min_weight) colour evaluated, and composited over the background. -> dict rgb (B, 3), acc, depth, walk_steps
	(mean walk steps per sample), active (fraction of samples coloured)."""
	B = o.shape[0]
	bounds = ray_bounds(o, d, near, far_radius)
	cells = torch.arange(n_coarse, device=o.device, dtype=o.dtype).expand(B, n_coarse)
	jitter = torch.rand_like(cells) if perturb else torch.full_like(cells, 0.5)
	s = (cells + jitter) / n_coarse
	with torch.no_grad():
		for n, mult in zip(n_fine, proposal_mult):
			extra = resample(s, proposal_weights(model, o, d, s, bounds, start, mult), n, det=not perturb)
			s = torch.sort(torch.cat([s, extra], 1), 1).values
		t = s_to_t(s, *bounds)
		site, steps = model.walk(o, d, t, start)
	S = t.shape[1]
	x, site = _points(o, d, t), site.reshape(-1)
	sigma = ext.density(model.graph, model.raw, model.d_log_scale, model.d_quat, x, site).view(B, S)
	w, t_last = composite(sigma, t, bounds[2])
	coloured = torch.nonzero(w.detach().reshape(-1) > min_weight).squeeze(1)
	ray_dirs = d.unsqueeze(1).expand(B, S, 3).reshape(-1, 3)
	c = ext.color(model.graph, model.c_log_scale, model.c_quat, model.sh(), x[coloured], ray_dirs[coloured],
				  site[coloured], model.sh_deg)
	per_sample = torch.zeros(B * S, 3, device=o.device, dtype=c.dtype).index_put((coloured,), c).view(B, S, 3)
	rgb = torch.einsum('bs,bsc->bc', w, per_sample) + t_last.unsqueeze(-1) * torch.sigmoid(model.bg_logit)
	return {'rgb': rgb, 'acc': 1.0 - t_last, 'depth': (w * t).sum(1), 'walk_steps': steps.float().mean() / S,
			'active': coloured.numel() / (B * S)}


# ------------------------------------------------------------------------------------ fused-kernel renderers


def _with_background(model, fg, T):
	return fg + T.unsqueeze(-1) * torch.sigmoid(model.bg_logit)


def render_rays_uniform(model, o, d, start, dt=1 / 512, n_bg=64, near=0.02, far_radius=4.0, t_thresh=1e-4,
						w_thresh=1e-4, scale_floor=None, perturb=False):
	"""One vgr_march_forward launch (render.py:109-124): steps of dt inside the unit ball, n_bg steps uniform in
	disparity beyond it, NeRF alpha, early termination at T < t_thresh; every Gaussian's scale gets scale_floor
	(default dt / 2) added in quadrature. -> dict rgb, acc, depth, samples (mean per ray), active (coloured
	fraction of the samples), walk_steps (per sample)."""
	t_near, t_mid, t_far = ray_bounds(o, d, near, far_radius)
	floor = dt / 2 if scale_floor is None else scale_floor
	conics = [ext.conic(ls, q, floor) for ls, q in ((model.d_log_scale, model.d_quat),
													(model.c_log_scale, model.c_quat))]
	fg, T, depth, stats = ext.march(model.graph, model.raw, *conics, model.sh(), model.sh_deg, o, d, start, t_near,
									t_mid, t_far, dt, n_bg, t_thresh, w_thresh)
	n_samples, n_coloured, n_steps = stats.float().sum(0).unbind()
	return {'rgb': _with_background(model, fg, T), 'acc': 1.0 - T, 'depth': depth,
			'samples': n_samples / stats.shape[0], 'active': (n_coloured / n_samples).item(),
			'walk_steps': n_steps / n_samples}


def render_rays_foam(model, o, d, start, near=0.02, far_radius=4.0, t_thresh=1e-4, w_thresh=1e-4, scale_floor=0.0,
					 perturb=False):
	"""The training renderer (render.py:127-140): samples at x(near), at every Voronoi-face crossing and at x(far),
	trapezoid compositing, one vgr_foam_forward launch with its backward under autograd (ext.foam). -> dict rgb,
	acc, depth, samples (mean per ray), active (coloured fraction of the segments), walk_steps (mean per ray)."""
	t_near, _, t_far = ray_bounds(o, d, near, far_radius)
	conics = [ext.conic(ls, q, scale_floor) for ls, q in ((model.d_log_scale, model.d_quat),
														  (model.c_log_scale, model.c_quat))]
	fg, T, depth, stats = ext.foam(model.graph, model.raw, *conics, model.sh(), model.sh_deg, o, d, start, t_near,
								   t_far, t_thresh, w_thresh)
	st = stats.float()
	segments = torch.clamp_min((st[:, 0] - 1).sum(), 1)
	return {'rgb': _with_background(model, fg, T), 'acc': 1.0 - T, 'depth': depth, 'samples': st[:, 0].mean(),
			'active': (st[:, 1].sum() / segments).item(), 'walk_steps': st[:, 2].mean()}


# ------------------------------------------------------------------------------------------------ SH basis

# Real spherical harmonics up to degree 3 in the sign convention of 3D Gaussian splatting (the constants of
# render.py:143-165 and foam_infer.cu:95-118); the kernels evaluate the same polynomials.
_SH0 = 0.28209479177387814
_SH1 = 0.4886025119029199
_SH2 = (1.0925484305920792, 0.31539156525252005, 0.5462742152960396)
_SH3 = (0.5900435899266435, 2.890611442640554, 0.4570457994644658, 0.3731763325901154, 1.445305721320277)


def sh_basis(d, deg):
	"""(B, 16) basis values at the unit directions d (B, 3), zero beyond degree `deg`."""
	x, y, z = d.unbind(-1)
	cols = [torch.full_like(x, _SH0)]
	if deg >= 1:
		cols += [-_SH1 * y, _SH1 * z, -_SH1 * x]
	if deg >= 2:
		a, b, c = _SH2
		xx, yy, zz = x * x, y * y, z * z
		cols += [a * x * y, -a * y * z, b * (2 * zz - xx - yy), -a * x * z, c * (xx - yy)]
	if deg >= 3:
		a, b, c, e, f = _SH3
		lat = 4 * zz - xx - yy
		cols += [-a * y * (3 * xx - yy), b * x * y * z, -c * y * lat, e * z * (2 * zz - 3 * xx - 3 * yy), -c * x * lat,
				 f * z * (xx - yy), -a * x * (xx - 3 * yy)]
	basis = torch.stack(cols, -1)
	return F.pad(basis, (0, 16 - basis.shape[-1]))


# ------------------------------------------------------------------------------ Z-order and the inference pack


def _dilate3(v):
	"""Spreads the low 21 bits of v (int64) so that bit i lands at bit 3 i."""
	v = v & 0x1FFFFF
	v = (v | (v << 32)) & 0x1F00000000FFFF
	v = (v | (v << 16)) & 0x1F0000FF0000FF
	v = (v | (v << 8)) & 0x100F00F00F00F00F
	v = (v | (v << 4)) & 0x10C30C30C30C30C3
	return (v | (v << 2)) & 0x1249249249249249


def morton_codes(points, bits=10):
	"""Z-order keys of the points over their bounding box, `bits` bits per axis, x in the lowest bit of each triple
	(the keys morton_order sorts, render.py:168-176): on the GPU vgr_morton_codes, on the host the same quantisation
	(p - lo) / (hi - lo) * (2^bits - 1), truncated, then bit-interleaved."""
	if points.is_cuda:
		return ext.morton_codes(points.float().contiguous(), bits)
	lo, hi = points.amin(0), points.amax(0)
	q = ((points - lo) / (hi - lo).clamp_min(1e-12) * (2 ** bits - 1)).long()
	return _dilate3(q[:, 0]) | (_dilate3(q[:, 1]) << 1) | (_dilate3(q[:, 2]) << 2)


def morton_order(points, bits=10):
	"""Permutation that sorts the points along the Z-order curve of their bounding box (render.py:168-176)."""
	return torch.argsort(morton_codes(points, bits))


def cut_bits(r2, lam):
	"""float32 words whose bits are two halves, r2 in the low 16 bits and lam in the high 16, each rounded to the
	nearest even half (the packing of render.py:197)."""
	lo = r2.half().view(torch.int16).to(torch.int32) & 0xFFFF
	hi = lam.half().view(torch.int16).to(torch.int32) << 16
	return (lo | hi).view(torch.float32)


def _cut_words(raw, d_log_scale, c_log_scale, scale_floor, eps_density):
	"""Per site, the word of half2(r2, lam): r2 the squared distance beyond which exp(raw) G(x) < eps_density
	(2 s_max^2 max(raw - ln eps, 0), +inf when eps_density = 0) and lam the smallest eigenvalue of the colour conic,
	each moved by 2^-9 to the safe side of its half rounding, lam at most 65000."""
	floor2 = scale_floor * scale_floor
	if eps_density > 0:
		s_max2 = (torch.exp(2 * d_log_scale.clamp(-20, 20)) + floor2).amax(-1)
		r2 = 2 * s_max2 * (raw - math.log(eps_density)).clamp_min(0) * (1 + 2 ** -9)
	else:
		r2 = torch.full_like(raw, math.inf)
	lam = 1.0 / (torch.exp(2 * c_log_scale.clamp(-20, 20)) + floor2).amax(-1)
	return cut_bits(r2, (lam * (1 - 2 ** -9)).clamp(max=65000.0))


@torch.no_grad()
def pack_foam_arrays(points, offsets, adj, raw, d_log_scale, c_log_scale, dA, cA, sh, scale_floor=0.0,
					 eps_density=0.0, sh_half=False, reorder=False):
	"""The inference records (the format of render.py:179-225) from plain tensors with the conics given, in torch
	on any device; pack_foam builds the same records on the GPU. Each site's neighbourhood is listed self first,
	then its Delaunay neighbours in CSR order, as one stable sort of (cell, entry) pairs; renumbering (reorder)
	is a second stable sort by the cells' new numbers, which keeps every neighbourhood's order.
	-> dict points (N, 4), offsets (N + 1), nbr (E), edge (E, 4), attr (N, 20), sh, sh32, perm, inv, orig."""
	n, dev = points.shape[0], points.device
	raw = raw.clamp(max=30.0)
	ids = torch.arange(n, device=dev)
	deg = (offsets[1:] - offsets[:-1]).long()
	cell = torch.cat([ids, torch.repeat_interleave(ids, deg)])  # selves first, then the CSR rows
	member = torch.cat([ids, adj.long()])
	order = torch.argsort(cell, stable=True)
	cell, nbr = cell[order], member[order]
	words = _cut_words(raw, d_log_scale, c_log_scale, scale_floor, eps_density)
	edge = torch.cat([points[nbr], words[nbr].unsqueeze(1)], 1)
	pts4 = F.pad(points, (0, 1))
	attr = points.new_zeros(n, 20)
	attr[:, 0:6], attr[:, 6], attr[:, 8:14] = dA, raw, cA
	sizes = deg + 1
	perm = inv = None
	if reorder:
		perm = morton_order(points)
		inv = torch.empty_like(perm)
		inv[perm] = ids
		regroup = torch.argsort(inv[cell], stable=True)
		nbr, edge = inv[nbr[regroup]], edge[regroup]
		pts4, attr, sh, sizes = pts4[perm], attr[perm], sh[perm], sizes[perm]
	offsets_sf = F.pad(torch.cumsum(sizes, 0), (1, 0))
	sh = sh.contiguous()
	return {'points': pts4.contiguous(), 'offsets': offsets_sf.int(), 'nbr': nbr.int().contiguous(),
			'edge': edge.contiguous(), 'attr': attr.contiguous(), 'sh': sh.half() if sh_half else sh, 'sh32': sh,
			'perm': perm, 'inv': inv, 'orig': (perm if reorder else torch.empty(0, device=dev)).int().contiguous(),
			'baked_center': None}


@torch.no_grad()
def pack_foam(model, scale_floor=0.0, eps_density=0.0, sh_half=False, reorder=False, index=True):
	"""The inference renderer's records for a field (render.py:179-225), built on the GPU by vgr_pack_foam (the
	renumbering's Z-order sort by torch): self-first neighbourhoods (offsets (N + 1), nbr (E)), one float4 per
	neighbourhood entry (p_j, half2(r2_j, lam_j)), attr (N, 20) = (density conic, min(raw, 30), colour conic,
	baked rgb), sh in fp32 or fp16; reorder renumbers the sites along a Z-order curve (perm: new -> old, inv: old ->
	new, orig: the tie order of the original numbering). index (an addition to the reference's arguments): also
	build the derived records of index_pack (+16 B per neighbourhood entry and 208 B per site), through which
	render_rays_foam_infer renders fused and exact colours fastest; index=False gives the reference's pack alone."""
	g = model.graph
	dA = ext.conic(model.d_log_scale, model.d_quat, scale_floor)
	cA = ext.conic(model.c_log_scale, model.c_quat, scale_floor)
	perm = inv = None
	if reorder:
		perm = morton_order(g.points)
		inv = torch.empty_like(perm)
		inv[perm] = torch.arange(len(perm), device=perm.device)
	out = ext.pack_foam(g.points, g.offsets, g.adj, *[t.detach().contiguous() for t in (
		model.raw, model.d_log_scale, model.c_log_scale, dA, cA)], model.sh().detach().float().contiguous(), perm,
		scale_floor, eps_density, sh_half)
	empty = torch.empty(0, device=g.points.device)
	pack = {'points': out['points'], 'offsets': out['offsets'], 'nbr': out['nbr'], 'edge': out['edge'],
			'attr': out['attr'], 'sh': out['sh16'] if sh_half else out['sh32'], 'sh32': out['sh32'], 'perm': perm,
			'inv': inv, 'orig': (empty if perm is None else perm).int().contiguous(), 'baked_center': None}
	return index_pack(pack) if index else pack


@torch.no_grad()
def index_pack(pack):
	"""Adds the indexed edge records (ext.index_pack: edge_i, attr_i) and the slot table of the reference's colour
	cache (ext.slot_table: slots) to a GPU pack; render_rays_foam_infer then renders fused colours with one record
	stream per neighbourhood entry, bit-identical to the reference records, and counts the cache misses of
	stats[:, 4] once per neighbourhood pass; and the site rows that the group layouts' fused blend reads (rows:
	the first 16 columns of the records; with fp32 SH, 256-byte site blocks (N, 64) that hold the SH row after
	them, so a neighbour visit reads two 128-byte lines for both, else 64-byte rows (N, 16), two per line). A
	snapshot: call again after changing the pack."""
	pack['edge_i'], pack['attr_i'] = ext.index_pack(pack['offsets'], pack['nbr'], pack['edge'], pack['attr'])
	pack['slots'] = ext.slot_table(pack['offsets'], pack['nbr'])
	n = pack['attr_i'].size(0)
	if pack['sh'].dtype == torch.float32:
		pack['rows'] = torch.cat([pack['attr_i'][:, :16], pack['sh'].reshape(n, 48)], 1).contiguous()
	else:
		pack['rows'] = pack['attr_i'][:, :16].contiguous()
	return pack


@torch.no_grad()
def bake_colors(model, pack, center):
	"""Bakes one view's site colours max(SH_k(d_k) + 1/2, 0), d_k the unit direction from `center` to site k, into
	the packed records (attr[:, 16:19]) for the baked colour mode (render.py:228-235): vgr_bake_colors for packs on
	the GPU, torch for host packs."""
	if pack['attr'].is_cuda:
		ext.bake_colors(pack['points'], pack['sh32'], model.sh_deg, center, pack['attr'])
	else:
		sites = pack['points'][:, :3]
		basis = sh_basis(F.normalize(sites - center.view(1, 3), dim=-1), model.sh_deg)
		pack['attr'][:, 16:19] = torch.einsum('nj,njc->nc', basis, pack['sh32']).add(0.5).clamp_min(0.0)
	pack['baked_center'] = center


# ------------------------------------------------------------------------------------- inference renderer

_COLOR_MODES = {'exact': 0, 'baked': 1, 'fused': 2}


@torch.no_grad()
def render_rays_foam_infer(model, pack, o, d, start, near=0.02, far_radius=4.0, t_thresh=1e-4, w_thresh=1e-4,
						   colors='exact', eps_color=0.0, stage=2, cap=None, trace_cap=0):
	"""Rendering at the ray / Voronoi-face crossings with the packed records, one vgr_foam_infer launch
	(render.py:238-257). colors: 'exact' (SH evaluated in a second pass for segments of weight > w_thresh),
	'fused' (blended in the density pass) or 'baked' (bake_colors); eps_color > 0 skips colour terms of relative
	weight below it. start: sites in the model's numbering. -> dict rgb (with the background), acc, depth, stats
	(B, 5): samples, coloured segments, walk steps, density terms, SH evaluations; with trace_cap > 0 also trace
	(B, trace_cap), each sample's cell in the model's numbering. A pack with indexed records (index_pack) renders
	fused colours through them, and exact colours with eps_color = 0 too, as the one-pass blend (the same normalised
	sum over the neighbours, kept relative to a running minimum; the statistics are the exact mode's)."""
	t_near, _, t_far = ray_bounds(o, d, near, far_radius)
	if pack['inv'] is not None:
		start = pack['inv'][start.long()]
	empty = torch.empty(0, dtype=torch.int32, device=o.device)
	out = ext.foam_infer_extension().foam_infer(
		pack['points'], pack['offsets'], pack['nbr'], pack['edge'], pack['attr'], pack['sh'], model.sh_deg,
		o.float().contiguous(), d.float().contiguous(), start.int().contiguous(), t_near.contiguous(),
		t_far.contiguous(), float(t_thresh), float(w_thresh), 2 * math.log(1 / eps_color) if eps_color > 0 else math.inf,
		_COLOR_MODES[colors], int(stage), empty if cap is None else cap.int().contiguous(), pack['orig'],
		trace_cap=trace_cap, indexed=(pack['edge_i'], pack['attr_i'], pack.get('rows')) if 'edge_i' in pack else None,
		slots=pack.get('slots'))
	fg, T, depth, stats = out[:4]
	res = {'rgb': _with_background(model, fg, T), 'acc': 1.0 - T, 'depth': depth, 'stats': stats}
	if trace_cap > 0:
		res['trace'] = out[4]
	return res


@torch.no_grad()
def render_image(model, scene, i, start, chunk=8192, renderer=render_rays, **kw):
	"""View i of a scene with image_rays(i) -> (o, d, gt), rendered `chunk` rays at a time from the start site
	`start` -> (image (H, W, 3) clamped to [0, 1], gt) (render.py:260-266)."""
	o, d, gt = scene.image_rays(i)
	starts = torch.full((o.shape[0],), int(start), dtype=torch.int32, device=o.device)
	parts = [renderer(model, o[a:a + chunk], d[a:a + chunk], starts[a:a + chunk], perturb=False, **kw)['rgb']
			 for a in range(0, o.shape[0], chunk)]
	return torch.cat(parts).view(scene.H, scene.W, 3).clamp(0, 1), gt
