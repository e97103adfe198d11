"""Operator boundary of the renderers and field operators: the reference's ext.py API (ext.py:11-216) backed by the
hand-written gfx950 kernels of libvgr.so instead of JIT-built CUDA extensions.

Same names, argument meaning and error behaviour as the reference:
  extension().walk / density_forward / color_forward / conic_forward       (csrc/vgf.cu:438-546)
  extension().density_backward / color_backward / conic_backward          (csrc/vgf.cu:121-148,179-198,284-424)
  march_extension().march_forward / march_backward                         (csrc/march.cu:383-428)
  foam_extension().foam_forward / foam_backward                            (csrc/foam.cu:471-531)
  foam_infer_extension().foam_infer                                        (csrc/foam_infer.cu:376-435)
  Graph, density, color, conic, conic_reference, march, foam               (ext.py:46-216)
Inputs are checked like the reference's TORCH_CHECKs (CUDA, contiguous, dtype, shapes) and a violation raises
RuntimeError; outputs are allocated here with torch on the input's device and the kernels run asynchronously on
torch's current stream. density, color, conic, march and foam are autograd Functions whose backward runs the
gradient kernels."""

import os

import torch

from . import _lib
from ._lib import call, ptr, stream_of


def _check(x, name, dtype):
	if not isinstance(x, torch.Tensor) or not x.is_cuda:
		raise RuntimeError(f'{name} must be a CUDA tensor')
	if not x.is_contiguous():
		raise RuntimeError(f'{name} must be contiguous')
	if x.dtype != dtype:
		raise RuntimeError(f'{name} has the wrong dtype')


def _require(cond, msg):
	if not cond:
		raise RuntimeError(msg)


# ============================================================================ vgf.cu forward operators

class _FieldExtension:
	"""Forward operators of csrc/vgf.cu (walk, density_forward, color_forward, conic_forward)."""

	@staticmethod
	def walk(points, offsets, adj, o, d, z, start):
		for t, n, dt in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32),
						 (adj, 'adj', torch.int32), (o, 'o', torch.float32), (d, 'd', torch.float32),
						 (z, 'z', torch.float32), (start, 'start', torch.int32)):
			_check(t, n, dt)
		B, S = z.size(0), z.size(1)
		site = torch.empty(B, S, dtype=torch.int32, device=z.device)
		steps = torch.empty(B, dtype=torch.int32, device=z.device)
		if B == 0:
			return [site, steps]
		with torch.cuda.device(z.device):
			call('vgr_walk', ptr(points), points.size(0), ptr(offsets), ptr(adj), adj.numel(), ptr(o), ptr(d),
				 ptr(z), ptr(start), B, S, ptr(site), ptr(steps), stream_of(z.device))
		return [site, steps]

	@staticmethod
	def density_forward(points, offsets, adj, raw, log_scale, quat, x, site, scale_mult, records=True):
		"""records: give the library scratch for per-site Gaussian records (used when m >= N / 8; same bits)."""
		for t, n, dt in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32),
						 (adj, 'adj', torch.int32), (log_scale, 'log_scale', torch.float32),
						 (quat, 'quat', torch.float32), (raw, 'raw', torch.float32), (x, 'x', torch.float32),
						 (site, 'site', torch.int32)):
			_check(t, n, dt)
		m = x.size(0)
		sigma = torch.empty(m, dtype=torch.float32, device=x.device)
		if m == 0:
			return sigma
		work, wb = _field_work(points, m, records)
		with torch.cuda.device(x.device):
			call('vgr_density_forward', ptr(points), points.numel() // 3, ptr(offsets), ptr(adj), adj.numel(),
				 ptr(raw), ptr(log_scale), ptr(quat), ptr(x), ptr(site), m, float(scale_mult), ptr(sigma),
				 ptr(work), wb, stream_of(x.device))
		return sigma

	@staticmethod
	def color_forward(points, offsets, adj, log_scale, quat, sh, sh_deg, x, dirs, site, records=True):
		"""records: as for density_forward."""
		for t, n, dt in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32),
						 (adj, 'adj', torch.int32), (log_scale, 'log_scale', torch.float32),
						 (quat, 'quat', torch.float32), (sh, 'sh', torch.float32), (x, 'x', torch.float32),
						 (dirs, 'dirs', torch.float32), (site, 'site', torch.int32)):
			_check(t, n, dt)
		_require(sh.dim() == 3 and sh.size(1) == 16 and sh.size(2) == 3, 'sh must be (N, 16, 3)')
		m = x.size(0)
		rgb = torch.empty(m, 3, dtype=torch.float32, device=x.device)
		if m == 0:
			return rgb
		work, wb = _field_work(points, m, records)
		with torch.cuda.device(x.device):
			call('vgr_color_forward', ptr(points), points.numel() // 3, ptr(offsets), ptr(adj), adj.numel(),
				 ptr(log_scale), ptr(quat), ptr(sh), int(sh_deg), ptr(x), ptr(dirs), ptr(site), m, ptr(rgb),
				 ptr(work), wb, stream_of(x.device))
		return rgb

	@staticmethod
	def conic_forward(log_scale, quat, floor):
		_check(log_scale, 'log_scale', torch.float32)
		_check(quat, 'quat', torch.float32)
		n = quat.size(0)
		A = torch.empty(n, 6, dtype=torch.float32, device=quat.device)
		if n == 0:
			return A
		with torch.cuda.device(quat.device):
			call('vgr_conic_forward', ptr(log_scale), ptr(quat), n, float(floor), ptr(A), stream_of(quat.device))
		return A

	@staticmethod
	def density_backward(points, offsets, adj, raw, log_scale, quat, x, site, grad_sigma, gather=False):
		"""-> g_raw (N,), g_ls (N, 3), g_quat (N, 4) (vgf.cu:477-492). gather: the gradients gathered per site through
		a workspace from torch's allocator (vgr_density_backward_work_size), else (the default, faster for density:
		8 atomics per sample and neighbour against a per-site loop that is as long as the busiest site of its wave)
		scattered with atomics."""
		for t, n, dt in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32),
						 (adj, 'adj', torch.int32), (raw, 'raw', torch.float32),
						 (log_scale, 'log_scale', torch.float32), (quat, 'quat', torch.float32), (x, 'x', torch.float32),
						 (site, 'site', torch.int32), (grad_sigma, 'grad_sigma', torch.float32)):
			_check(t, n, dt)
		g_raw, g_ls, g_quat = torch.zeros_like(raw), torch.zeros_like(log_scale), torch.zeros_like(quat)
		m = x.size(0)
		if m == 0:
			return g_raw, g_ls, g_quat
		work, wb = None, 0
		if gather:
			wb = int(_lib.load().vgr_density_backward_work_size(points.numel() // 3, m))
			work = torch.empty(wb, dtype=torch.uint8, device=x.device)
		with torch.cuda.device(x.device):
			call('vgr_density_backward', ptr(points), points.numel() // 3, ptr(offsets), ptr(adj), adj.numel(),
				 ptr(raw), ptr(log_scale), ptr(quat), ptr(x), ptr(site), m, ptr(grad_sigma), ptr(g_raw), ptr(g_ls),
				 ptr(g_quat), ptr(work), wb, stream_of(x.device))
		return g_raw, g_ls, g_quat

	@staticmethod
	def color_backward(points, offsets, adj, log_scale, quat, sh, sh_deg, x, dirs, site, rgb, grad_rgb, gather=True):
		"""-> g_ls (N, 3), g_quat (N, 4), g_sh (N, 16, 3) (vgf.cu:515-533). gather (the default): the gradients
		gathered per site through a workspace from torch's allocator (vgr_color_backward_work_size), else scattered
		with up to 55 atomics per sample and neighbour."""
		for t, n, dt in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32),
						 (adj, 'adj', torch.int32), (log_scale, 'log_scale', torch.float32),
						 (quat, 'quat', torch.float32), (sh, 'sh', torch.float32), (x, 'x', torch.float32),
						 (dirs, 'dirs', torch.float32), (site, 'site', torch.int32), (rgb, 'rgb', torch.float32),
						 (grad_rgb, 'grad_rgb', torch.float32)):
			_check(t, n, dt)
		_require(sh.dim() == 3 and sh.size(1) == 16 and sh.size(2) == 3, 'sh must be (N, 16, 3)')
		g_ls, g_quat, g_sh = torch.zeros_like(log_scale), torch.zeros_like(quat), torch.zeros_like(sh)
		m = x.size(0)
		if m == 0:
			return g_ls, g_quat, g_sh
		work, wb = None, 0
		if gather:
			wb = int(_lib.load().vgr_color_backward_work_size(points.numel() // 3, m))
			work = torch.empty(wb, dtype=torch.uint8, device=x.device)
		with torch.cuda.device(x.device):
			call('vgr_color_backward', ptr(points), points.numel() // 3, ptr(offsets), ptr(adj), adj.numel(),
				 ptr(log_scale), ptr(quat), ptr(sh), int(sh_deg), ptr(x), ptr(dirs), ptr(site), m, ptr(rgb),
				 ptr(grad_rgb), ptr(g_ls), ptr(g_quat), ptr(g_sh), ptr(work), wb, stream_of(x.device))
		return g_ls, g_quat, g_sh

	@staticmethod
	def conic_backward(log_scale, quat, floor, gA):
		"""-> g_ls (n, 3), g_quat (n, 4) (vgf.cu:548-560)."""
		for t, n, dt in ((log_scale, 'log_scale', torch.float32), (quat, 'quat', torch.float32),
						 (gA, 'gA', torch.float32)):
			_check(t, n, dt)
		g_ls, g_quat = torch.empty_like(log_scale), torch.empty_like(quat)
		n = quat.size(0)
		if n == 0:
			return g_ls, g_quat
		with torch.cuda.device(quat.device):
			call('vgr_conic_backward', ptr(log_scale), ptr(quat), n, float(floor), ptr(gA), ptr(g_ls), ptr(g_quat),
				 stream_of(quat.device))
		return g_ls, g_quat


def _field_work(points, m, records):
	"""Scratch for the per-site Gaussian records of density_forward / color_forward when the call is large enough
	for the library to use them (m >= N / 8), else (None, 0)."""
	n = points.numel() // 3
	if not records or m * 8 < n:
		return None, 0
	wb = int(_lib.load().vgr_field_work_size(n))
	return torch.empty(wb, dtype=torch.uint8, device=points.device), wb


# ============================================================================ march.cu forward

class _MarchExtension:
	@staticmethod
	def march_forward(points, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, start, near, mid, far, dt, n_bg,
					  t_thresh, w_thresh, trace_cap=0, lanes=0, work=None, order=None):
		"""-> [rgb (B, 3), T (B,), depth (B,), stats (B, 3) int32] (+ trace (B, trace_cap) when trace_cap > 0).
		lanes: 1 ray per lane (1), 16 lanes per ray (16) or by batch size (0). work: optional uint8 device workspace
		(at least vgr_march_work_size bytes); a training step passes the backward's, which then reuses its blocks.
		order: optional int32 (B,) permutation of 0 .. B - 1, the order in which the rays are traced
		(a ray it leaves out keeps uninitialised outputs; VGR_CHECK_ORDER=1 verifies it) (ray_order); same results."""
		for t, n, dtp in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32),
						  (adj, 'adj', torch.int32), (raw, 'raw', torch.float32), (dA, 'dA', torch.float32),
						  (cA, 'cA', torch.float32), (sh, 'sh', torch.float32), (o, 'o', torch.float32),
						  (d, 'd', torch.float32), (start, 'start', torch.int32), (near, 'near', torch.float32),
						  (mid, 'mid', torch.float32), (far, 'far', torch.float32)):
			_check(t, n, dtp)
		_require(sh.dim() == 3 and sh.size(1) == 16 and sh.size(2) == 3, 'sh must be (N, 16, 3)')
		_require(dA.size(1) == 6 and cA.size(1) == 6, 'conics must be (N, 6)')
		B = o.size(0)
		dev = o.device
		rgb = torch.empty(B, 3, dtype=torch.float32, device=dev)
		T = torch.empty(B, dtype=torch.float32, device=dev)
		depth = torch.empty(B, dtype=torch.float32, device=dev)
		stats = torch.empty(B, 3, dtype=torch.int32, device=dev)
		trace = torch.full((B, trace_cap), -1, dtype=torch.int32, device=dev) if trace_cap > 0 else None
		out = [rgb, T, depth, stats] + ([trace] if trace is not None else [])
		if B == 0:
			return out
		work_bytes = int(_lib.load().vgr_march_work_size(points.numel() // 3, int(sh_deg)))
		if work is None:
			work = torch.empty(max(work_bytes, 1), dtype=torch.uint8, device=dev)
		else:
			work_bytes = work.numel()
		with torch.cuda.device(dev):
			call('vgr_march_forward_lanes', ptr(points), points.numel() // 3, ptr(offsets), ptr(adj), adj.numel(),
				 ptr(raw), ptr(dA), ptr(cA), ptr(sh), int(sh_deg), ptr(o), ptr(d), ptr(start), ptr(near), ptr(mid),
				 ptr(far), B, float(dt), int(n_bg), float(t_thresh), float(w_thresh), ptr(rgb), ptr(T), ptr(depth),
				 ptr(stats), ptr(trace), int(trace_cap), ptr(_order(order, B, dev)), int(lanes), ptr(work), work_bytes,
				 stream_of(dev))
		return out

	@staticmethod
	def march_backward(points, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, start, near, mid, far, dt, n_bg,
					   t_thresh, w_thresh, rgb, T, g_rgb, g_T, lanes=0, work=None):
		"""-> [g_raw (N,), g_dA (N, 6), g_cA (N, 6), g_sh (N, 16, 3)] (march.cu:405-428). lanes: the layout of the
		forward that produced rgb and T. work: the forward's workspace (vgr_march_backward_work_size bytes), whose
		site blocks are reused, or None to pack them again."""
		for t, n, dtp in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32),
						  (adj, 'adj', torch.int32), (raw, 'raw', torch.float32), (dA, 'dA', torch.float32),
						  (cA, 'cA', torch.float32), (sh, 'sh', torch.float32), (o, 'o', torch.float32),
						  (d, 'd', torch.float32), (start, 'start', torch.int32), (near, 'near', torch.float32),
						  (mid, 'mid', torch.float32), (far, 'far', torch.float32), (rgb, 'rgb', torch.float32),
						  (T, 'T', torch.float32), (g_rgb, 'g_rgb', torch.float32), (g_T, 'g_T', torch.float32)):
			_check(t, n, dtp)
		_require(sh.dim() == 3 and sh.size(1) == 16 and sh.size(2) == 3, 'sh must be (N, 16, 3)')
		_require(dA.size(1) == 6 and cA.size(1) == 6, 'conics must be (N, 6)')
		B, dev = o.size(0), o.device
		_require(rgb.shape == g_rgb.shape == (B, 3) and T.shape == g_T.shape == (B,),
				 'rgb, g_rgb must be (B, 3) and T, g_T (B,)')
		n = points.numel() // 3
		g = [torch.empty(n, device=dev), torch.empty(n, 6, device=dev), torch.empty(n, 6, device=dev),
			 torch.empty(n, 16, 3, device=dev)]
		work_bytes = int(_lib.load().vgr_march_backward_work_size(n, int(sh_deg)))
		ready = work is not None
		if ready:
			_require(work.dtype == torch.uint8 and work.numel() >= work_bytes, 'work is too small')
			work_bytes = work.numel()
		else:
			work = torch.empty(max(work_bytes, 1), dtype=torch.uint8, device=dev)
		with torch.cuda.device(dev):
			call('vgr_march_backward', ptr(points), n, ptr(offsets), ptr(adj), adj.numel(), ptr(raw), ptr(dA),
				 ptr(cA), ptr(sh), int(sh_deg), ptr(o), ptr(d), ptr(start), ptr(near), ptr(mid), ptr(far), B,
				 float(dt), int(n_bg), float(t_thresh), float(w_thresh), ptr(rgb), ptr(T), ptr(g_rgb), ptr(g_T),
				 *[ptr(x) for x in g], int(lanes), int(ready), ptr(work), work_bytes, stream_of(dev))
		return g


# ============================================================================ foam_infer.cu

class _FoamInferExtension:
	@staticmethod
	def foam_infer(points, offsets, nbr, edge, attr, sh, sh_deg, o, d, start, near, far, t_thresh, w_thresh,
				   color_cut, color_mode, stage, cap, orig, trace_cap=0, lanes=None, order=None, indexed=None,
				   slots=None):
		"""-> [rgb (B, 3), T (B,), depth (B,), stats (B, 5) int32] (+ trace (B, trace_cap) int32, the cell of
		every sample in original numbering, -1 past the last sample, when trace_cap > 0). lanes: None for the
		library's default layout, else 1 (one ray per lane) or 2 / 4 / 8 (that many lanes per ray,
		vgr_foam_infer_lanes). order: optional int32 (B,) permutation of 0 .. B - 1, the order in which the rays are traced
		(a ray it leaves out keeps uninitialised outputs; VGR_CHECK_ORDER=1 verifies it)
		(ray_order); the results are the same. indexed: optional (edge_i, attr_i) from index_pack, read by the
		fused rendering with one ray per lane in place of nbr / edge / attr (vgr_foam_infer_indexed, bit-identical
		results), or (edge_i, attr_i, rows) with site rows that the group layouts' fused blend then reads in place
		of attr (bit-identical results): the 64-byte rows (N, 16), or 256-byte site blocks (N, 64) whose last 48
		floats are the fp32 SH row (sh must then be float32), read in place of sh too; other stages, colour modes
		and layouts ignore them. slots: optional int32 (N, 16) slot table
		(slot_table) of the same pack: with color_cut = +inf the reference's colour-cache misses (stats[:, 4]) are
		counted from it once per neighbourhood pass instead of per lookup (the same counts, faster)."""
		for t, n, dt in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32),
						 (nbr, 'nbr', torch.int32), (edge, 'edge', torch.float32), (attr, 'attr', torch.float32),
						 (o, 'o', torch.float32), (d, 'd', torch.float32), (start, 'start', torch.int32),
						 (near, 'near', torch.float32), (far, 'far', torch.float32), (cap, 'cap', torch.int32),
						 (orig, 'orig', torch.int32)):
			_check(t, n, dt)
		_require(isinstance(sh, torch.Tensor) and sh.is_cuda and sh.is_contiguous(),
				 'sh must be a contiguous CUDA tensor')
		half = sh.dtype == torch.float16
		_require(half or sh.dtype == torch.float32, 'sh must be float32 or float16')
		n = points.size(0)
		_require(points.dim() == 2 and points.size(1) == 4, 'points must be (N, 4)')
		_require(offsets.numel() == n + 1, 'offsets must be (N + 1)')
		_require(edge.dim() == 2 and edge.size(1) == 4 and edge.size(0) == nbr.numel(), 'edge must be (E, 4)')
		_require(attr.dim() == 2 and attr.size(1) == 20 and attr.size(0) == n, 'attr must be (N, 20)')
		_require(0 <= color_mode <= 2, 'color_mode must be 0 (lazy), 1 (baked) or 2 (fused)')
		baked = color_mode == 1
		_require(baked or (sh.dim() == 3 and sh.size(0) == n and sh.size(1) == 16 and sh.size(2) == 3),
				 'sh must be (N, 16, 3)')
		_require(0 <= stage <= 2, 'stage must be 0, 1 or 2')
		B = o.size(0)
		dev = o.device
		rgb = torch.empty(B, 3, dtype=torch.float32, device=dev)
		T = torch.empty(B, dtype=torch.float32, device=dev)
		depth = torch.empty(B, dtype=torch.float32, device=dev)
		stats = torch.empty(B, 5, dtype=torch.int32, device=dev)
		trace = torch.full((B, trace_cap), -1, dtype=torch.int32, device=dev) if trace_cap > 0 else None
		out = [rgb, T, depth, stats] + ([trace] if trace is not None else [])
		if B == 0:
			return out
		cp = cap if cap.numel() == B else None
		og = orig if orig.numel() == n else None
		args = [ptr(points), n, ptr(offsets), ptr(nbr), ptr(edge), nbr.numel(), ptr(attr),
				None if baked else ptr(sh), int(half), int(sh_deg), ptr(o), ptr(d), ptr(start), ptr(near), ptr(far), B,
				float(t_thresh), float(w_thresh), float(color_cut), int(color_mode), int(stage), ptr(cp), ptr(og),
				ptr(rgb), ptr(T), ptr(depth), ptr(stats)]
		rows = None
		if indexed is not None:
			edge_i, attr_i = indexed[0], indexed[1]
			rows = indexed[2] if len(indexed) > 2 else None
			_check(edge_i, 'edge_i', torch.float32)
			_check(attr_i, 'attr_i', torch.float32)
			_require(edge_i.shape == edge.shape and attr_i.shape == attr.shape,
					 'edge_i and attr_i must have the shapes of edge and attr')
			if rows is not None:
				_check(rows, 'rows', torch.float32)
				blocks = rows.dim() == 2 and rows.shape == (n, 64)
				_require((rows.dim() == 2 and rows.shape == (n, 16) and rows.data_ptr() % 64 == 0) or
						 (blocks and rows.data_ptr() % 256 == 0),
						 'rows must be (N, 16) 64-byte aligned, or site blocks (N, 64) 256-byte aligned')
				_require(not blocks or not half, 'site blocks hold fp32 SH rows: sh must be float32')
		if slots is not None:
			_check(slots, 'slots', torch.int32)
			_require(slots.dim() == 2 and slots.shape == (n, 16), 'slots must be (N, 16)')
		with torch.cuda.device(dev):
			if indexed is not None:
				call('vgr_foam_infer_indexed', *args, ptr(trace), int(trace_cap) if trace is not None else 0,
					 ptr(_order(order, B, dev)), 0 if lanes is None else int(lanes), ptr(edge_i), ptr(attr_i),
					 ptr(slots), ptr(rows), 16 if rows is None else rows.size(1), stream_of(dev))
			elif lanes is not None or order is not None or slots is not None:
				call('vgr_foam_infer_lanes', *args, ptr(trace), int(trace_cap) if trace is not None else 0,
					 ptr(_order(order, B, dev)), 0 if lanes is None else int(lanes), ptr(slots), stream_of(dev))
			elif trace is None:
				call('vgr_foam_infer', *args, stream_of(dev))
			else:
				call('vgr_foam_infer_traced', *args, ptr(trace), int(trace_cap), stream_of(dev))
		return out


def index_pack(offsets, nbr, edge, attr):
	"""Indexed edge records of a foam pack (vgr_foam_index_pack) -> (edge_i (E, 4), attr_i (N, 20)): edge_i[e] =
	(p_j, the bits of j = nbr[e]), attr_i = attr with column 7 holding site k's cut-off word edge[offsets[k], 3].
	A snapshot of the pack: rebuild it after changing edge or attr."""
	for t, n, dt in ((offsets, 'offsets', torch.int32), (nbr, 'nbr', torch.int32), (edge, 'edge', torch.float32),
					 (attr, 'attr', torch.float32)):
		_check(t, n, dt)
	n = attr.size(0)
	_require(attr.dim() == 2 and attr.size(1) == 20, 'attr must be (N, 20)')
	_require(offsets.numel() == n + 1, 'offsets must be (N + 1)')
	_require(edge.dim() == 2 and edge.size(1) == 4 and edge.size(0) == nbr.numel(), 'edge must be (E, 4)')
	edge_i, attr_i = torch.empty_like(edge), torch.empty_like(attr)
	dev = edge.device
	with torch.cuda.device(dev):
		call('vgr_foam_index_pack', ptr(offsets), ptr(nbr), ptr(edge), ptr(attr), n, nbr.numel(), ptr(edge_i),
			 ptr(attr_i), stream_of(dev))
	return edge_i, attr_i


def slot_table(offsets, nbr):
	"""Slot table of a foam pack (vgr_foam_slot_table) -> int32 (N, 16): per site and slot s (site & 7) of its
	self-first neighbourhood in CSR order, the first and the last entry at columns 2s, 2s + 1, -2 for an empty slot. foam_infer
	counts the reference's per-ray colour-cache misses from it (foam_infer.cu:151-168). A snapshot of the pack."""
	for t, name in ((offsets, 'offsets'), (nbr, 'nbr')):
		_check(t, name, torch.int32)
	n = offsets.numel() - 1
	_require(n >= 0 and nbr.numel() >= n, 'offsets must be (N + 1) and nbr (E >= N)')
	slots = torch.empty(n, 16, dtype=torch.int32, device=nbr.device)
	with torch.cuda.device(nbr.device):
		call('vgr_foam_slot_table', ptr(offsets), ptr(nbr), n, nbr.numel(), ptr(slots), stream_of(nbr.device))
	return slots


# Set VGR_CHECK_ORDER=1 to verify that every processing order is a permutation (a sort and a device sync per call).
CHECK_ORDER = os.environ.get('VGR_CHECK_ORDER', '0') == '1'


def _order(order, B, dev):
	"""Checks an optional processing order (int32 CUDA tensor of B entries) -> the tensor or None. The order must be
	a permutation of 0 .. B - 1: the kernels write the outputs of the rays it lists, so a ray left out keeps
	uninitialised outputs and a ray listed twice is traced twice. Entries outside [0, B) are skipped by the kernels.
	With VGR_CHECK_ORDER=1 the permutation is verified (RuntimeError otherwise)."""
	if order is None:
		return None
	_check(order, 'order', torch.int32)
	_require(order.numel() == B and order.device == dev, 'order must hold one entry per ray, on the rays\' device')
	if CHECK_ORDER:
		ok = bool(torch.equal(torch.sort(order.long())[0], torch.arange(B, device=dev)))
		_require(ok, 'order must be a permutation of 0 .. B - 1')
	return order


def ray_order(o, d, dir_res=8, pos_bits=7):
	"""Coherent processing order of a ray batch (vgr_ray_order): int32 (B,) permutation sorting the rays by the
	octahedral bin of the direction (dir_res x dir_res bins), then by the Z-order of the origin (pos_bits bits per
	axis). Passed as `order` to foam_infer / march_forward, it changes the order in which rays are traced (the
	lanes of a wave then share cache lines), not their results."""
	_check(o, 'o', torch.float32)
	_check(d, 'd', torch.float32)
	B, dev = o.size(0), o.device
	_require(o.dim() == 2 and o.size(1) == 3 and d.shape == o.shape, 'o and d must be (B, 3)')
	out = torch.empty(B, dtype=torch.int32, device=dev)
	if B == 0:
		return out
	wb = int(_lib.load().vgr_ray_order_work_size(B))
	work = torch.empty(wb, dtype=torch.uint8, device=dev)
	with torch.cuda.device(dev):
		call('vgr_ray_order', ptr(o), ptr(d), B, int(dir_res), int(pos_bits), ptr(out), ptr(work), wb, stream_of(dev))
	return out


def traverse_faces(points, offsets, nbr, edge, o, d, start, near, far, cap=None, orig=None, trace_cap=0, lanes=4):
	"""Cell traversal alone with a group of `lanes` (4, 8 or 16) lanes per ray (vgr_foam_traverse_faces, the
	lane-per-face layout): the outputs foam_infer gives with stage 0 -> stats (B, 5) int32 [samples, 0, walk
	steps, 0, 0] (+ trace (B, trace_cap), the cell of every sample in original numbering, -1 past the last, when
	trace_cap > 0)."""
	for t, n, dt in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32), (nbr, 'nbr', torch.int32),
					 (edge, 'edge', torch.float32), (o, 'o', torch.float32), (d, 'd', torch.float32),
					 (start, 'start', torch.int32), (near, 'near', torch.float32), (far, 'far', torch.float32)):
		_check(t, n, dt)
	n = points.size(0)
	B = o.size(0)
	dev = o.device
	stats = torch.empty(B, 5, dtype=torch.int32, device=dev)
	trace = torch.full((B, trace_cap), -1, dtype=torch.int32, device=dev) if trace_cap > 0 else None
	if B > 0:
		cp = cap if cap is not None and cap.numel() == B else None
		og = orig if orig is not None and orig.numel() == n else None
		with torch.cuda.device(dev):
			call('vgr_foam_traverse_faces', ptr(points), n, ptr(offsets), ptr(nbr), ptr(edge), nbr.numel(), ptr(o),
				 ptr(d), ptr(start), ptr(near), ptr(far), B, ptr(cp), ptr(og), ptr(stats), ptr(trace), int(trace_cap),
				 int(lanes), stream_of(dev))
	return (stats, trace) if trace is not None else stats


def pack_foam(points, offsets, adj, raw, d_log_scale, c_log_scale, dA, cA, sh, perm=None, scale_floor=0.0,
			  eps_density=0.0, sh_half=False):
	"""The inference records on the GPU (vgr_pack_foam, render.py:179-225) from the model's device tensors and the
	conics; perm (N,) new -> old renumbers the sites (None: none). -> points (N, 4), offsets (N + 1), nbr (E),
	edge (E, 4), attr (N, 20), sh32 (N, 16, 3) fp32, sh16 (N, 16, 3) fp16 or None, all in the new numbering."""
	for t, n, dt in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32), (adj, 'adj', torch.int32),
					 (raw, 'raw', torch.float32), (d_log_scale, 'd_log_scale', torch.float32),
					 (c_log_scale, 'c_log_scale', torch.float32), (dA, 'dA', torch.float32), (cA, 'cA', torch.float32),
					 (sh, 'sh', torch.float32)):
		_check(t, n, dt)
	n, m = points.size(0), adj.numel()
	_require(sh.dim() == 3 and sh.size(0) == n and sh.size(1) == 16 and sh.size(2) == 3, 'sh must be (N, 16, 3)')
	dev = points.device
	p32 = None
	if perm is not None:
		p32 = perm.to(torch.int32).contiguous()
		_check(p32, 'perm', torch.int32)
	f = dict(dtype=torch.float32, device=dev)
	out = {'points': torch.empty(n, 4, **f), 'offsets': torch.empty(n + 1, dtype=torch.int32, device=dev),
		   'nbr': torch.empty(m + n, dtype=torch.int32, device=dev), 'edge': torch.empty(m + n, 4, **f),
		   'attr': torch.empty(n, 20, **f), 'sh32': torch.empty(n, 16, 3, **f),
		   'sh16': torch.empty(n, 16, 3, dtype=torch.float16, device=dev) if sh_half else None}
	wb = int(_lib.load().vgr_pack_work_size(n))
	work = torch.empty(wb, dtype=torch.uint8, device=dev)
	with torch.cuda.device(dev):
		call('vgr_pack_foam', ptr(points), n, ptr(offsets), ptr(adj), m, ptr(raw), ptr(d_log_scale), ptr(c_log_scale),
			 ptr(dA), ptr(cA), ptr(sh), ptr(p32), float(scale_floor), float(eps_density), ptr(out['points']),
			 ptr(out['offsets']), ptr(out['nbr']), ptr(out['edge']), ptr(out['attr']), ptr(out['sh32']),
			 ptr(out['sh16']), ptr(work), wb, stream_of(dev))
	return out


def morton_codes(points, bits=10):
	"""(N,) int64 Z-order keys of points (N, 3) over their bounding box (vgr_morton_codes, render.py:168-176)."""
	_check(points, 'points', torch.float32)
	n = points.size(0)
	code = torch.empty(n, dtype=torch.int64, device=points.device)
	if n == 0:
		return code
	wb = int(_lib.load().vgr_morton_work_size(n))
	work = torch.empty(wb, dtype=torch.uint8, device=points.device)
	with torch.cuda.device(points.device):
		call('vgr_morton_codes', ptr(points), n, int(bits), ptr(code), ptr(work), wb, stream_of(points.device))
	return code


def bake_colors(points4, sh32, sh_deg, center, attr):
	"""Write the baked colours max(SH_k(d_k) + 1/2, 0) of the view from center (3,) into attr[:, 16:19] in place
	(vgr_bake_colors, render.py:228-235); points4 (N, 4), sh32 (N, 16, 3) and attr (N, 20) are packed records."""
	_check(points4, 'points4', torch.float32)
	_check(sh32, 'sh32', torch.float32)
	_check(attr, 'attr', torch.float32)
	n = points4.size(0)
	_require(points4.dim() == 2 and points4.size(1) == 4, 'points4 must be (N, 4)')
	_require(sh32.shape == (n, 16, 3) and attr.shape == (n, 20), 'sh32 must be (N, 16, 3) and attr (N, 20)')
	_require(sh32.device == points4.device == attr.device, 'points4, sh32 and attr must share a device')
	cx, cy, cz = (float(v) for v in torch.as_tensor(center, dtype=torch.float32).reshape(3).tolist())
	with torch.cuda.device(points4.device):
		call('vgr_bake_colors', ptr(points4), ptr(sh32), n, int(sh_deg), cx, cy, cz, ptr(attr),
			 stream_of(points4.device))
	return attr


# ============================================================================ foam.cu (training renderer)

class _FoamExtension:
	@staticmethod
	def _check_args(points, offsets, adj, raw, dA, cA, sh, o, d, start, near, far):
		for t, n, dtp in ((points, 'points', torch.float32), (offsets, 'offsets', torch.int32),
						  (adj, 'adj', torch.int32), (raw, 'raw', torch.float32), (dA, 'dA', torch.float32),
						  (cA, 'cA', torch.float32), (sh, 'sh', torch.float32), (o, 'o', torch.float32),
						  (d, 'd', torch.float32), (start, 'start', torch.int32), (near, 'near', torch.float32),
						  (far, 'far', torch.float32)):
			_check(t, n, dtp)
		_require(sh.dim() == 3 and sh.size(1) == 16 and sh.size(2) == 3, 'sh must be (N, 16, 3)')
		_require(dA.size(1) == 6 and cA.size(1) == 6, 'conics must be (N, 6)')

	@staticmethod
	def foam_forward(points, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, start, near, far, t_thresh, w_thresh,
					 record_cap, work=None):
		"""-> [rgb (B, 3), T (B,), depth (B,), stats (B, 3) int32, rec (B or 0, record_cap, 8)]
		(foam.cu:471-497)."""
		_FoamExtension._check_args(points, offsets, adj, raw, dA, cA, sh, o, d, start, near, far)
		B, dev, n = o.size(0), o.device, points.numel() // 3
		K = int(record_cap)
		_require(K >= 0, 'record_cap must be >= 0')
		rgb = torch.empty(B, 3, device=dev)
		T = torch.empty(B, device=dev)
		depth = torch.empty(B, device=dev)
		stats = torch.empty(B, 3, dtype=torch.int32, device=dev)
		rec = torch.empty(B if K > 0 else 0, K, 8, device=dev)
		if B == 0:
			return [rgb, T, depth, stats, rec]
		wb = int(_lib.load().vgr_foam_work_size(n, int(sh_deg)))
		if work is None:
			work = torch.empty(max(wb, 1), dtype=torch.uint8, device=dev)
		else:
			_require(work.dtype == torch.uint8 and work.numel() >= wb, 'work is too small')
			wb = work.numel()
		with torch.cuda.device(dev):
			call('vgr_foam_forward', ptr(points), n, ptr(offsets), ptr(adj), adj.numel(), ptr(raw), ptr(dA), ptr(cA),
				 ptr(sh), int(sh_deg), ptr(o), ptr(d), ptr(start), ptr(near), ptr(far), B, float(t_thresh),
				 float(w_thresh), ptr(rgb), ptr(T), ptr(depth), ptr(stats), ptr(rec) if K > 0 else None, K,
				 ptr(work), wb, stream_of(dev))
		return [rgb, T, depth, stats, rec]

	@staticmethod
	def foam_backward(points, offsets, adj, raw, dA, cA, sh, sh_deg, o, d, start, near, far, t_thresh, w_thresh,
					  rgb, T, g_rgb, g_T, rec, stats, work=None):
		"""-> [g_raw (N,), g_dA (N, 6), g_cA (N, 6), g_sh (N, 16, 3)] (foam.cu:499-531). rec (B, K, 8) with the
		forward's stats, or an empty rec to re-trace every ray. work: the forward's workspace, whose site blocks are
		reused, or None to pack them again."""
		_FoamExtension._check_args(points, offsets, adj, raw, dA, cA, sh, o, d, start, near, far)
		for t, nm in ((rgb, 'rgb'), (T, 'T'), (g_rgb, 'g_rgb'), (g_T, 'g_T'), (rec, 'rec')):
			_check(t, nm, torch.float32)
		_check(stats, 'stats', torch.int32)
		B, dev, n = o.size(0), o.device, points.numel() // 3
		_require(rgb.shape == g_rgb.shape == (B, 3) and T.shape == g_T.shape == (B,),
				 'rgb, g_rgb must be (B, 3) and T, g_T (B,)')
		replay = rec.numel() > 0
		_require(not replay or (rec.dim() == 3 and rec.size(0) == B and rec.size(2) == 8), 'rec must be (B, K, 8)')
		_require(not replay or stats.shape == (B, 3), 'stats must be (B, 3)')
		K = rec.size(1) if replay else 0
		g = [torch.empty(n, device=dev), torch.empty(n, 6, device=dev), torch.empty(n, 6, device=dev),
			 torch.empty(n, 16, 3, device=dev)]
		wb = int(_lib.load().vgr_foam_work_size(n, int(sh_deg)))
		ready = work is not None
		if ready:
			_require(work.dtype == torch.uint8 and work.numel() >= wb, 'work is too small')
			wb = work.numel()
		else:
			work = torch.empty(max(wb, 1), dtype=torch.uint8, device=dev)
		with torch.cuda.device(dev):
			call('vgr_foam_backward', ptr(points), n, ptr(offsets), ptr(adj), adj.numel(), ptr(raw), ptr(dA),
				 ptr(cA), ptr(sh), int(sh_deg), ptr(o), ptr(d), ptr(start), ptr(near), ptr(far), B, float(t_thresh),
				 float(w_thresh), ptr(rgb), ptr(T), ptr(g_rgb), ptr(g_T), ptr(rec) if replay else None, K,
				 ptr(stats) if replay else None, *[ptr(x) for x in g], int(ready), ptr(work), wb, stream_of(dev))
		return g


_FIELD, _MARCH, _FOAM_INFER, _FOAM = _FieldExtension(), _MarchExtension(), _FoamInferExtension(), _FoamExtension()


def extension():
	"""vgf.cu forward operators (reference: ext.py:30-31)."""
	_lib.load()
	return _FIELD


def foam_extension():
	"""foam.cu, the training renderer (reference: ext.py:38-39)."""
	_lib.load()
	return _FOAM


def march_extension():
	"""march.cu forward (reference: ext.py:34-35)."""
	_lib.load()
	return _MARCH


def foam_infer_extension():
	"""foam_infer.cu (reference: ext.py:42-43)."""
	_lib.load()
	return _FOAM_INFER


class Graph:
	"""Fixed sites (N, 3) and their Delaunay adjacency as int32 CSR, resident on the GPU (the reference's ext.Graph,
	ext.py:46-58)."""

	def __init__(self, points, offsets, adj):
		self.points = points.float().contiguous()
		self.offsets = offsets.int().contiguous()
		self.adj = adj.int().contiguous()

	def walk(self, o, d, z, start):
		"""-> (site (B, S), steps (B,)) int32: the nearest site of each sample o + z d, z (B, S) sorted along each
		ray, by greedy Delaunay walks from start (B,), a site near each origin."""
		return extension().walk(self.points, self.offsets, self.adj, o.float().contiguous(), d.float().contiguous(),
								z.float().contiguous(), start.int().contiguous())


# Differentiable operators. Each _*Op below pairs a forward kernel call with its gradient kernel call; one generic
# autograd Function (_Differentiable) runs any of them, so the reference's density / color / conic / march / foam
# (ext.py:61-216) keep their signatures and gradients while the plumbing lives in one place. An op's forward returns
# (outputs, extra tensors the backward needs, state shared with the backward); its leading `n_diff` outputs carry
# gradients, the rest (depths, counters) are marked non-differentiable.

class _Differentiable(torch.autograd.Function):

	@staticmethod
	def forward(ctx, op, args, *params):
		outs, extra, state = op.forward(params, args)
		ctx.op, ctx.args, ctx.state = op, args, state
		ctx.split = (len(params), len(params) + len(outs))
		ctx.save_for_backward(*params, *outs, *extra)
		ctx.mark_non_differentiable(*outs[op.n_diff:])
		return outs

	@staticmethod
	def backward(ctx, *grad_outs):
		saved = ctx.saved_tensors
		a, b = ctx.split
		outs = saved[a:b]
		upstream = [torch.zeros_like(o, dtype=torch.float32) if g is None else g.float().contiguous()
					for o, g in zip(outs, grad_outs)]
		grads = ctx.op.backward(saved[:a], ctx.args, outs, saved[b:], upstream, ctx.state)
		ctx.state = None  # the workspace goes back to torch's allocator
		return (None, None, *grads)


def _evaluate(op, args, params):
	"""The op's outputs: through autograd when grad mode is on and a parameter requires a gradient, else the plain
	forward kernel on the detached parameters."""
	params = [p.contiguous() for p in params]
	if torch.is_grad_enabled() and any(p.requires_grad for p in params):
		return _Differentiable.apply(op, args, *params)
	return op.forward([p.detach() for p in params], args)[0]


class _DensityOp:
	"""params (raw, log_scale, quat); args (graph, x, site)."""
	n_diff = 1

	@staticmethod
	def forward(p, a):
		g, x, site = a
		return (extension().density_forward(g.points, g.offsets, g.adj, *p, x, site, 1.0),), (), None

	@staticmethod
	def backward(p, a, outs, extra, grads, state):
		g, x, site = a
		return extension().density_backward(g.points, g.offsets, g.adj, *p, x, site, grads[0])


class _ColorOp:
	"""params (log_scale, quat, sh); args (graph, x, dirs, site, sh_deg)."""
	n_diff = 1

	@staticmethod
	def forward(p, a):
		g, x, dirs, site, sh_deg = a
		return (extension().color_forward(g.points, g.offsets, g.adj, *p, sh_deg, x, dirs, site),), (), None

	@staticmethod
	def backward(p, a, outs, extra, grads, state):
		g, x, dirs, site, sh_deg = a
		return extension().color_backward(g.points, g.offsets, g.adj, *p, sh_deg, x, dirs, site, outs[0], grads[0])


class _ConicOp:
	"""params (log_scale, quat); args (floor,)."""
	n_diff = 1

	@staticmethod
	def forward(p, a):
		return (extension().conic_forward(*p, a[0]),), (), None

	@staticmethod
	def backward(p, a, outs, extra, grads, state):
		return extension().conic_backward(*p, a[0], grads[0])


class _MarchOp:
	"""params (raw, dA, cA, sh); args (graph, rays (o, d, start, near, mid, far), (sh_deg, dt, n_bg, t_thresh,
	w_thresh)). Under autograd both passes run 16 lanes per ray, the faster layout for a training step at every batch
	size measured, and share one workspace: the backward reuses the site blocks the forward packed."""
	n_diff = 2

	@staticmethod
	def forward(p, a):
		g, rays, cfg = a
		n = g.points.numel() // 3
		work = torch.empty(max(int(_lib.load().vgr_march_backward_work_size(n, cfg[0])), 1), dtype=torch.uint8,
						   device=g.points.device)
		outs = march_extension().march_forward(g.points, g.offsets, g.adj, *p, cfg[0], *rays, *cfg[1:], lanes=16,
											   work=work)
		return tuple(outs), (), work

	@staticmethod
	def backward(p, a, outs, extra, grads, work):
		g, rays, cfg = a
		return march_extension().march_backward(g.points, g.offsets, g.adj, *p, cfg[0], *rays, *cfg[1:], outs[0],
												outs[1], grads[0], grads[1], lanes=16, work=work)


class _FoamOp:
	"""params (raw, dA, cA, sh); args (graph, rays (o, d, start, near, far), (sh_deg, t_thresh, w_thresh),
	record_cap). The forward keeps up to record_cap samples per ray for the backward, which replays them (or
	re-traces rays that did not fit) with the forward's site blocks."""
	n_diff = 2

	@staticmethod
	def forward(p, a):
		g, rays, cfg, record_cap = a
		n = g.points.numel() // 3
		work = torch.empty(max(int(_lib.load().vgr_foam_work_size(n, cfg[0])), 1), dtype=torch.uint8,
						   device=g.points.device)
		rgb, T, depth, stats, rec = foam_extension().foam_forward(g.points, g.offsets, g.adj, *p, cfg[0], *rays,
																  *cfg[1:], record_cap, work=work)
		return (rgb, T, depth, stats), (rec,), work

	@staticmethod
	def backward(p, a, outs, extra, grads, work):
		g, rays, cfg, _ = a
		rgb, T, _, stats = outs
		return foam_extension().foam_backward(g.points, g.offsets, g.adj, *p, cfg[0], *rays, *cfg[1:], rgb, T,
											  grads[0], grads[1], extra[0], stats, work=work)


def density(graph, raw, log_scale, quat, x, site, scale_mult=1.0):
	"""sigma(x) (m,): sum over the neighbourhood {site} U adj(site) of exp(raw_k) G_k(x), differentiable in raw,
	log_scale and quat. scale_mult != 1 widens every Gaussian (the proposal rounds) and is never differentiated
	(ext.py:78-87)."""
	x, site = x.detach().float().contiguous(), site.int().contiguous()
	if scale_mult != 1.0:
		return extension().density_forward(graph.points, graph.offsets, graph.adj,
										   *[p.detach().contiguous() for p in (raw, log_scale, quat)], x, site,
										   float(scale_mult))
	out = _evaluate(_DensityOp, (graph, x, site), (raw, log_scale, quat))
	return out[0] if isinstance(out, tuple) else out


def color(graph, log_scale, quat, sh, x, dirs, site, sh_deg=3):
	"""C(x, d) (m, 3): the colours max(SH_k(d) + 1/2, 0) of the neighbourhood of site, blended with the normalised
	colour-Gaussian weights H_k(x); sh (N, 16, 3); differentiable in log_scale, quat and sh (ext.py:108-117)."""
	args = (graph, x.detach().float().contiguous(), dirs.detach().float().contiguous(), site.int().contiguous(),
			int(sh_deg))
	out = _evaluate(_ColorOp, args, (log_scale, quat, sh))
	return out[0] if isinstance(out, tuple) else out


def conic(log_scale, quat, floor=0.0):
	"""(N, 6) conics (xx, xy, xz, yy, yz, zz) = the inverses of R diag(e^(2 log_scale) + floor^2) R^T, R the rotation
	of the normalised quaternion; differentiable (ext.py:134-136)."""
	out = _evaluate(_ConicOp, (float(floor),), (log_scale, quat))
	return out[0] if isinstance(out, tuple) else out


def conic_reference(log_scale, quat, floor=0.0):
	"""The conic in plain torch ops, for tests (the reference's ext.py:139-149): R = (w^2 - |v|^2) I + 2 v v^T +
	2 w [v]_x for the unit quaternion (w, v), A = sum over the axes a of r_a r_a^T / (e^(2 s_a) + floor^2), r_a the
	columns of R."""
	q = quat / quat.norm(dim=-1, keepdim=True).clamp_min(1e-12)
	w, v = q[:, 0], q[:, 1:]
	zero = torch.zeros_like(w)
	skew = torch.stack([zero, -v[:, 2], v[:, 1], v[:, 2], zero, -v[:, 0], -v[:, 1], v[:, 0], zero], -1).view(-1, 3, 3)
	eye = torch.eye(3, dtype=q.dtype, device=q.device)
	R = ((w * w - (v * v).sum(-1))[:, None, None] * eye + 2 * v[:, :, None] * v[:, None, :] +
		 2 * w[:, None, None] * skew)
	inv_var = 1.0 / (torch.exp(2 * log_scale.clamp(-20, 20)) + floor * floor)
	A = (R[:, :, None, :] * R[:, None, :, :] * inv_var[:, None, None, :]).sum(-1)
	rows, cols = [0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2]
	return A[:, rows, cols].contiguous()


def march(graph, raw, dA, cA, sh, sh_deg, o, d, start, near, mid, far, dt, n_bg, t_thresh=1e-4, w_thresh=1e-4):
	"""The uniform-step fused renderer (ext.py:172-182) -> foreground rgb (B, 3) (no background), transmittance T
	(B,), depth (B,), stats (B, 3) int32: samples, coloured samples, walk steps. rgb and T are differentiable in raw,
	dA, cA and sh."""
	rays = tuple(t.float().contiguous() for t in (o, d)) + (start.int().contiguous(),) + \
		tuple(t.float().contiguous() for t in (near, mid, far))
	return _evaluate(_MarchOp, (graph, rays, (int(sh_deg), float(dt), int(n_bg), float(t_thresh), float(w_thresh))),
					 [p.float() for p in (raw, dA, cA, sh)])


def foam(graph, raw, dA, cA, sh, sh_deg, o, d, start, near, far, t_thresh=1e-4, w_thresh=1e-4, record_cap=256):
	"""The training renderer at the ray / Voronoi-face crossings (ext.py:205-216) -> foreground rgb (B, 3),
	transmittance (B,), depth (B,), stats (B, 3) int32: samples, coloured segments, walk steps to x(near). Under
	autograd up to record_cap samples per ray are recorded for the backward (0: it re-traces every ray)."""
	rays = tuple(t.float().contiguous() for t in (o, d)) + (start.int().contiguous(),) + \
		tuple(t.float().contiguous() for t in (near, far))
	params = [p.float() for p in (raw, dA, cA, sh)]
	args = (graph, rays, (int(sh_deg), float(t_thresh), float(w_thresh)), int(record_cap))
	if torch.is_grad_enabled() and any(p.requires_grad for p in params):
		return _Differentiable.apply(_FoamOp, args, *[p.contiguous() for p in params])
	g = graph
	return foam_extension().foam_forward(g.points, g.offsets, g.adj, *[p.detach().contiguous() for p in params],
										 args[2][0], *rays, *args[2][1:], 0)[:4]
