"""Benchmark of the inference path: foam_infer (ray / Voronoi-face renderer) on benchmark configuration 3 -- the
2M-site surface-dominated scene seen by 4 cameras at 1920x1080 -- on one MI355X.

One step = one foam_infer launch rendering all 4 frames (8,294,400 rays) with the scene packed and the rays
resident in HBM. Prints one JSON line: Mrays/s (value), ms per step, FPS at 1080p, the roofline of the kernel
(algorithmic bytes per launch from the kernel's own per-ray counters / the launch time measured with HIP events
on the launch stream) and the CPU oracle timed on the host on a bounded, deterministic subset of the same rays.

  python bench.py [--steps K] [--warmup W] [--colors exact|fused] [--no-reorder] [--no-indexed] [--cpu-seconds S]

Other rows of the path, each as one JSON line of the same form (not the headline):
  --workload march    march_forward on config 5 (4M sites, 16,777,216 incoherent rays, dt = 1/512, 64 bg steps)
  --workload locate   start-cell location on config 5 (nearest site of 16,777,216 ray origins among 4M sites)
  --workload pack     pack_foam with Z-order renumbering on config 3 (the step before the kernel)
  --workload grad     the backward of the field operators on the frame of --workload field
  --workload traverse the cell traversal alone (foam_infer stage 0) on config 3 in both layouts: one ray per lane
                      (foam_infer) against a group of lanes per ray testing a cell's faces in parallel (--lanes)
  --workload march-grad  a training step of the uniform march on config 5: forward + backward of --batch rays
  --workload foam-grad   a training step of the training renderer (foam.cu) on config 3: forward with records +
                         backward of --batch rays
  --workload field    the NeRF-path operators (walk, density_forward, color_forward, conic_forward) on config 3,
                      one 1920x1080 frame at 64 stratified samples per ray (render_rays' first round)
"""

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, 'voronoi-gauss_amd'))

METRIC = 'Mrays/s and FPS @1080p (2M sites) on 1 MI355X; achieved HBM GB/s vs peak'
HBM_PEAK_GBS = 8000.0
PROFILES = os.path.join(ROOT, 'profiles')


def log(*a):
	print('[bench]', *a, file=sys.stderr, flush=True)


def copy_probe(dev):
	"""A 1 GiB device-to-device copy: the PMC runs scale the kernels' FETCH_SIZE / WRITE_SIZE by what the same
	counters read for it."""
	import torch
	src = torch.empty(1 << 28, dtype=torch.float32, device=dev)
	dst = torch.empty_like(src)
	dst.copy_(src)
	torch.cuda.synchronize()
	log('copy probe: 1 GiB read + 1 GiB written')


def source_hash(*names):
	"""16 hex digits of SHA-256 over the named kernel sources, the two headers every kernel includes and the hipcc
	flags: it names the build a DRAM-traffic profile was measured on."""
	import hashlib

	from vgr import build
	h = hashlib.sha256()
	for n in sorted(set(names) | {'vgr_device.h', 'vgr_abi.h'}):
		h.update(n.encode())
		with open(os.path.join(build.CSRC, n), 'rb') as f:
			h.update(f.read())
	h.update(' '.join(build.HIPCC_FLAGS).encode())
	return h.hexdigest()[:16]


def measured_traffic(workload, src):
	"""DRAM bytes per launch of this workload from a committed rocprofv3 PMC summary under profiles/ (a line
	'traffic_bytes_per_launch: <bytes> workload: <key> source: <hash>'), only when it was measured on this build
	(same source hash) -> (bytes or None, where it came from or why it is missing)."""
	import glob
	import re
	stale = None
	for path in sorted(glob.glob(os.path.join(PROFILES, '*.md'))):
		for line in open(path):
			m = re.match(r'\s*traffic_bytes_per_launch:\s*([0-9.eE+]+)\s+workload:\s*(\S+)\s+source:\s*(\S+)', line)
			if m and m.group(2) == workload:
				if m.group(3) == src:
					return float(m.group(1)), f'{os.path.relpath(path, ROOT)} (rocprofv3 FETCH_SIZE + WRITE_SIZE, source {src})'
				stale = f'{os.path.relpath(path, ROOT)} was measured on source {m.group(3)}, not this build ({src})'
	return None, stale or f'no PMC profile of workload {workload} under profiles/'


def hbm_roofline(ms, workload, src, model_bytes, model, kernel):
	"""The HBM roofline of a launch of `ms` milliseconds: achieved = DRAM bytes per launch (rocprofv3, this build)
	/ the launch time, frac = achieved / 8 TB/s; both null when no profile of this build exists. The byte model of
	the workload (model_bytes, described by `model`) is reported beside it under its own keys and never feeds them."""
	traffic, source = measured_traffic(workload, src)
	r = {'bound': 'hbm', 'kernel': kernel, 'achieved': None, 'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': None,
		 'traffic': traffic, 'traffic_source': source, 'source_hash': src}
	if traffic is not None:
		gbs = traffic / (ms * 1e-3) / 1e9
		r['achieved'], r['frac'] = round(gbs, 1), round(gbs / HBM_PEAK_GBS, 4)
	r['model'] = model
	r['model_bytes_per_launch'] = model_bytes
	r['model_GBps'] = round(model_bytes / (ms * 1e-3) / 1e9, 1)
	if traffic is not None:
		r['model_over_dram'] = round(model_bytes / traffic, 3)
	return r


def cpu_model():
	"""The host CPU's model name and logical core count (lscpu's 'Model name', from /proc/cpuinfo)."""
	name = None
	try:
		for line in open('/proc/cpuinfo'):
			if line.startswith('model name'):
				name = line.split(':', 1)[1].strip()
				break
	except OSError:
		pass
	return f'{name or "unknown CPU"} ({os.cpu_count()} logical cores visible)'


def timed_cpu(run, reps=3):
	"""1 untimed warmup run, then the median of `reps` timed runs of run() -> (median seconds, last result)."""
	import numpy as np
	run()
	times, res = [], None
	for _ in range(reps):
		res = run()
		times.append(res['seconds'])
	return float(np.median(times)), res


def algorithmic_bytes(stats, sh_bytes, u_sh_per_ray, indexed=False):
	"""Cache-oblivious bytes of one launch from the per-ray counters (B, 5) = samples, coloured segments, walk
	steps, density terms, SH evaluations:
	  56 per ray (o, d, near, far, start in; rgb, T, depth out)
	  + 24 per sample (cell position 16 + offsets 8)
	  + 84 per neighbourhood edge = density term (edge record 16 + nbr 4 + density record 32 + colour-conic record 32;
	    80 with indexed edge records, which carry the neighbour index in the edge record)
	  + sh_bytes per distinct site whose colour the ray blends (u_sh_per_ray, measured on traced rays)."""
	s = stats.double()
	per_edge = 80 if indexed else 84
	return float(56 * len(s) + 24 * s[:, 0].sum() + per_edge * s[:, 3].sum() + sh_bytes * u_sh_per_ray * len(s))


def wave_balance(stats, rays_per_wave=64, cols=(('samples', 0), ('density_terms', 3))):
	"""Lane use bounds of one-ray-per-lane waves (64 consecutive rays in processing order, one 8x8 tile for camera
	rays) from the per-ray counters: the mean over waves of mean/max of each named column (samples per ray: a wave
	runs until its longest ray ends; foam_infer's density terms, the neighbourhood edges, since its lockstep also
	waits for the largest neighbourhood)."""
	n = (len(stats) // rays_per_wave) * rays_per_wave
	s = stats[:n].double().view(-1, rays_per_wave, stats.shape[1])
	out = {}
	for name, col in cols:
		v = s[:, :, col]
		out[name] = round(float((v.mean(1) / v.max(1).values.clamp_min(1)).mean()), 4)
	return out


def distinct_blended_sites(fi, pack, args_of, n_rays, sh_deg, tiles=256):
	"""Mean number of distinct sites whose colour a ray blends, over `tiles` 8x8 ray tiles spread evenly over the
	launch: the rays are traced again (same kernel, outside the timed region) and, exact colours blending every
	neighbour of every visited cell, the distinct neighbours of each ray's cells are counted."""
	import torch
	dev = pack['points'].device
	n_tiles = n_rays // 64
	pick = torch.linspace(0, n_tiles - 1, min(tiles, n_tiles), device=dev).long()
	rays = (pick[:, None] * 64 + torch.arange(64, device=dev)).reshape(-1)
	cap = 4096
	out = fi.foam_infer(*args_of(rays), trace_cap=cap)
	stats, trace = out[3], out[4]
	n = stats[:, 0].long().clamp(max=cap)
	valid = torch.arange(cap, device=dev)[None, :] < n[:, None]
	ray_id = torch.arange(len(rays), device=dev)[:, None].expand(-1, cap)[valid]
	cells = trace[valid].long()
	if pack['inv'] is not None:
		cells = pack['inv'][cells]
	start = pack['offsets'][cells].long()
	count = (pack['offsets'][cells + 1] - pack['offsets'][cells]).long()
	total = int(count.sum())
	first = torch.repeat_interleave(torch.cumsum(count, 0) - count, count)
	edge = torch.repeat_interleave(start, count) + torch.arange(total, device=dev) - first
	sites = pack['nbr'][edge].long()
	keys = torch.unique(torch.repeat_interleave(ray_id, count) * len(pack['points']) + sites)
	u = torch.bincount(keys // len(pack['points']), minlength=len(rays)).double()
	return float(u.mean()), len(rays)


def main():
	ap = argparse.ArgumentParser()
	ap.add_argument('--gpus', type=int, default=1)
	ap.add_argument('--steps', type=int, default=None, help='timed steps (default 20; march: 3)')
	ap.add_argument('--warmup', type=int, default=None, help='untimed steps (default 3; march: 1)')
	ap.add_argument('--config', type=int, default=3)
	ap.add_argument('--scale', type=float, default=1.0, help='site-count scale (1 = the full configuration)')
	ap.add_argument('--colors', default='fused', choices=['exact', 'fused', 'baked'],
				help='exact colour modes (eps_color = 0): lazy second pass or fused online blend; baked: per-view '
					 'site colours, baked per camera inside the timed step (approximate)')
	ap.add_argument('--sh-half', action='store_true', help='fp16 SH coefficients (approximate)')
	ap.add_argument('--eps-color', type=float, default=0.0, help='skip colour terms of relative weight < eps')
	ap.add_argument('--eps-density', type=float, default=0.0, help='skip density terms below eps')
	ap.add_argument('--no-reorder', action='store_true', help='keep the generator order of the sites')
	ap.add_argument('--no-rows', action='store_true',
					help='group layouts read the 80-byte attr rows instead of the site rows')
	ap.add_argument('--site-rows', type=int, default=256, choices=[64, 256],
					help="group layouts' site rows: 256-byte site blocks holding the fp32 SH row (the default with "
						 'fp32 SH), or the 64-byte rows beside the SH rows')
	ap.add_argument('--no-slots', action='store_true',
					help="no slot table: the reference's colour-cache misses counted with per-lookup tags in LDS")
	ap.add_argument('--no-indexed', action='store_true',
					help='fused colours: read the reference edge records (nbr + edge) instead of the indexed ones')
	ap.add_argument('--tile', type=int, default=8, help='pixel tile edge (8: one 8x8 tile per wave64)')
	ap.add_argument('--tile-curve', default='morton', choices=['row', 'morton'],
					help='order of the pixel tiles of a camera (row-major or Z-order of the tile coordinates)')
	ap.add_argument('--cpu-seconds', type=float, default=15.0, help='target CPU-oracle time (0: skip)')
	ap.add_argument('--copy-probe', action='store_true', help='also run a 1 GiB device copy (PMC calibration)')
	ap.add_argument('--batch', type=int, default=4096, help='grad workload: random rays per training step')
	ap.add_argument('--lanes-per-ray', type=int, default=None, choices=[1, 2, 4, 8, 16],
					help='foam workload: ray layout (1: one ray per lane, 2 / 4 / 8: lanes per ray); march workload: '
						 '1 or 16; default: the library default')
	ap.add_argument('--lanes', type=int, default=4, choices=[4, 8, 16],
					help='traverse workload: lanes per ray of the layout the JSON line reports')
	ap.add_argument('--order', default='auto', choices=['auto', 'on', 'off'],
					help='trace the rays in the coherent order of vgr_ray_order, computed inside the timed step (auto: '
						 'on for the incoherent ray batch of config 5, off for camera rays in pixel tiles)')
	ap.add_argument('--order-dir-res', type=int, default=None, help='direction bins per side of the octahedral map')
	ap.add_argument('--order-pos-bits', type=int, default=None, help='Z-order bits per axis of the ray origins')
	ap.add_argument('--workload', default='foam',
					choices=['foam', 'march', 'locate', 'field', 'grad', 'pack', 'traverse', 'march-grad',
							 'foam-grad'],
					help='foam: the headline (foam_infer, config 3); march / locate (config 5), field (config 3): '
						 'the other rows')
	args = ap.parse_args()
	if args.steps is None:
		args.steps = 3 if args.workload == 'march' else 20
	if args.warmup is None:
		args.warmup = 1 if args.workload == 'march' else 3
	if args.gpus != 1:
		print(f'bench.py renders on one GPU only (got --gpus {args.gpus}): rays are independent, so N GPUs would '
			  f'each render 1/N of the cameras with a replicated scene; multi-GPU runs are not part of this build.',
			  file=sys.stderr)
		sys.exit(2)
	if args.workload == 'march':
		return bench_march(args)
	if args.workload == 'locate':
		return bench_locate(args)
	if args.workload == 'field':
		return bench_field(args)
	if args.workload == 'pack':
		return bench_pack(args)
	if args.workload == 'traverse':
		return bench_traverse(args)
	if args.workload == 'march-grad':
		return bench_march_grad(args)
	if args.workload == 'foam-grad':
		return bench_foam_grad(args)
	if args.workload == 'grad':
		return bench_grad(args)
	bench_foam(args)


def bench_foam(args):
	import numpy as np
	import torch

	from vgr import ext, render, scenes
	from vgr.model import VoronoiGaussField

	dev = torch.device('cuda:0')
	t0 = time.time()
	sc = scenes.make_scene(args.config, scale=args.scale, log=log)
	log(f'scene config {args.config}: {sc.n_sites} sites, {len(sc.adj)} adjacency entries ({time.time() - t0:.0f} s)')
	model = VoronoiGaussField.from_scene(sc, dev)
	fast = args.sh_half or args.eps_color > 0 or args.eps_density > 0 or args.colors == 'baked'
	pack = render.pack_foam(model, reorder=not args.no_reorder, sh_half=args.sh_half, eps_density=args.eps_density,
							index=False)
	o_np, d_np, start_np, _ = sc.camera_rays(tile=args.tile, curve=args.tile_curve)
	o, d = torch.from_numpy(o_np).to(dev), torch.from_numpy(d_np).to(dev)
	start = torch.from_numpy(start_np).to(dev)
	if pack['inv'] is not None:
		start = pack['inv'][start.long()].int()
	near, _, far = render.ray_bounds(o, d, 0.02, sc.far_radius)
	B = len(o)
	W, H = (sc.cameras[0].width, sc.cameras[0].height) if sc.cameras else (0, 0)
	frames = len(sc.cameras)
	mode = {'exact': 0, 'baked': 1, 'fused': 2}[args.colors]
	color_cut = 2 * math.log(1 / args.eps_color) if args.eps_color > 0 else math.inf
	empty = torch.empty(0, dtype=torch.int32, device=dev)
	fi = ext.foam_infer_extension()

	ordered = args.order == 'on' or (args.order == 'auto' and not sc.cameras)
	dir_res, pos_bits = args.order_dir_res or 8, args.order_pos_bits or 7
	# exact colours with the colour cut-off +inf, the indexed records and the slot table run as the one-pass blend
	# (one ray per lane); otherwise as two passes, 4 lanes per ray
	blend_ok = not args.no_indexed and not args.no_slots and color_cut == math.inf
	# camera rays in 8x8 tiles: the library's default layout (one ray per lane; 4 lanes per ray for exact colours
	# in two passes); an incoherent batch in coherence order: 8 lanes per ray, the fastest layout on config 5 for
	# every colour mode
	lanes = args.lanes_per_ray or (8 if ordered else (4 if args.colors == 'exact' and not blend_ok else 1))
	# fused colours (and exact colours by the blend) with one ray per lane read the indexed edge records (built once
	# with the pack, untimed)
	exact_blend = mode == 0 and lanes == 1 and blend_ok
	indexed = not args.no_indexed and lanes == 1 and (mode == 2 or exact_blend)
	# the derived records, built once with the pack (untimed): indexed edge records, the slot table of the reference's
	# colour cache, the site rows of the group layouts
	if not args.no_indexed and args.colors != 'baked':
		render.index_pack(pack)
	elif args.colors != 'baked':
		pack['slots'] = ext.slot_table(pack['offsets'], pack['nbr'])
	if args.no_slots:
		pack.pop('slots', None)
	if args.no_rows or lanes == 1 or mode != 2:  # the site rows serve the group layouts' fused blend
		pack.pop('rows', None)
	elif args.site_rows == 64 and 'rows' in pack and pack['rows'].size(1) == 64:
		pack['rows'] = pack['rows'][:, :16].contiguous()
	row_kind = None if 'rows' not in pack else '64-byte rows' if pack['rows'].size(1) == 16 else \
		'256-byte site blocks (record + fp32 SH row)'

	def launch(p, sel, m=mode, cut=color_cut):
		order = ext.ray_order(o[sel], d[sel], dir_res, pos_bits) if ordered else None
		return fi.foam_infer(p['points'], p['offsets'], p['nbr'], p['edge'], p['attr'], p['sh'], sc.sh_deg, o[sel],
							 d[sel], start[sel], near[sel], far[sel], 1e-4, 1e-4, cut, m, 2, empty, p['orig'],
							 lanes=lanes, order=order,
							 indexed=(p['edge_i'], p['attr_i'], p.get('rows')) if 'edge_i' in p and m != 1 else None,
							 slots=p.get('slots'))

	if args.colors == 'baked':  # one launch per camera, each after baking that view's site colours
		per = B // frames
		centers = [torch.tensor(c.eye, dtype=torch.float32, device=dev) for c in sc.cameras]

		def call():
			outs = []
			for f, cen in enumerate(centers):
				render.bake_colors(model, pack, cen)
				outs.append(launch(pack, slice(f * per, (f + 1) * per)))
			return [torch.cat(x) for x in zip(*outs)]
	else:
		call = lambda: launch(pack, slice(None))  # noqa
	log(f'{B} rays ({frames} x {W}x{H}), pack ready ({time.time() - t0:.0f} s); warmup {args.warmup}')
	for _ in range(args.warmup):
		out = call()
	torch.cuda.synchronize()
	stream = torch.cuda.current_stream(dev)
	ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
	torch.cuda.synchronize()
	wall0 = time.perf_counter()
	for a, b in ev:
		a.record(stream)
		out = call()
		b.record(stream)
	torch.cuda.synchronize()
	wall = time.perf_counter() - wall0
	launch_ms = [a.elapsed_time(b) for a, b in ev]
	ms = float(np.mean(launch_ms))
	rgb, T, depth, stats = out
	log(f'{args.steps} steps: mean {ms:.3f} ms, median {np.median(launch_ms):.3f} ms, '
		f'wall {wall * 1e3 / args.steps:.3f} '
		f'ms/step')
	sh_bytes = (6 if args.sh_half else 12) * (sc.sh_deg + 1) ** 2 if args.colors != 'baked' else 0
	if fast:  # SH bytes per SH evaluation (an upper bound of the distinct sites); quality against the exact image
		u_sh, u_rays = float(stats[:, 4].double().mean()), 0
		exact = render.pack_foam(model, reorder=not args.no_reorder, index=False)
		ref = launch(exact, slice(None), 2, math.inf)
		bg = 0.5
		img, img_ref = rgb + T[:, None] * bg, ref[0] + ref[1][:, None] * bg
		mse = float(((img - img_ref) ** 2).double().mean())
		quality = {'psnr_vs_exact_db': round(10 * math.log10(1 / max(mse, 1e-30)), 2),
				   'max_abs_vs_exact': float((img - img_ref).abs().max())}
		log(f'vs exact (fused, fp32, no skipping): PSNR {quality["psnr_vs_exact_db"]} dB, max |diff| '
			f'{quality["max_abs_vs_exact"]:.3e}')
		del exact
	else:
		args_of = lambda sel: (pack['points'], pack['offsets'], pack['nbr'], pack['edge'], pack['attr'],  # noqa
							   pack['sh'], sc.sh_deg, o[sel], d[sel], start[sel], near[sel], far[sel], 1e-4, 1e-4,
							   math.inf, mode, 2, empty, pack['orig'])
		u_sh, u_rays = distinct_blended_sites(fi, pack, args_of, B, sc.sh_deg)
		quality = None
		log(f'distinct blended sites per ray: {u_sh:.1f} (over {u_rays} traced rays)')
	abytes = algorithmic_bytes(stats.cpu(), sh_bytes, u_sh, indexed)
	st = stats.double()
	key = f'config{args.config}-scale{args.scale}-{args.colors}-reorder{int(not args.no_reorder)}-l{lanes}'
	if not ordered:
		key += f'-tiles{args.tile}{args.tile_curve}'
	if ordered:
		key += f'-order{dir_res}x{pos_bits}'
	if fast:
		key += f'-sh{"16" if args.sh_half else "32"}-ec{args.eps_color:g}-ed{args.eps_density:g}'
	if indexed:
		key += '-idx'
	if row_kind is not None:
		key += '-rows64' if pack['rows'].size(1) == 16 else '-blocks256'
	src = source_hash('foam_infer.hip')
	log(f'kernel source hash (foam_infer.hip): {src}; workload key {key}')
	roofline = hbm_roofline(ms, key, src, abytes,
							'cache-oblivious gather bytes from the per-ray counters: 56 B per ray + 24 B per sample + '
							f'{80 if indexed else 84} B per neighbourhood edge + SH bytes per distinct blended site '
							'(counts every L1/L2/LDS hit as a fetch, so it can exceed the HBM peak)',
							'foam_infer_kernel' if lanes == 1 else 'foam_group_kernel')
	if roofline['frac'] is not None and not fast and (mode == 2 or exact_blend) and lanes == 1:
		roofline['limiter'] = ('not HBM: the texture data path is busy 94 % of the launch and the L2 serves 93 % of '
							   'the gathers (profiles/foam_infer_config3_counters.md)')

	cpu = None
	if args.cpu_seconds > 0 and args.colors != 'baked':
		cpu = cpu_baseline(pack, sc, o_np, d_np, start.cpu().numpy(), near.cpu().numpy(), far.cpu().numpy(), mode,
						   args.cpu_seconds, rgb.cpu().numpy(), T.cpu().numpy(), color_cut)
	if args.copy_probe:
		copy_probe(dev)

	mrays = B / (ms * 1e-3) / 1e6
	res = {
		'metric': METRIC, 'value': round(mrays, 3), 'unit': 'Mrays/s', 'n_gpus': 1, 'steps': args.steps,
		'warmup': args.warmup, 'ms_per_step': round(ms, 4), 'higher_is_better': True, 'scaling': 'weak',
		'vs_baseline': None, 'dtype': 'f32', 'data': 'synthetic',
		'config': {
			'workload': f'BASELINE config {args.config}: foam_infer on the seeded {sc.n_sites}-site scene, '
						f'{frames} cameras x {W}x{H} = {B} rays per step',
			'sites': sc.n_sites, 'rays_per_step': B, 'frames_per_step': frames,
			'fps_1080p': round(frames / (ms * 1e-3), 2) if frames else None,
			'colors': args.colors, 'sh': 'f16' if args.sh_half else 'f32', 'sh_deg': sc.sh_deg,
			'lanes_per_ray': lanes,
			'edge_records': 'indexed (vgr_foam_infer_indexed)' if indexed else 'reference',
			'exact_colours': (('one-pass blend' if exact_blend else 'two passes') if mode == 0 else None),
			'site_rows': row_kind or '80-byte attr rows',
			'cache_misses': ('slot table, once per pass' if 'slots' in pack and lanes != 8 and math.isinf(color_cut)
							 else 'per-lookup tags in LDS')
			if args.colors != 'baked' else None,
			'eps_color': args.eps_color, 'eps_density': args.eps_density, 'morton_reorder': not args.no_reorder,
			'ray_order': (f'vgr_ray_order ({dir_res}x{dir_res} direction bins, {pos_bits}-bit origin Z-order) inside '
						  f'the timed step' if ordered else f'{args.tile}x{args.tile} tiles, {args.tile_curve} order'),
			't_thresh': 1e-4, 'w_thresh': 1e-4,
			'samples_per_ray': round(float(st[:, 0].mean()), 2),
			'density_terms_per_ray': round(float(st[:, 3].mean()), 1),
			'sh_cache_misses_per_ray': round(float(st[:, 4].mean()), 1),
			'distinct_blended_sites_per_ray': None if fast else round(u_sh, 1),
			'distinct_sites_traced_rays': u_rays or None, 'quality': quality,
			'mean_T': round(float(T.double().mean()), 4),
			'wave_lane_use_bound': wave_balance(stats),
		},
		'roofline': roofline,
		'cpu_baseline': cpu,
	}
	print(json.dumps(res), flush=True)


def cpu_baseline(pack, sc, o, d, start, near, far, mode, seconds, rgb_gpu, T_gpu, color_cut=math.inf):
	"""The CPU oracle (C/OpenMP, thread per ray, all host cores) on every k-th ray of the same workload, k chosen so
	that one timed pass takes about seconds / 4: 1 untimed warmup pass, then the median of 3 timed passes (the
	parallel loop only, steady_clock inside the oracle). Also the max |rgb - GPU| and |T - GPU| on that subset."""
	import numpy as np

	sys.path.insert(0, os.path.join(ROOT, 'oracle'))
	import oracle
	pk = {k: pack[k].cpu().numpy() for k in ('points', 'offsets', 'nbr', 'edge', 'attr', 'sh', 'orig')}
	threads = oracle.max_threads()
	B = len(o)
	probe = np.arange(0, B, max(1, B // 20000), dtype=np.int64)
	r = oracle.foam_infer(pk, sc.sh_deg, o, d, start, near, far, color_cut=color_cut, color_mode=mode, rays=probe)
	rate = len(probe) / max(r['seconds'], 1e-6)
	k = max(1, int(B / (rate * seconds / 4)))
	sel = np.arange(0, B, k, dtype=np.int64)
	secs, r = timed_cpu(lambda: oracle.foam_infer(pk, sc.sh_deg, o, d, start, near, far, color_cut=color_cut,
												  color_mode=mode, rays=sel))
	err = float(np.abs(r['rgb'] - rgb_gpu[sel]).max())
	errT = float(np.abs(r['T'] - T_gpu[sel]).max())
	log(f'cpu oracle: {len(sel)} rays (every {k}th), median of 3 passes {secs:.2f} s on {threads} threads '
		f'({cpu_model()}); max |rgb - gpu| {err:.2e}, max |T - gpu| {errT:.2e}')
	return {'value': round(len(sel) / secs / 1e6, 4), 'unit': 'Mrays/s', 'cores': threads, 'kind': 'port',
			'cpu': cpu_model(), 'timing': '1 warmup pass, then the median of 3 timed passes of the parallel loop',
			'sample': f'every {k}th ray of the same {B}-ray workload ({len(sel)} rays), same pack and colour mode, '
					  f'C/OpenMP thread per ray, schedule(dynamic)',
			'parity_max_abs_rgb': err, 'parity_max_abs_T': errT}


def time_steps(call, steps, warmup, stream):
	"""Runs `call` warmup times, then times `steps` calls with HIP events on `stream` -> (per-call ms list, last
	output, wall ms per step)."""
	import torch
	out = None
	for _ in range(warmup):
		out = call()
	torch.cuda.synchronize()
	ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
	torch.cuda.synchronize()
	wall0 = time.perf_counter()
	for a, b in ev:
		a.record(stream)
		out = call()
		b.record(stream)
	torch.cuda.synchronize()
	wall = (time.perf_counter() - wall0) * 1e3 / steps
	return [a.elapsed_time(b) for a, b in ev], out, wall


def emit(metric, value, unit, args, ms, config, roofline, cpu, dtype='f32'):
	res = {'metric': metric, 'value': round(value, 3), 'unit': unit, 'n_gpus': 1, 'steps': args.steps,
		   'warmup': args.warmup, 'ms_per_step': round(ms, 4), 'higher_is_better': True, 'scaling': 'weak',
		   'vs_baseline': None, 'dtype': dtype, 'data': 'synthetic', 'config': config, 'roofline': roofline,
		   'cpu_baseline': cpu}
	print(json.dumps(res), flush=True)


def training_rays(sc, points, B, dev, seed=0):
	"""B rays drawn uniformly over the pixels of the scene's cameras (scene.random_rays, train.py:132), with the
	start site of each camera's eye -> o, d, start (device tensors)."""
	import numpy as np
	import torch

	from vgr.sites import nearest_sites
	rng = np.random.default_rng(seed)
	cams = rng.integers(0, len(sc.cameras), B)
	o_l, d_l, e_l = [], [], []
	for c in range(len(sc.cameras)):
		n_c = int((cams == c).sum())
		o_c, d_c = sc.cameras[c].rays()
		pick = rng.choice(len(o_c), n_c, replace=False)
		o_l.append(o_c[pick]), d_l.append(d_c[pick]), e_l.append(np.repeat(sc.cameras[c].eye[None], n_c, 0))
	o = torch.from_numpy(np.concatenate(o_l)).to(dev)
	d = torch.from_numpy(np.concatenate(d_l)).to(dev)
	pts = torch.from_numpy(np.concatenate(e_l).astype(np.float32)).to(dev)
	return o, d, nearest_sites(points, pts)


def bench_foam_grad(args):
	"""A training step of the training renderer (render_rays_foam under autograd, train.py's default renderer,
	train.py:117,132) on config 3: --batch rays (train.py's default 4096) drawn over the pixels of the 4 cameras;
	vgr_foam_forward recording up to 256 samples per ray (ext.foam's default), then vgr_foam_backward replaying the
	records with random upstream gradients. value = rays per second through forward + backward; a second leg times
	16 x the batch. CPU baseline: the C oracle's backward (one thread, re-tracing) on a bounded subset.

	Algorithmic bytes of the backward launch (E = mean self-inclusive neighbourhood, SHB = 12 (deg + 1)^2): per
	sample the record 32 B and one scatter round E (16 + 28 + 28) (point, raw and density conic read, gradients
	written); per coloured sample E (SHB + 24 + SHB) more (SH read, colour-conic and SH gradient)."""
	import numpy as np
	import torch

	from vgr import _lib, ext, render, scenes
	from vgr.model import VoronoiGaussField
	dev = torch.device('cuda:0')
	sc = scenes.make_scene(3, scale=args.scale, log=log)
	model = VoronoiGaussField.from_scene(sc, dev)
	g = model.graph
	dA = ext.conic(model.d_log_scale, model.d_quat, 0.0).contiguous()
	cA = ext.conic(model.c_log_scale, model.c_quat, 0.0).contiguous()
	sh = model.sh().contiguous()
	fx = ext.foam_extension()
	stream = torch.cuda.current_stream(dev)
	E = 1.0 + len(sc.adj) / sc.n_sites
	SHB = 12 * (sc.sh_deg + 1) ** 2
	legs = {}
	for B in (args.batch, 16 * args.batch):
		o, d, start = training_rays(sc, g.points, B, dev)
		near, _, far = render.ray_bounds(o, d, 0.02, sc.far_radius)
		rays = (o, d, start, near, far)
		fwd = (g.points, g.offsets, g.adj, model.raw, dA, cA, sh, sc.sh_deg, *rays, 1e-4, 1e-4)
		gen = torch.Generator(device=dev).manual_seed(0)
		g_rgb, g_T = torch.randn(B, 3, device=dev, generator=gen), torch.randn(B, device=dev, generator=gen)
		# one workspace for both passes, as ext.foam's autograd uses it: the backward reuses the forward's blocks
		work = torch.empty(int(_lib.load().vgr_foam_work_size(sc.n_sites, sc.sh_deg)), dtype=torch.uint8, device=dev)
		f_ms, out, _ = time_steps(lambda: fx.foam_forward(*fwd, 256, work=work), args.steps, args.warmup, stream)
		rgb, T, _, stats, rec = out
		b_ms, _, _ = time_steps(lambda: fx.foam_backward(*fwd, rgb, T, g_rgb, g_T, rec, stats, work=work),
								args.steps, args.warmup, stream)
		st = stats.double()
		bwd_bytes = float(st[:, 0].sum() * (32 + E * 72) + st[:, 1].sum() * 2 * E * (2 * SHB + 24))
		legs[B] = dict(fwd=float(np.mean(f_ms)), bwd=float(np.mean(b_ms)), bytes=bwd_bytes, rays=rays, rgb=rgb, T=T,
					   g_rgb=g_rgb, g_T=g_T, samples=float(st[:, 0].mean()), coloured=float(st[:, 1].mean()),
					   fits=float((stats[:, 0] <= 256).double().mean()))
		L = legs[B]
		log(f'{B} rays: forward {L["fwd"]:.3f} ms, backward {L["bwd"]:.3f} ms; samples/ray {L["samples"]:.1f}, '
			f'coloured segments {L["coloured"]:.1f}, rays within the records {100 * L["fits"]:.1f} %')
	L = legs[args.batch]
	ms = L['fwd'] + L['bwd']
	cpu = None
	if args.cpu_seconds > 0:
		sys.path.insert(0, os.path.join(ROOT, 'oracle'))
		import oracle
		host = [x.cpu().numpy() for x in (g.points, g.offsets, g.adj, model.raw, dA, cA, sh)]
		rays = [x.cpu().numpy() for x in L['rays']]
		up = [x.cpu().numpy() for x in (L['rgb'], L['T'], L['g_rgb'], L['g_T'])]
		B = args.batch
		probe = np.arange(0, B, max(1, B // 16))
		t1 = time.perf_counter()
		oracle.foam_backward(*host, sc.sh_deg, *[r[probe] for r in rays], *[u[probe] for u in up])
		rate = len(probe) / max(time.perf_counter() - t1, 1e-6)
		sel = np.arange(0, B, max(1, int(B / (rate * args.cpu_seconds))))
		t1 = time.perf_counter()
		oracle.foam_backward(*host, sc.sh_deg, *[r[sel] for r in rays], *[u[sel] for u in up])
		secs = time.perf_counter() - t1
		cpu = {'value': round(len(sel) / secs / 1e3, 4), 'unit': 'Krays/s (backward only)', 'cores': 1,
			   'kind': 'port', 'sample': f'{sample_words(B, len(sel))}, C oracle '
										 f'foam_backward (re-tracing), one thread'}
	big = legs[16 * args.batch]
	emit('Mrays/s through foam forward + backward (training batch)', mrays_per_s(args.batch, ms), 'Mrays/s', args, ms,
		 {'workload': f'config 3 training step of the training renderer: {args.batch} random rays over the 4 '
					  f'cameras, foam_forward (256 records per ray) + foam_backward', 'sites': sc.n_sites,
		  'rays_per_step': args.batch, 'forward_ms': round(L['fwd'], 4), 'backward_ms': round(L['bwd'], 4),
		  'samples_per_ray': round(L['samples'], 2), 'coloured_segments_per_ray': round(L['coloured'], 2),
		  'rays_within_records': round(L['fits'], 4),
		  f'rays_{16 * args.batch}': {'forward_ms': round(big['fwd'], 3), 'backward_ms': round(big['bwd'], 3),
									  'Mrays_per_s': round(mrays_per_s(16 * args.batch, big['fwd'] + big['bwd']), 3)}},
		 hbm_roofline(L['bwd'], f'config3-foam-grad-b{args.batch}', source_hash('march.hip'), L['bytes'],
					  'cache-oblivious bytes of the backward launch (records, site blocks and gradient rows per sample)',
					  'train_backward_kernel'), cpu)


def bench_march_grad(args):
	"""A training step of the uniform march (render_rays_uniform under autograd, train.py:114,132) on config 5:
	--batch rays (train.py's default 4096) drawn at random from the config-5 ray batch, dt = 1/512 and 64 disparity
	steps (train.py:35-36); march_forward, then march_backward with random upstream gradients of rgb and T. value =
	rays per second through forward + backward. A second leg times 16 x the batch, since 4,096 rays (64 waves of one
	ray per lane) occupy a fraction of the 1,024 SIMDs. CPU baseline: the C oracle's backward (one thread) on a
	bounded subset of the batch.

	Algorithmic bytes of the backward launch (E = mean self-inclusive neighbourhood, SHB = 12 (deg + 1)^2): the
	forward's (rays 56 B; per walk step 8 + 16 E; per sample 8 + 44 E; per coloured sample E (24 + SHB)) again for
	the re-march, plus the gradient pass: per sample E (16 + 28) record reads and E 28 B of raw and density-conic
	gradient, per coloured sample E (SHB + 24 + SHB) SH reads and colour-conic and SH gradient."""
	import numpy as np
	import torch

	from vgr import _lib, ext, grid, render, scenes
	from vgr.model import VoronoiGaussField
	dev = torch.device('cuda:0')
	sc = scenes.make_scene(5, scale=args.scale, log=log)
	model = VoronoiGaussField.from_scene(sc, dev)
	o_np, d_np = sc.ray_batch
	dt, n_bg = 1 / 512, 64
	floor = 0.5 * dt
	dA = ext.conic(model.d_log_scale, model.d_quat, floor).contiguous()
	cA = ext.conic(model.c_log_scale, model.c_quat, floor).contiguous()
	sh = model.sh().contiguous()
	me = ext.march_extension()
	g = model.graph
	sites = g.points
	locator = grid.SiteGrid(sites)
	stream = torch.cuda.current_stream(dev)
	E = 1.0 + len(sc.adj) / sc.n_sites
	SHB = 12 * (sc.sh_deg + 1) ** 2
	rng = np.random.default_rng(0)
	legs = {}
	for B in (args.batch, 16 * args.batch):
		pick = rng.choice(len(o_np), B, replace=False)
		o, d = torch.from_numpy(o_np[pick]).to(dev), torch.from_numpy(d_np[pick]).to(dev)
		start = locator.nearest(o)
		near, mid, far = render.ray_bounds(o, d, 0.02, sc.far_radius)
		rays = (o, d, start, near, mid, far)
		fwd_args = (g.points, g.offsets, g.adj, model.raw, dA, cA, sh, sc.sh_deg, *rays, dt, n_bg, 1e-4, 1e-4)
		gen = torch.Generator(device=dev).manual_seed(0)
		g_rgb, g_T = torch.randn(B, 3, device=dev, generator=gen), torch.randn(B, device=dev, generator=gen)
		# one workspace for both passes, as ext.march's autograd uses it: the backward reuses the forward's blocks
		work = torch.empty(int(_lib.load().vgr_march_backward_work_size(sc.n_sites, sc.sh_deg)), dtype=torch.uint8,
						   device=dev)
		for lanes in (1, 16):  # both ray layouts; the library's default picks 16 below 524288 rays
			f_ms, out, _ = time_steps(lambda: me.march_forward(*fwd_args, lanes=lanes, work=work), args.steps,
									  args.warmup, stream)
			rgb, T, _, stats = out
			b_ms, grads, _ = time_steps(lambda: me.march_backward(*fwd_args, rgb, T, g_rgb, g_T, lanes=lanes,
																  work=work), args.steps, args.warmup, stream)
			st = stats.double()
			fwd_bytes = float(56 * B + st[:, 2].sum() * (8 + 16 * E) + st[:, 0].sum() * (8 + E * 44) +
							  st[:, 1].sum() * E * (24 + SHB))
			bwd_bytes = fwd_bytes + float(st[:, 0].sum() * E * (44 + 28) + st[:, 1].sum() * E * (2 * SHB + 24))
			legs[B, lanes] = dict(fwd=float(np.mean(f_ms)), bwd=float(np.mean(b_ms)), bytes=bwd_bytes, rays=rays,
								  rgb=rgb, T=T, g_rgb=g_rgb, g_T=g_T, samples=float(st[:, 0].mean()),
								  coloured=float(st[:, 1].mean()))
			L = legs[B, lanes]
			log(f'{B} rays, {lanes} lane(s) per ray: forward {L["fwd"]:.3f} ms, backward {L["bwd"]:.3f} ms '
				f'({bwd_bytes / L["bwd"] / 1e6:.0f} GB/s algorithmic); samples/ray {L["samples"]:.1f}, coloured '
				f'{L["coloured"]:.1f}')
	auto = 16 if args.batch < 524288 else 1
	L = legs[args.batch, auto]
	ms = L['fwd'] + L['bwd']
	cpu = None
	if args.cpu_seconds > 0:
		sys.path.insert(0, os.path.join(ROOT, 'oracle'))
		import oracle
		host = [x.cpu().numpy() for x in (g.points, g.offsets, g.adj, model.raw, dA, cA, sh)]
		rays = [x.cpu().numpy() for x in L['rays']]
		up = [x.cpu().numpy() for x in (L['rgb'], L['T'], L['g_rgb'], L['g_T'])]
		B = args.batch
		t1 = time.perf_counter()
		probe = np.arange(0, B, max(1, B // 16))
		oracle.march_backward(*host, sc.sh_deg, *[r[probe] for r in rays], dt, n_bg, *[u[probe] for u in up])
		rate = len(probe) / max(time.perf_counter() - t1, 1e-6)
		sel = np.arange(0, B, max(1, int(B / (rate * args.cpu_seconds))))
		t1 = time.perf_counter()
		oracle.march_backward(*host, sc.sh_deg, *[r[sel] for r in rays], dt, n_bg, *[u[sel] for u in up])
		secs = time.perf_counter() - t1
		cpu = {'value': round(len(sel) / secs / 1e3, 4), 'unit': 'Krays/s (backward only)', 'cores': 1,
			   'kind': 'port', 'sample': f'{sample_words(B, len(sel))}, C oracle '
										 f'march_backward, one thread'}
	layouts = {f'{B} rays, {lanes} lanes/ray': {'forward_ms': round(v['fwd'], 3), 'backward_ms': round(v['bwd'], 3),
												'Mrays_per_s': round(mrays_per_s(B, v['fwd'] + v['bwd']), 3)}
			   for (B, lanes), v in legs.items()}
	emit('Mrays/s through march forward + backward (training batch)', mrays_per_s(args.batch, ms), 'Mrays/s', args, ms,
		 {'workload': f'config 5 uniform march training step: {args.batch} random rays of the config-5 batch, dt = '
					  f'1/512, 64 bg steps, march_forward + march_backward', 'sites': sc.n_sites,
		  'rays_per_step': args.batch, 'lanes_per_ray': auto, 'forward_ms': round(L['fwd'], 4),
		  'backward_ms': round(L['bwd'], 4), 'samples_per_ray': round(L['samples'], 2),
		  'coloured_per_ray': round(L['coloured'], 2), 'layouts': layouts},
		 hbm_roofline(L['bwd'], f'config5-march-grad-b{args.batch}', source_hash('march.hip'), L['bytes'],
					  'cache-oblivious bytes of the backward launch (site blocks per neighbour visit, gradient rows)',
					  'march_group_backward_kernel' if auto == 16 else 'march_backward_kernel'), cpu)


def sample_words(B, n):
	"""How a CPU-baseline subset of n of the batch's B rays was drawn."""
	return f'all {B} rays of the batch' if n == B else f'every {B // n}th ray of the batch ({n} rays)'


def mrays_per_s(B, ms):
	return B / (ms * 1e-3) / 1e6


def bench_locate(args):
	"""Start-cell location for config 5: the nearest of 4,000,000 sites for each of the 16,777,216 ray origins
	(vgr_grid_nearest_points over a grid and its cell-ordered sites built once, outside the timed region; the
	origins answered in their Z-order, computed inside the timed step, unless --order off). CPU baseline: the
	reference's own nearest_sites (scipy cKDTree, sites.py:38-39, single-threaded as called there) on a bounded
	sample."""
	import numpy as np
	import torch

	from vgr import grid, scenes
	dev = torch.device('cuda:0')
	pts_np = scenes.site_points(5, args.scale)
	o_np, _ = scenes.ray_batch(5)
	pts, q = torch.from_numpy(pts_np).to(dev), torch.from_numpy(o_np).to(dev)
	N, B = len(pts), len(q)
	log(f'config 5 sites {N}, ray origins {B}')
	stream = torch.cuda.current_stream(dev)
	build_ms, g, _ = time_steps(lambda: grid.SiteGrid(pts), 3, 1, stream)
	n_cells = g.res[0] * g.res[1] * g.res[2]
	ordered = args.order != 'off'  # the origins of a ray batch come in no spatial order
	pos_bits = args.order_pos_bits or 8
	if ordered:
		step = lambda: g.nearest(q, order=grid.query_order(q, pos_bits))  # noqa: E731
	else:
		step = lambda: g.nearest(q)  # noqa: E731
	launch_ms, out, wall = time_steps(step, args.steps, args.warmup, stream)
	ms = float(np.mean(launch_ms))
	log(f'grid {g.res} ({n_cells} cells) built in {np.mean(build_ms):.3f} ms; {args.steps} queries launches: '
		f'mean {ms:.3f} ms, wall {wall:.3f} ms/step')
	# compulsory bytes of one launch: query in (12 B), site out (4 B); the grid and points read once
	abytes = 16.0 * B + 16.0 * N + 4.0 * N + 4.0 * (n_cells + 1)
	cpu = None
	if args.cpu_seconds > 0:
		from scipy.spatial import cKDTree
		t0 = time.perf_counter()
		tree = cKDTree(pts_np)
		t_build = time.perf_counter() - t0
		probe = o_np[:20000]
		t0 = time.perf_counter()
		tree.query(probe)
		rate = len(probe) / (time.perf_counter() - t0)
		k = max(1, int(B / (rate * args.cpu_seconds)))
		sel = np.arange(0, B, k)
		t0 = time.perf_counter()
		ref = tree.query(o_np[sel])[1]
		t = time.perf_counter() - t0
		mism = int((out.cpu().numpy()[sel] != ref).sum())
		log(f'cpu cKDTree: build {t_build:.2f} s, {len(sel)} queries (every {k}th) in {t:.2f} s; '
			f'{mism} mismatches against the GPU')
		cpu = {'value': round(len(sel) / t / 1e6, 4), 'unit': 'Mqueries/s', 'cores': 1, 'kind': 'reference',
			   'sample': f'every {k}th of the {B} ray origins ({len(sel)} queries), scipy cKDTree.query as in the '
						 f'reference nearest_sites (sites.py:38-39), single-threaded; tree build {t_build:.2f} s '
						 f'not included', 'parity_mismatches': mism}
	emit('Mqueries/s nearest-site start location (config 5: 4M sites, 16.7M ray origins) on 1 MI355X', B / ms / 1e3,
		 'Mqueries/s', args, ms,
		 {'workload': f'config 5 start cells: nearest of {N} sites (seeded uniform draw) for each of {B} ray '
					  f'origins', 'sites': N, 'queries': B, 'grid_res': g.res,
		  'grid_build_ms': round(float(np.mean(build_ms)), 3),
		  'query_order': (f'Z-order of the origins, {pos_bits} bits per axis (vgr_ray_order, one direction bin), '
						  f'inside the timed step' if ordered else 'as given')},
		 hbm_roofline(ms, 'config5-locate' + (f'-order{pos_bits}' if ordered else ''), source_hash('grid.hip'), abytes,
					  'compulsory bytes: each query point, site and grid word read once, each answer written once',
					  'grid_nearest'), cpu)


def bench_march(args):
	"""march_forward on config 5: 4,000,000 uniform sites of low density (no early termination), 16,777,216
	incoherent rays from inside [-0.9, 0.9]^3, start sites from the GPU grid, dt = 1/512 inside the unit ball and 64
	disparity steps beyond (render.py:109-124 defaults). CPU baseline: the C/OpenMP oracle on a bounded sample."""
	import numpy as np
	import torch

	from vgr import ext, grid, render, scenes
	from vgr.model import VoronoiGaussField
	dev = torch.device('cuda:0')
	t0 = time.time()
	sc = scenes.make_scene(5, scale=args.scale, log=log)
	log(f'scene config 5: {sc.n_sites} sites ({time.time() - t0:.0f} s)')
	model = VoronoiGaussField.from_scene(sc, dev)
	o_np, d_np = sc.ray_batch
	o, d = torch.from_numpy(o_np).to(dev), torch.from_numpy(d_np).to(dev)
	start = grid.SiteGrid(model.graph.points).nearest(o)
	dt, n_bg = 1 / 512, 64
	near, mid, far = render.ray_bounds(o, d, 0.02, sc.far_radius)
	floor = 0.5 * dt
	dA = ext.conic(model.d_log_scale, model.d_quat, floor)
	cA = ext.conic(model.c_log_scale, model.c_quat, floor)
	sh = model.sh().contiguous()
	B = len(o)
	me = ext.march_extension()
	args_of = lambda sel=slice(None): (model.graph.points, model.graph.offsets, model.graph.adj, model.raw, dA, cA, sh,  # noqa
									   sc.sh_deg, o[sel], d[sel], start[sel], near[sel], mid[sel], far[sel], dt, n_bg,
									   1e-4, 1e-4)
	stream = torch.cuda.current_stream(dev)
	lanes = args.lanes_per_ray or 0
	ordered = args.order != 'off'
	dir_res, pos_bits = args.order_dir_res or 4, args.order_pos_bits or 8

	def step():
		order = ext.ray_order(o, d, dir_res, pos_bits) if ordered else None
		return me.march_forward(*args_of(), lanes=lanes, order=order)
	launch_ms, out, wall = time_steps(step, args.steps, args.warmup, stream)
	ms = float(np.mean(launch_ms))
	rgb, T, depth, stats = out
	st = stats.double()
	log(f'{args.steps} steps: mean {ms:.3f} ms, wall {wall:.3f} ms/step; samples/ray {st[:, 0].mean():.1f}, '
		f'coloured {st[:, 1].mean():.1f}, walk steps {st[:, 2].mean():.1f}')
	E = 1.0 + len(sc.adj) / sc.n_sites  # mean self-inclusive neighbourhood
	SHB = 12 * (sc.sh_deg + 1) ** 2
	# per sample: walk steps (8 + 16 E) each, density (8 + E (16 + 28)), colour when active E (24 + SHB); rays 56 B
	abytes = float(56 * B + st[:, 2].sum() * (8 + 16 * E) + st[:, 0].sum() * (8 + E * 44) +
				   st[:, 1].sum() * E * (24 + SHB))
	cpu = None
	if args.cpu_seconds > 0:
		sys.path.insert(0, os.path.join(ROOT, 'oracle'))
		import oracle
		host = [x.cpu().numpy() for x in (model.graph.points, model.graph.offsets, model.graph.adj, model.raw, dA, cA,
										  sh)]
		rays = [x.cpu().numpy() for x in (o, d, start, near, mid, far)]
		probe = np.arange(0, B, max(1, B // 2000), dtype=np.int64)
		r = oracle.march_forward(*host, sc.sh_deg, *rays, dt, n_bg, rays=probe)
		rate = len(probe) / max(r['seconds'], 1e-6)
		k = max(1, int(B / (rate * args.cpu_seconds)))
		sel = np.arange(0, B, k, dtype=np.int64)
		r = oracle.march_forward(*host, sc.sh_deg, *rays, dt, n_bg, rays=sel)
		err = float(np.abs(r['rgb'] - rgb.cpu().numpy()[sel]).max())
		errT = float(np.abs(r['T'] - T.cpu().numpy()[sel]).max())
		# the same rays with the thresholds off (t_thresh = 0, w_thresh = -1): every sample coloured, no early stop,
		# so no decision can flip on the few-ulp difference between the device exp and the host's
		sub = sel[:: max(1, len(sel) // 20000)]
		gs = me.march_forward(*args_of(torch.from_numpy(sub).to(dev))[:-2], 0.0, -1.0)
		rs = oracle.march_forward(*host, sc.sh_deg, *rays, dt, n_bg, t_thresh=0.0, w_thresh=-1.0, rays=sub)
		err_off = float(np.abs(rs['rgb'] - gs[0].cpu().numpy()).max())
		errT_off = float(np.abs(rs['T'] - gs[1].cpu().numpy()).max())
		log(f'cpu oracle: {len(sel)} rays (every {k}th) in {r["seconds"]:.2f} s on {oracle.max_threads()} threads; '
			f'max |rgb - gpu| {err:.2e}, max |T - gpu| {errT:.2e}; thresholds off ({len(sub)} rays): '
			f'{err_off:.2e}, {errT_off:.2e}')
		cpu = {'value': round(len(sel) / r['seconds'] / 1e6, 5), 'unit': 'Mrays/s', 'cores': oracle.max_threads(),
			   'kind': 'port', 'sample': f'every {k}th ray of the same {B}-ray batch ({len(sel)} rays), C/OpenMP '
										 f'thread per ray', 'parity_max_abs_rgb': err, 'parity_max_abs_T': errT,
			   'parity_thresholds_off_max_abs_rgb': err_off, 'parity_thresholds_off_max_abs_T': errT_off,
			   'parity_note': 'with w_thresh = 1e-4 many config-5 samples have weight within ulps of the threshold, so '
							  'device and host exp (the reference uses __expf, march.cu:241) colour slightly different '
							  'sample sets; the thresholds-off figures compare the arithmetic'}
	if args.copy_probe:
		copy_probe(dev)
	emit('Mrays/s march_forward (config 5: 4M sites, 16.7M incoherent rays) on 1 MI355X', B / ms / 1e3, 'Mrays/s',
		 args, ms,
		 {'workload': f'config 5 march: {sc.n_sites} sites, {B} rays, dt 1/512 inside the unit ball + {n_bg} '
					  f'disparity steps, starts from the GPU grid', 'sites': sc.n_sites, 'rays': B,
		  'samples_per_ray': round(float(st[:, 0].mean()), 2),
		  'coloured_samples_per_ray': round(float(st[:, 1].mean()), 2),
		  'walk_steps_per_ray': round(float(st[:, 2].mean()), 2), 'mean_T': round(float(T.double().mean()), 4),
		  'wave_lane_use_bound': wave_balance(stats[ext.ray_order(o, d, dir_res, pos_bits).long()] if ordered else stats,
											  cols=(('samples', 0), ('walk_steps', 2))),
		  'lanes_per_ray': lanes or (16 if B < 524288 else 1),
		  'ray_order': f'vgr_ray_order ({dir_res}x{dir_res} direction bins, {pos_bits}-bit origin Z-order) inside the '
					   f'timed step' if ordered else 'batch order'},
		 hbm_roofline(ms, f'config5-scale{args.scale}-march-l{lanes or (16 if B < 524288 else 1)}' +
					  (f'-order{dir_res}x{pos_bits}' if ordered else ''), source_hash('march.hip', 'order.hip'), abytes,
					  'cache-oblivious bytes from the per-ray counters: per walk step 8 + 16 E, per sample 8 + 44 E, '
					  'per coloured sample E (24 + SH bytes)', 'march_forward_kernel'), cpu)


def bench_traverse(args):
	"""The traversal alone (walk to the start cell, then exit faces cell to cell: foam_infer with stage 0) of the
	config-3 workload in the two wave64 layouts: one ray per lane over 8x8 tiles (vgr_foam_infer_lanes with 1 lane
	per ray) and a group of 4, 8 or 16 lanes per ray, each testing every 4th / 8th / 16th face, with a group
	min-reduction (vgr_foam_traverse_faces). All must give the same per-ray statistics; the JSON line is the
	lane-per-face layout of --lanes, the others beside it."""
	import numpy as np
	import torch

	from vgr import ext, render, scenes
	from vgr.model import VoronoiGaussField
	dev = torch.device('cuda:0')
	sc = scenes.make_scene(args.config, scale=args.scale, log=log)
	model = VoronoiGaussField.from_scene(sc, dev)
	pack = render.pack_foam(model, reorder=True, index=False)
	o_np, d_np, start_np, _ = sc.camera_rays(tile=args.tile, curve=args.tile_curve)
	o, d = torch.from_numpy(o_np).to(dev), torch.from_numpy(d_np).to(dev)
	start = pack['inv'][torch.from_numpy(start_np).to(dev).long()].int()
	near, _, far = render.ray_bounds(o, d, 0.02, sc.far_radius)
	B = len(o)
	empty = torch.empty(0, dtype=torch.int32, device=dev)
	fi = ext.foam_infer_extension()
	stream = torch.cuda.current_stream(dev)
	lane_ms, out_lane, _ = time_steps(
		lambda: fi.foam_infer(pack['points'], pack['offsets'], pack['nbr'], pack['edge'], pack['attr'], pack['sh'],
							  sc.sh_deg, o, d, start, near, far, 1e-4, 1e-4, math.inf, 0, 0, empty, pack['orig'],
							  lanes=1),
		args.steps, args.warmup, stream)
	ms_lane = float(np.mean(lane_ms))
	group_ms, same = {}, True
	for lanes in (4, 8, 16):
		face_ms, stats_face, _ = time_steps(
			lambda: ext.traverse_faces(pack['points'], pack['offsets'], pack['nbr'], pack['edge'], o, d, start, near,
									   far, orig=pack['orig'], lanes=lanes), args.steps, args.warmup, stream)
		group_ms[lanes] = float(np.mean(face_ms))
		same = same and bool(torch.equal(out_lane[3], stats_face))
	ms_face = group_ms[args.lanes]
	st = stats_face.double()
	log(f'stage-0 traversal of {B} rays: one ray per lane {ms_lane:.3f} ms; ' +
		', '.join(f'{g} lanes per ray {ms:.3f} ms' for g, ms in group_ms.items()) +
		f'; per-ray statistics identical: {same}; {st[:, 0].mean():.1f} cells per ray')
	cpu = None
	if args.cpu_seconds > 0:  # the oracle's traversal (stage 0) on every k-th ray: rate and stats parity
		sys.path.insert(0, os.path.join(ROOT, 'oracle'))
		import oracle
		pk = {k: pack[k].cpu().numpy() for k in ('points', 'offsets', 'nbr', 'edge', 'attr', 'sh', 'orig')}
		args_np = (pk, sc.sh_deg, o_np, d_np, start.cpu().numpy(), near.cpu().numpy(), far.cpu().numpy())
		probe = np.arange(0, B, max(1, B // 20000), dtype=np.int64)
		r = oracle.foam_infer(*args_np, stage=0, rays=probe)
		k = max(1, int(B / (len(probe) / max(r['seconds'], 1e-6) * args.cpu_seconds)))
		sel = np.arange(0, B, k, dtype=np.int64)
		r = oracle.foam_infer(*args_np, stage=0, rays=sel)
		cpu_same = bool(np.array_equal(r['stats'], stats_face.cpu().numpy()[sel]))
		log(f'cpu oracle traversal: {len(sel)} rays in {r["seconds"]:.2f} s; stats identical to the GPU: {cpu_same}')
		cpu = {'value': round(len(sel) / r['seconds'] / 1e6, 4), 'unit': 'Mrays/s', 'cores': oracle.max_threads(),
			   'kind': 'port', 'sample': f'every {k}th ray of the same {B}-ray workload ({len(sel)} rays), stage 0, '
										 f'C/OpenMP thread per ray', 'identical_stats': cpu_same}
	if args.copy_probe:
		copy_probe(dev)
	E = 1.0 + len(sc.adj) / sc.n_sites
	# per visited cell: the cell position (16 B) and offsets (8 B), then per face the edge record (16 B) and nbr (4 B)
	abytes = float(56 * B + st[:, 0].sum() * (24 + 20 * E))
	emit(f'Mrays/s cell traversal, {args.lanes} lanes per ray (config {args.config}: {sc.n_sites} sites, 4 x 1080p)',
		 B / ms_face / 1e3, 'Mrays/s', args, ms_face,
		 {'workload': f'config {args.config}: foam_infer stage 0 (walk + exit faces) over {B} camera rays',
		  'layout': f'{args.lanes} lanes per ray, DPP group min-reduction of the exit face',
		  'thread_per_ray_ms': round(ms_lane, 4),
		  'lane_per_face_ms': {str(g): round(ms, 4) for g, ms in group_ms.items()},
		  'identical_stats': same, 'cells_per_ray': round(float(st[:, 0].mean()), 2)},
		 hbm_roofline(ms_face, f'config{args.config}-traverse-l{args.lanes}', source_hash('foam_faces.hip'), abytes,
					  'cache-oblivious bytes: 56 B per ray, per visited cell 24 B + 20 B per face',
					  'foam_faces_kernel'), cpu)


def bench_pack(args):
	"""The step before the kernel (render.py:168-225): pack_foam with the Z-order renumbering of the config-3 scene
	(conics on the GPU, self-first CSR, edge records with the half2 cut-offs, site records, SH rows), from the model's
	device tensors, timed whole. CPU baseline: the same pack on host tensors (torch on the host cores), whose
	non-renumbered records must equal the GPU's bit for bit."""
	import numpy as np
	import torch

	from vgr import ext, render, scenes
	from vgr.model import VoronoiGaussField
	dev = torch.device('cuda:0')
	sc = scenes.make_scene(args.config, scale=args.scale, log=log)
	model = VoronoiGaussField.from_scene(sc, dev)
	N, M = sc.n_sites, len(sc.adj)
	stream = torch.cuda.current_stream(dev)
	torch.cuda.synchronize()
	torch.cuda.reset_peak_memory_stats()
	base = torch.cuda.memory_allocated()
	launch_ms, pk, wall = time_steps(lambda: render.pack_foam(model, reorder=True, index=False), args.steps, args.warmup, stream)
	peak = (torch.cuda.max_memory_allocated() - base) / 2 ** 30
	ms = float(np.mean(launch_ms))
	log(f'pack_foam (reorder) of {N} sites, {M} adjacency entries: mean {ms:.3f} ms, wall {wall:.3f} ms/step, '
		f'peak +{peak:.2f} GiB')
	# compulsory bytes: inputs (points 12, offsets 4, raw 4, log-scales 24, quaternions 32, SH 192 per site, adjacency
	# 4 per entry) read once; outputs (points 16, offsets 4, attr 80, SH 192, perm/inv/orig 20 per site, nbr 4 and
	# edge 16 per self-first entry) written once
	shb = 192
	abytes = float(N * (12 + 4 + 4 + 24 + 32 + shb) + 4 * M + N * (16 + 4 + 80 + shb + 20) + (M + N) * 20)
	cpu = None
	if args.cpu_seconds > 0:
		# the host pack takes the device conics (conic_forward is its own row), then builds everything else
		g = model.graph
		dA = ext.conic(model.d_log_scale, model.d_quat, 0.0)
		cA = ext.conic(model.c_log_scale, model.c_quat, 0.0)
		hin = [x.detach().cpu() for x in (g.points, g.offsets, g.adj, model.raw, model.d_log_scale,
										  model.c_log_scale, dA, cA, model.sh())]
		t0 = time.perf_counter()
		render.pack_foam_arrays(*hin, reorder=True)
		t_cpu = time.perf_counter() - t0
		g0, r0 = render.pack_foam(model, reorder=False, index=False), render.pack_foam_arrays(*hin, reorder=False)
		# copied fields must match bit for bit; the cut-off words come from torch exp on two devices (a few ulps
		# apart) rounded to half, so a rare one may differ in its last half bit
		same = all(torch.equal(g0[k].cpu(), r0[k]) for k in ('points', 'offsets', 'nbr', 'attr', 'sh'))
		same = same and torch.equal(g0['edge'][:, :3].cpu(), r0['edge'][:, :3])
		cut_g = g0['edge'][:, 3].cpu().view(torch.int32)
		cut_r = r0['edge'][:, 3].view(torch.int32)
		cut_diff = float((cut_g != cut_r).double().mean())
		log(f'cpu pack (torch, {torch.get_num_threads()} threads): {t_cpu:.2f} s; copied fields equal to the host '
			f'ones without renumbering: {same}; cut-off words differing: {cut_diff:.2e} of the edges')
		cpu = {'value': round(N / t_cpu / 1e6, 4), 'unit': 'Msites/s', 'cores': torch.get_num_threads(), 'kind': 'port',
			   'sample': f'the whole {N}-site pack with renumbering, torch on host tensors, from the device conics',
			   'parity_bitwise_copied_fields': same, 'parity_cut_words_differing': cut_diff}
	emit(f'Msites/s pack_foam with Z-order renumbering (config {args.config}: {N} sites) on 1 MI355X', N / ms / 1e3,
		 'Msites/s', args, ms,
		 {'workload': f'config {args.config} pack: {N} sites, {M} adjacency entries, SH degree {sc.sh_deg}, Z-order '
					  f'renumbering', 'sites': N, 'adjacency': M, 'peak_extra_GiB': round(peak, 2)},
		 hbm_roofline(ms, f'config{args.config}-pack', source_hash('pack.hip'), abytes,
					  'compulsory bytes: every input read once and every packed record written once',
					  'pack_foam (all passes)'), cpu)


def bench_field(args):
	"""The field operators of the NeRF path on config 3, one 1920x1080 frame (2,073,600 rays) at 64 stratified
	samples per ray, as the first round of render_rays (render.py:77-106): walk to the sample sites, density at
	every sample, colour at the samples whose compositing weight exceeds 1e-4; conic_forward over all sites.
	value = samples per second through walk + density + colour. Each operator is timed on its own with HIP events
	and beside the C/OpenMP oracle on a bounded sample.

	Algorithmic bytes (cache-oblivious; E = mean self-inclusive neighbourhood, SHB = 192 B at SH degree 3):
	  walk     per sample (1 + walk steps) (8 + 16 E) + 8     (offsets; point 12 + adj 4 per neighbour; z in, site out)
	  density  per sample 28 + 48 E    (x, site, sigma, offsets; point 12 + adj 4 + raw 4 + log_scale 12 + quat 16)
	  colour   per active sample 48 + E (44 + SHB)   (x, dir, site, rgb, offsets; point, adj, log_scale, quat, SH)
	  conic    per site 60 (log_scale 12 + quat 16 in, A 24 out)."""
	import numpy as np
	import torch

	from vgr import ext, render, scenes
	from vgr.model import VoronoiGaussField
	dev = torch.device('cuda:0')
	t0 = time.time()
	sc = scenes.make_scene(3, scale=args.scale, log=log)
	model = VoronoiGaussField.from_scene(sc, dev)
	g = model.graph
	cam = sc.cameras[0]
	o_np, d_np = cam.rays()
	o, d = torch.from_numpy(o_np).to(dev), torch.from_numpy(d_np).to(dev)
	from vgr.sites import nearest_sites
	eye = torch.tensor(cam.eye, dtype=torch.float32, device=dev)[None]
	start = nearest_sites(g.points, eye).expand(len(o)).contiguous()
	B, S = len(o), 64
	bounds = render.ray_bounds(o, d, 0.02, sc.far_radius)
	s_grid = (torch.linspace(0, 1, S + 1, device=dev)[:-1] + 0.5 / S).expand(B, S).contiguous()
	t = render.s_to_t(s_grid, *bounds).contiguous()
	fx = ext.extension()
	sh = model.sh().contiguous()
	stream = torch.cuda.current_stream(dev)
	log(f'config 3 frame: {B} rays x {S} samples, {sc.n_sites} sites ({time.time() - t0:.0f} s)')
	walk_ms, (site, steps), _ = time_steps(lambda: fx.walk(g.points, g.offsets, g.adj, o, d, t, start), args.steps,
										   args.warmup, stream)
	x = (o[:, None] + d[:, None] * t[..., None]).reshape(-1, 3).contiguous()
	site_f = site.reshape(-1).contiguous()
	dens_ms, sigma, _ = time_steps(lambda: fx.density_forward(g.points, g.offsets, g.adj, model.raw, model.d_log_scale,
															  model.d_quat, x, site_f, 1.0), args.steps, args.warmup,
								   stream)
	w, _ = render.composite(sigma.view(B, S), t, bounds[2])
	active = (w.reshape(-1) > 1e-4).nonzero().squeeze(1)
	xa = x[active].contiguous()
	da = d[:, None].expand(B, S, 3).reshape(-1, 3)[active].contiguous()
	sa = site_f[active].contiguous()
	col_ms, rgb, _ = time_steps(lambda: fx.color_forward(g.points, g.offsets, g.adj, model.c_log_scale, model.c_quat,
														 sh, sc.sh_deg, xa, da, sa), args.steps, args.warmup, stream)
	con_ms, _, _ = time_steps(lambda: fx.conic_forward(model.d_log_scale, model.d_quat, 0.0), args.steps, args.warmup,
							  stream)
	ms = {k: float(np.mean(v)) for k, v in (('walk', walk_ms), ('density', dens_ms), ('color', col_ms),
											('conic', con_ms))}
	m, ma = B * S, len(active)
	E = 1.0 + len(sc.adj) / sc.n_sites
	SHB = 12 * (sc.sh_deg + 1) ** 2
	nb = {'walk': float((m + steps.double().sum()) * (8 + 16 * E) + 8 * m), 'density': m * (28 + 48 * E),
		  'color': ma * (48 + E * (44 + SHB)), 'conic': sc.n_sites * 60.0}
	gbs = {k: nb[k] / (ms[k] * 1e-3) / 1e9 for k in ms}
	log('  '.join(f'{k} {ms[k]:.3f} ms ({gbs[k]:.0f} GB/s)' for k in ms) + f'; active samples {ma} of {m}')
	top = max(('walk', 'density', 'color'), key=lambda k: ms[k])
	cpu = None
	if args.cpu_seconds > 0:
		sys.path.insert(0, os.path.join(ROOT, 'oracle'))
		import oracle
		host = {k: v.cpu().numpy() for k, v in (('p', g.points), ('off', g.offsets), ('adj', g.adj), ('raw', model.raw),
												('dls', model.d_log_scale), ('dq', model.d_quat),
												('cls', model.c_log_scale), ('cq', model.c_quat), ('sh', sh))}
		# bounded samples, about args.cpu_seconds of host time in all at the measured oracle rates
		k_w = max(1, int(round(5.0 / max(args.cpu_seconds, 1e-3))))
		rays = np.arange(0, B, k_w)
		t1 = time.perf_counter()
		ws = oracle.walk(host['p'], host['off'], host['adj'], o_np[rays], d_np[rays], t.cpu().numpy()[rays],
						 start.cpu().numpy()[rays])
		t_walk = time.perf_counter() - t1
		walk_ok = bool((ws[0] == site.cpu().numpy()[rays]).all())
		x_np, s_np = x.cpu().numpy(), site_f.cpu().numpy()
		samp = np.arange(0, m, max(1, int(round(30.0 / max(args.cpu_seconds, 1e-3)))))
		t1 = time.perf_counter()
		sg = oracle.density(host['p'], host['off'], host['adj'], host['raw'], host['dls'], host['dq'], x_np[samp],
							s_np[samp])
		t_dens = time.perf_counter() - t1
		err_s = float(np.abs(sg - sigma.cpu().numpy()[samp]).max() / max(1.0, float(np.abs(sg).max())))
		ca = np.arange(0, ma, max(1, int(round(30.0 / max(args.cpu_seconds, 1e-3)))))
		t1 = time.perf_counter()
		cg = oracle.color(host['p'], host['off'], host['adj'], host['cls'], host['cq'], host['sh'], sc.sh_deg,
						  xa.cpu().numpy()[ca], da.cpu().numpy()[ca], sa.cpu().numpy()[ca])
		t_col = time.perf_counter() - t1
		err_c = float(np.abs(cg - rgb.cpu().numpy()[ca]).max())
		# host seconds for the whole frame, each operator's sample rate scaled to its full count
		t_frame = t_walk * m / (len(rays) * S) + t_dens * m / len(samp) + t_col * ma / len(ca)
		log(f'cpu oracle ({oracle.max_threads()} threads): walk {len(rays)} rays x {S} in {t_walk:.2f} s (sites equal: '
			f'{walk_ok}), density {len(samp)} samples in {t_dens:.2f} s (max rel err {err_s:.2e}), colour {len(ca)} '
			f'samples in {t_col:.2f} s (max abs err {err_c:.2e}); {t_frame:.1f} s per frame')
		cpu = {'value': round(m / t_frame / 1e6, 4),
			   'unit': 'Msamples/s', 'cores': oracle.max_threads(), 'kind': 'port',
			   'sample': f'walk: every {k_w}th ray ({len(rays)} x {S} samples); density: {len(samp)} samples; colour: '
						 f'{len(ca)} active samples; each rate scaled to the full frame',
			   'parity_walk_sites_equal': walk_ok, 'parity_density_max_rel': err_s, 'parity_color_max_abs': err_c}
	total = ms['walk'] + ms['density'] + ms['color']
	emit('Msamples/s NeRF-path field operators walk + density + colour (config 3, 1080p, 64 samples/ray) on 1 MI355X',
		 m / total / 1e3, 'Msamples/s', args, total,
		 {'workload': f'config 3, camera 0: {B} rays x {S} stratified samples ({m}), colour at the {ma} samples of '
					  f'weight > 1e-4; conic over {sc.n_sites} sites', 'samples': m, 'active_samples': ma,
		  'ms': {k: round(v, 3) for k, v in ms.items()}, 'GBps': {k: round(v, 1) for k, v in gbs.items()},
		  'walk_steps_per_sample': round(float(steps.double().sum()) / m, 3)},
		 hbm_roofline(ms[top], f'config3-field-{top}', source_hash('field.hip'), nb[top],
					  'cache-oblivious bytes per sample and neighbour (site record, adjacency, SH when coloured)',
					  f'{top}_forward' if top != 'walk' else 'walk'), cpu)


def bench_grad(args):
	"""Backward of the NeRF-path field operators for one training step on config 3: --batch random rays (train.py's
	default 4096, drawn uniformly over the pixels of the 4 cameras as scene.random_rays does, train.py:132) x 64
	stratified samples: density_backward at every sample, color_backward at the samples of compositing weight
	> 1e-4 (upstream gradients random normal, as the loss supplies them), conic_backward over all sites.
	value = samples per second through density + colour backward. CPU baseline: the C oracle's backward on one
	thread over a bounded sample.

	Algorithmic bytes (cache-oblivious; E = mean self-inclusive neighbourhood, SHB = 192 B at SH degree 3):
	  density  per sample 32 + 80 E       (x, site, dL/dsigma, offsets; per neighbour point 12 + adj 4 + raw 4 +
	                                        log_scale 12 + quat 16, and the gradients raw 4 + log_scale 12 + quat 16)
	  colour   per active sample 60 + E (3 x 44 + SHB + 28 + SHB)   (x, dir, site, rgb, dL/drgb, offsets; three
	                                        sweeps of point, adj, log_scale, quat; SH read, gradients of log_scale,
	                                        quat and SH written)
	  conic    per site 76 (log_scale 12 + quat 16 + dL/dA 24 in, gradients 28 out)."""
	import numpy as np
	import torch

	from vgr import ext, render, scenes
	from vgr.model import VoronoiGaussField
	from vgr.sites import nearest_sites
	dev = torch.device('cuda:0')
	sc = scenes.make_scene(3, scale=args.scale, log=log)
	model = VoronoiGaussField.from_scene(sc, dev)
	g = model.graph
	rng = np.random.default_rng(0)
	cams = rng.integers(0, len(sc.cameras), args.batch)
	o_l, d_l, e_l = [], [], []
	for c in range(len(sc.cameras)):
		n_c = int((cams == c).sum())
		o_c, d_c = sc.cameras[c].rays()
		pick = rng.choice(len(o_c), n_c, replace=False)
		o_l.append(o_c[pick]), d_l.append(d_c[pick]), e_l.append(np.repeat(sc.cameras[c].eye[None], n_c, 0))
	o = torch.from_numpy(np.concatenate(o_l)).to(dev)
	d = torch.from_numpy(np.concatenate(d_l)).to(dev)
	start = nearest_sites(g.points, torch.from_numpy(np.concatenate(e_l).astype(np.float32)).to(dev))
	B, S = len(o), 64
	bounds = render.ray_bounds(o, d, 0.02, sc.far_radius)
	s_grid = (torch.linspace(0, 1, S + 1, device=dev)[:-1] + 0.5 / S).expand(B, S).contiguous()
	t = render.s_to_t(s_grid, *bounds).contiguous()
	fx = ext.extension()
	sh = model.sh().contiguous()
	site, _ = fx.walk(g.points, g.offsets, g.adj, o, d, t, start.contiguous())
	x = (o[:, None] + d[:, None] * t[..., None]).reshape(-1, 3).contiguous()
	site_f = site.reshape(-1).contiguous()
	sigma = fx.density_forward(g.points, g.offsets, g.adj, model.raw, model.d_log_scale, model.d_quat, x, site_f, 1.0)
	w, _ = render.composite(sigma.view(B, S), t, bounds[2])
	active = (w.reshape(-1) > 1e-4).nonzero().squeeze(1)
	xa = x[active].contiguous()
	da = d[:, None].expand(B, S, 3).reshape(-1, 3)[active].contiguous()
	sa = site_f[active].contiguous()
	rgb = fx.color_forward(g.points, g.offsets, g.adj, model.c_log_scale, model.c_quat, sh, sc.sh_deg, xa, da, sa)
	gen = torch.Generator(device=dev).manual_seed(0)
	m, ma = B * S, len(active)
	g_sigma = torch.randn(m, device=dev, generator=gen)
	g_rgb = torch.randn(ma, 3, device=dev, generator=gen)
	gA = torch.randn(sc.n_sites, 6, device=dev, generator=gen)
	stream = torch.cuda.current_stream(dev)
	log(f'config 3 training batch: {B} random rays x {S} samples, {ma} active, {sc.n_sites} sites')
	dens_ms, dgrad, _ = time_steps(lambda: fx.density_backward(g.points, g.offsets, g.adj, model.raw,
															   model.d_log_scale, model.d_quat, x, site_f, g_sigma),
								   args.steps, args.warmup, stream)
	col_ms, cgrad, _ = time_steps(lambda: fx.color_backward(g.points, g.offsets, g.adj, model.c_log_scale,
															model.c_quat, sh, sc.sh_deg, xa, da, sa, rgb, g_rgb),
								  args.steps, args.warmup, stream)
	con_ms, _, _ = time_steps(lambda: fx.conic_backward(model.d_log_scale, model.d_quat, 0.0, gA), args.steps,
							  args.warmup, stream)
	ms = {k: float(np.mean(v)) for k, v in (('density', dens_ms), ('color', col_ms), ('conic', con_ms))}
	E = 1.0 + len(sc.adj) / sc.n_sites
	SHB = 12 * (sc.sh_deg + 1) ** 2
	nb = {'density': m * (32 + 80 * E), 'color': ma * (60 + E * (3 * 44 + 2 * SHB + 28)), 'conic': sc.n_sites * 76.0}
	gbs = {k: nb[k] / (ms[k] * 1e-3) / 1e9 for k in ms}
	log('  '.join(f'{k} backward {ms[k]:.3f} ms ({gbs[k]:.0f} GB/s)' for k in ms))
	top = max(('density', 'color'), key=lambda k: ms[k])
	cpu = None
	if args.cpu_seconds > 0:
		sys.path.insert(0, os.path.join(ROOT, 'oracle'))
		import oracle
		host = {k: v.detach().cpu().numpy() for k, v in (('p', g.points), ('off', g.offsets), ('adj', g.adj),
														  ('raw', model.raw), ('dls', model.d_log_scale),
														  ('dq', model.d_quat), ('cls', model.c_log_scale),
														  ('cq', model.c_quat), ('sh', sh))}
		# bounded samples; the oracle's gradients are sums over the sampled subset only, so they are timed here
		# and checked against the GPU in tests/test_gpu_field_grad.py
		ks = max(1, int(m / (4000.0 * max(args.cpu_seconds, 1e-3))))
		samp = np.arange(0, m, ks)
		t1 = time.perf_counter()
		oracle.density_backward(host['p'], host['off'], host['adj'], host['raw'], host['dls'], host['dq'],
								x.cpu().numpy()[samp], site_f.cpu().numpy()[samp], g_sigma.cpu().numpy()[samp])
		t_dens = time.perf_counter() - t1
		ca = np.arange(0, ma, max(1, int(ma / (700.0 * max(args.cpu_seconds, 1e-3)))))
		t1 = time.perf_counter()
		oracle.color_backward(host['p'], host['off'], host['adj'], host['cls'], host['cq'], host['sh'], sc.sh_deg,
							  xa.cpu().numpy()[ca], da.cpu().numpy()[ca], sa.cpu().numpy()[ca], rgb.cpu().numpy()[ca],
							  g_rgb.cpu().numpy()[ca])
		t_col = time.perf_counter() - t1
		t_frame = t_dens * m / len(samp) + t_col * ma / len(ca)
		log(f'cpu oracle (1 thread): density backward {len(samp)} samples in {t_dens:.2f} s, colour backward '
			f'{len(ca)} samples in {t_col:.2f} s; {t_frame:.1f} s per batch')
		cpu = {'value': round(m / t_frame / 1e6, 4), 'unit': 'Msamples/s', 'cores': 1, 'kind': 'port',
			   'sample': f'density backward: every {ks}th sample ({len(samp)}); colour backward: {len(ca)} active '
						 f'samples; each rate scaled to the whole batch'}
	total = ms['density'] + ms['color']
	emit(f'Msamples/s NeRF-path field backward density + colour (config 3, training batch of {B} random rays x {S} '
		 f'samples) on 1 MI355X', m / total / 1e3, 'Msamples/s', args, total,
		 {'workload': f'config 3: {B} random rays of the 4 cameras x {S} stratified samples ({m}); colour backward '
					  f'at the {ma} samples of weight > 1e-4; conic backward over {sc.n_sites} sites', 'samples': m,
		  'active_samples': ma, 'ms': {k: round(v, 3) for k, v in ms.items()},
		  'GBps': {k: round(v, 1) for k, v in gbs.items()},
		  'grad_norms': {'raw': float(dgrad[0].norm()), 'sh': float(cgrad[2].norm())}},
		 hbm_roofline(ms[top], f'config3-grad-{top}', source_hash('field_grad.hip'), nb[top],
					  'cache-oblivious bytes per sample and neighbour (site parameters, gradient scatter)',
					  f'{top}_backward'), cpu)


if __name__ == '__main__':
	main()
