"""Benchmark of the north-star path: foam_infer (ray / Voronoi-face renderer) on BASELINE config 3 -- the 2M-site
surface-dominated scene seen by 4 cameras at 1920x1080 -- on one MI355X.

One step = one foam_infer launch rendering all 4 frames (8,294,400 rays) with the scene packed and the rays
resident in HBM. Prints one JSON line: Mrays/s (value), ms per step, FPS at 1080p, the roofline of the kernel
(algorithmic bytes per launch from the kernel's own per-ray counters / the launch time measured with HIP events
on the launch stream) and the CPU oracle timed on the host on a bounded, deterministic subset of the same rays.

  python bench.py [--steps K] [--warmup W] [--colors exact|fused] [--no-reorder] [--cpu-seconds S]
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
TRAFFIC_FILE = os.path.join(ROOT, 'profiles', 'foam_infer_config3_pmc.md')


def log(*a):
	print('[bench]', *a, file=sys.stderr, flush=True)


def measured_traffic(workload):
	"""DRAM bytes per launch of this workload from the committed rocprofv3 PMC summary (a line
	'traffic_bytes_per_launch: <bytes> workload: <key>'), or None when no summary matches."""
	import re
	if not os.path.exists(TRAFFIC_FILE):
		return None
	for line in open(TRAFFIC_FILE):
		m = re.match(r'\s*traffic_bytes_per_launch:\s*([0-9.eE+]+)\s+workload:\s*(\S+)', line)
		if m and m.group(2) == workload:
			return float(m.group(1))
	return None


def algorithmic_bytes(stats, sh_bytes, u_sh_per_ray):
	"""Cache-oblivious bytes of one launch from the per-ray counters (B, 5) = samples, coloured segments, walk
	steps, density terms, SH evaluations:
	  56 per ray (o, d, near, far, start in; rgb, T, depth out)
	  + 24 per sample (cell position 16 + offsets 8)
	  + 84 per neighbourhood edge = density term (edge record 16 + nbr 4 + density record 32 + colour-conic record 32)
	  + sh_bytes per distinct site whose colour the ray blends (u_sh_per_ray, measured on traced rays)."""
	s = stats.double()
	return float(56 * len(s) + 24 * s[:, 0].sum() + 84 * s[:, 3].sum() + sh_bytes * u_sh_per_ray * len(s))


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
	ap.add_argument('--steps', type=int, default=20)
	ap.add_argument('--warmup', type=int, default=3)
	ap.add_argument('--config', type=int, default=3)
	ap.add_argument('--scale', type=float, default=1.0, help='site-count scale (1 = the BASELINE config)')
	ap.add_argument('--colors', default='fused', choices=['exact', 'fused'],
				help='exact colour modes (eps_color = 0): lazy second pass or fused online blend')
	ap.add_argument('--no-reorder', action='store_true', help='keep the generator order of the sites')
	ap.add_argument('--tile', type=int, default=8, help='pixel tile edge (8: one 8x8 tile per wave64)')
	ap.add_argument('--cpu-seconds', type=float, default=15.0, help='target CPU-oracle time (0: skip)')
	ap.add_argument('--copy-probe', action='store_true', help='also run a 1 GiB device copy (PMC calibration)')
	args = ap.parse_args()
	if args.gpus != 1:
		print(f'bench.py renders on one GPU only (got --gpus {args.gpus}): rays are independent, so N GPUs would '
			  f'each render 1/N of the cameras with a replicated scene; multi-GPU runs are not part of this build.',
			  file=sys.stderr)
		sys.exit(2)

	import numpy as np
	import torch

	from vgr import ext, render, scenes
	from vgr.model import VoronoiGaussField

	dev = torch.device('cuda:0')
	t0 = time.time()
	sc = scenes.make_scene(args.config, scale=args.scale, log=log)
	log(f'scene config {args.config}: {sc.n_sites} sites, {len(sc.adj)} adjacency entries ({time.time() - t0:.0f} s)')
	model = VoronoiGaussField.from_scene(sc, dev)
	pack = render.pack_foam(model, reorder=not args.no_reorder)
	o_np, d_np, start_np, _ = sc.camera_rays(tile=args.tile)
	o, d = torch.from_numpy(o_np).to(dev), torch.from_numpy(d_np).to(dev)
	start = torch.from_numpy(start_np).to(dev)
	if pack['inv'] is not None:
		start = pack['inv'][start.long()].int()
	near, _, far = render.ray_bounds(o, d, 0.02, sc.far_radius)
	B = len(o)
	W, H = (sc.cameras[0].width, sc.cameras[0].height) if sc.cameras else (0, 0)
	frames = len(sc.cameras)
	mode = {'exact': 0, 'fused': 2}[args.colors]
	empty = torch.empty(0, dtype=torch.int32, device=dev)
	fi = ext.foam_infer_extension()
	call = lambda: fi.foam_infer(pack['points'], pack['offsets'], pack['nbr'], pack['edge'], pack['attr'],  # noqa
								 pack['sh'], sc.sh_deg, o, d, start, near, far, 1e-4, 1e-4, math.inf, mode, 2, empty,
								 pack['orig'])
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
	log(f'{args.steps} steps: mean {ms:.3f} ms, median {np.median(launch_ms):.3f} ms, wall {wall * 1e3 / args.steps:.3f} '
		f'ms/step')
	sh_bytes = 12 * (sc.sh_deg + 1) ** 2
	args_of = lambda sel: (pack['points'], pack['offsets'], pack['nbr'], pack['edge'], pack['attr'], pack['sh'],  # noqa
						   sc.sh_deg, o[sel], d[sel], start[sel], near[sel], far[sel], 1e-4, 1e-4, math.inf, mode, 2,
						   empty, pack['orig'])
	u_sh, u_rays = distinct_blended_sites(fi, pack, args_of, B, sc.sh_deg)
	log(f'distinct blended sites per ray: {u_sh:.1f} (over {u_rays} traced rays)')
	abytes = algorithmic_bytes(stats.cpu(), sh_bytes, u_sh)
	achieved = abytes / (ms * 1e-3) / 1e9
	st = stats.double()
	traffic = measured_traffic(f'config{args.config}-scale{args.scale}-{args.colors}-reorder{int(not args.no_reorder)}')

	cpu = None
	if args.cpu_seconds > 0:
		cpu = cpu_baseline(pack, sc, o_np, d_np, start.cpu().numpy(), near.cpu().numpy(), far.cpu().numpy(), mode,
						   args.cpu_seconds, rgb.cpu().numpy(), T.cpu().numpy())
	if args.copy_probe:
		src = torch.empty(1 << 28, dtype=torch.float32, device=dev)
		dst = torch.empty_like(src)
		dst.copy_(src)
		torch.cuda.synchronize()
		log('copy probe: 1 GiB read + 1 GiB written')

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
			'colors': args.colors, 'sh': 'f32', 'sh_deg': sc.sh_deg, 'morton_reorder': not args.no_reorder,
			'ray_order': f'{args.tile}x{args.tile} tiles', 't_thresh': 1e-4, 'w_thresh': 1e-4,
			'samples_per_ray': round(float(st[:, 0].mean()), 2),
			'density_terms_per_ray': round(float(st[:, 3].mean()), 1),
			'sh_evals_per_ray': round(float(st[:, 4].mean()), 1),
			'distinct_blended_sites_per_ray': round(u_sh, 1), 'distinct_sites_traced_rays': u_rays,
			'mean_T': round(float(T.double().mean()), 4),
		},
		'roofline': {
			'bound': 'hbm', 'achieved': round(achieved, 1), 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
			'frac': round(achieved / HBM_PEAK_GBS, 4), 'traffic': traffic,
			'algorithmic_bytes_per_launch': abytes,
			'dram_GBps': None if traffic is None else round(traffic / (ms * 1e-3) / 1e9, 1),
		},
		'cpu_baseline': cpu,
	}
	print(json.dumps(res), flush=True)


def cpu_baseline(pack, sc, o, d, start, near, far, mode, seconds, rgb_gpu, T_gpu):
	"""The CPU oracle (C/OpenMP, thread per ray) on every k-th ray of the same workload, k chosen so the timed
	loop takes about `seconds` on all host cores; also the max |rgb - GPU| on that subset."""
	import numpy as np

	sys.path.insert(0, os.path.join(ROOT, 'oracle'))
	import oracle
	pk = {k: pack[k].cpu().numpy() for k in ('points', 'offsets', 'nbr', 'edge', 'attr', 'sh', 'orig')}
	threads = oracle.max_threads()
	B = len(o)
	probe = np.arange(0, B, max(1, B // 20000), dtype=np.int64)
	r = oracle.foam_infer(pk, sc.sh_deg, o, d, start, near, far, color_mode=mode, rays=probe)
	rate = len(probe) / max(r['seconds'], 1e-6)
	k = max(1, int(B / (rate * seconds)))
	sel = np.arange(0, B, k, dtype=np.int64)
	r = oracle.foam_infer(pk, sc.sh_deg, o, d, start, near, far, color_mode=mode, rays=sel)
	err = float(np.abs(r['rgb'] - rgb_gpu[sel]).max())
	errT = float(np.abs(r['T'] - T_gpu[sel]).max())
	log(f'cpu oracle: {len(sel)} rays (every {k}th) in {r["seconds"]:.2f} s on {threads} threads; '
		f'max |rgb - gpu| {err:.2e}, max |T - gpu| {errT:.2e}')
	return {'value': round(len(sel) / r['seconds'] / 1e6, 4), 'unit': 'Mrays/s', 'cores': threads, 'kind': 'port',
			'sample': f'every {k}th ray of the same {B}-ray workload ({len(sel)} rays), exact colours, C/OpenMP '
					  f'thread per ray',
			'parity_max_abs_rgb': err, 'parity_max_abs_T': errT}


if __name__ == '__main__':
	main()
