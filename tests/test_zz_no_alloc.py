"""vgr_grid_build_noalloc (the start-cell grid built in the library's static device scratch, for callers that cannot
allocate) against vgr_grid_build with a caller-given workspace, through the C ABI: identical cell ranges, the same
sites in every cell (the order inside a cell is arbitrary in both) and identical nearest-site answers; two calls in
a row, the second on fewer sites (the scratch keeps the first call's contents), and a build too large for the
scratch rejected with an error."""

import ctypes

import numpy as np
import pytest
import torch

import dense
from vgr import _lib

pytestmark = pytest.mark.gpu


def geometry(pts, per_cell=2.0):
	lo = pts.min(0).astype(np.float64)
	hi = pts.max(0).astype(np.float64)
	ext = np.maximum(hi - lo, 1e-6)
	lo = lo - 1e-6 * ext
	ext = ext * (1 + 2e-6)
	edge = (ext.prod() * per_cell / len(pts)) ** (1 / 3)
	res = [int(min(max(np.ceil(e / edge), 1), 1024)) for e in ext]
	cell = [float(e) / r for e, r in zip(ext, res)]
	return (ctypes.c_float * 3)(*lo), (ctypes.c_float * 3)(*cell), (ctypes.c_int32 * 3)(*res), int(np.prod(res))


def build(dev, pts_t, geom, noalloc):
	lib = _lib.load()
	lo, cell, res, n_cells = geom
	n = pts_t.shape[0]
	cell_start = torch.full((n_cells + 1,), -7, dtype=torch.int32, device=dev)
	cell_sites = torch.full((n,), -7, dtype=torch.int32, device=dev)
	stream = _lib.stream_of(dev)
	if noalloc:
		rc = lib.vgr_grid_build_noalloc(_lib.ptr(pts_t), n, 3, lo, cell, res, _lib.ptr(cell_start),
										_lib.ptr(cell_sites), stream)
	else:
		work = torch.empty(int(lib.vgr_grid_work_size(n, n_cells)), dtype=torch.int32, device=dev)
		rc = lib.vgr_grid_build(_lib.ptr(pts_t), n, 3, lo, cell, res, _lib.ptr(cell_start), _lib.ptr(cell_sites),
								_lib.ptr(work), stream)
	assert rc == 0, lib.vgr_last_error()
	torch.cuda.synchronize()
	return cell_start, cell_sites


def nearest(dev, pts_t, geom, grid, q):
	lib = _lib.load()
	lo, cell, res, _ = geom
	qt = torch.as_tensor(q, device=dev)
	out = torch.empty(len(q), dtype=torch.int32, device=dev)
	rc = lib.vgr_grid_nearest(_lib.ptr(pts_t), pts_t.shape[0], 3, lo, cell, res, _lib.ptr(grid[0]), _lib.ptr(grid[1]),
							  _lib.ptr(qt), len(q), _lib.ptr(out), _lib.stream_of(dev))
	assert rc == 0, lib.vgr_last_error()
	torch.cuda.synchronize()
	return out.cpu().numpy()


def test_noalloc_grid_matches_workspace_build(gpu):
	rng = np.random.default_rng(21)
	for n in (300000, 40000):  # the second call is smaller: stale counters of the first must not leak into it
		pts = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
		pts_t = torch.as_tensor(pts, device=gpu)
		geom = geometry(pts)
		print(f'[no-alloc grid] {n} sites, {geom[3]} cells', flush=True)
		ref = build(gpu, pts_t, geom, noalloc=False)
		got = build(gpu, pts_t, geom, noalloc=True)
		cs_ref, cs_got = ref[0].cpu().numpy(), got[0].cpu().numpy()
		np.testing.assert_array_equal(cs_got, cs_ref)
		assert cs_got[0] == 0 and cs_got[-1] == n
		s_ref, s_got = ref[1].cpu().numpy(), got[1].cpu().numpy()
		cell_of = np.repeat(np.arange(len(cs_ref) - 1), np.diff(cs_ref))
		np.testing.assert_array_equal(s_got[np.lexsort((s_got, cell_of))], s_ref[np.lexsort((s_ref, cell_of))])
		q = np.concatenate([rng.uniform(-1, 1, (20000, 3)), rng.uniform(-1.5, 1.5, (5000, 3))]).astype(np.float32)
		a, b = nearest(gpu, pts_t, geom, ref, q), nearest(gpu, pts_t, geom, got, q)
		np.testing.assert_array_equal(b, a)
		np.testing.assert_array_equal(b[:2000], dense.nearest_brute(pts, q[:2000]))


def test_noalloc_grid_rejects_builds_beyond_its_scratch(gpu):
	lib = _lib.load()
	limit = 1 << 24
	n = limit  # N + G + tiles + 1 > 2^24 ints for any grid
	lo = (ctypes.c_float * 3)(-1, -1, -1)
	cell = (ctypes.c_float * 3)(0.01, 0.01, 0.01)
	res = (ctypes.c_int32 * 3)(200, 200, 200)
	rc = lib.vgr_grid_build_noalloc(None, n, 3, lo, cell, res, None, None, _lib.stream_of(gpu))
	assert rc != 0 and b'beyond the static' in lib.vgr_last_error()


def test_noalloc_grid_allocates_nothing_and_replays_in_a_graph(gpu):
	"""After one warm call on the device (which looks up the scratch array's address), repeated calls leave the
	device's free memory unchanged; and a call captured in a HIP graph (torch.cuda.graph), replayed three times with
	eager work between the replays, gives the workspace build's cells every time."""
	lib = _lib.load()
	rng = np.random.default_rng(22)
	n = 100000
	pts = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
	pts_t = torch.as_tensor(pts, device=gpu)
	geom = geometry(pts)
	lo, cell, res, n_cells = geom
	ref = build(gpu, pts_t, geom, noalloc=False)
	cs_ref, s_ref = ref[0].cpu().numpy(), ref[1].cpu().numpy()
	cell_of = np.repeat(np.arange(len(cs_ref) - 1), np.diff(cs_ref))
	sorted_ref = s_ref[np.lexsort((s_ref, cell_of))]
	cs = torch.full((n_cells + 1,), -7, dtype=torch.int32, device=gpu)
	sites = torch.full((n,), -7, dtype=torch.int32, device=gpu)

	def call():
		return lib.vgr_grid_build_noalloc(_lib.ptr(pts_t), n, 3, lo, cell, res, _lib.ptr(cs), _lib.ptr(sites),
										  _lib.stream_of(gpu))

	assert call() == 0, lib.vgr_last_error()  # the warm call
	torch.cuda.synchronize()
	free0 = torch.cuda.mem_get_info(gpu)[0]
	for _ in range(3):
		assert call() == 0, lib.vgr_last_error()
	torch.cuda.synchronize()
	assert torch.cuda.mem_get_info(gpu)[0] == free0
	np.testing.assert_array_equal(cs.cpu().numpy(), cs_ref)

	graph = torch.cuda.CUDAGraph()
	with torch.cuda.graph(graph):
		rc = call()
	assert rc == 0, lib.vgr_last_error()
	for rep in range(3):
		cs.fill_(-7)
		sites.fill_(-7)
		torch.cuda.synchronize()
		graph.replay()
		torch.cuda.synchronize()
		got_cs, got_s = cs.cpu().numpy(), sites.cpu().numpy()
		print(f'[no-alloc grid] graph replay {rep}', flush=True)
		np.testing.assert_array_equal(got_cs, cs_ref)
		np.testing.assert_array_equal(got_s[np.lexsort((got_s, cell_of))], sorted_ref)
