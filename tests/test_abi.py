"""The C-ABI library: it loads without a GPU, exports every entry point include/vgr.h declares, and the Python
binding declares each with the header's parameter count. No compute call is made here."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'vgr.h')


def declared():
	"""{name: parameter count} of every function declared in include/vgr.h."""
	text = open(HEADER).read()
	text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
	out = {}
	for m in re.finditer(r'\b(?:int|int64_t|const char\*)\s+(vgr_\w+)\s*\(([^)]*)\)\s*;', text):
		params = m.group(2).strip()
		out[m.group(1)] = 0 if params in ('', 'void') else params.count(',') + 1
	return out


def test_header_declares_the_entry_points():
	names = declared()
	for n in ('vgr_foam_infer', 'vgr_foam_infer_traced', 'vgr_foam_infer_lanes', 'vgr_foam_traverse_faces',
			  'vgr_march_forward', 'vgr_march_work_size', 'vgr_march_backward', 'vgr_march_backward_work_size',
			  'vgr_march_forward_lanes', 'vgr_foam_work_size', 'vgr_foam_forward', 'vgr_foam_backward',
			  'vgr_walk', 'vgr_density_forward', 'vgr_color_forward', 'vgr_field_work_size', 'vgr_conic_forward', 'vgr_density_backward', 'vgr_density_backward_work_size',
			  'vgr_color_backward', 'vgr_color_backward_work_size', 'vgr_conic_backward', 'vgr_pack_work_size',
			  'vgr_pack_foam', 'vgr_morton_work_size', 'vgr_morton_codes', 'vgr_bake_colors', 'vgr_grid_work_size',
			  'vgr_grid_build', 'vgr_grid_nearest', 'vgr_ray_order_work_size', 'vgr_ray_order', 'vgr_last_error',
			  'vgr_abi_version', 'vgr_foam_index_pack', 'vgr_foam_infer_indexed', 'vgr_grid_build_noalloc',
			  'vgr_foam_slot_table', 'vgr_grid_cell_points', 'vgr_grid_nearest_points'):
		assert n in names


def test_library_exports_every_declared_symbol():
	from vgr import _lib
	if not os.path.exists(_lib.LIB_PATH):
		pytest.fail('libvgr.so is not built (run __graft_entry__.build())')
	lib = ctypes.CDLL(_lib.LIB_PATH)
	for name, nparams in declared().items():
		assert hasattr(lib, name), f'{name} not exported'
		assert len(_lib.SIGNATURES[name]) == nparams, f'{name}: binding has {len(_lib.SIGNATURES[name])} args'


def test_library_reports_argument_errors_without_a_gpu():
	"""Argument validation runs on the host before any HIP call."""
	from vgr import _lib
	lib = _lib.load()
	assert lib.vgr_abi_version() == _lib.ABI_VERSION
	rc = lib.vgr_conic_forward(None, None, -1, 0.0, None, None)
	assert rc == 1 and b'n must be >= 0' in lib.vgr_last_error()
	rc = lib.vgr_conic_forward(None, None, 0, 0.0, None, None)  # empty: nothing to launch
	assert rc == 0
	args = [None, 10, None, None, None, 10, None, None, 0, 3, None, None, None, None, None, 5, 1e-4, 1e-4, 1e30, 7, 2,
			None, None, None, None, None, None, None]
	assert lib.vgr_foam_infer(*args) == 1 and b'color_mode' in lib.vgr_last_error()
	args[19], args[20] = 0, 9
	assert lib.vgr_foam_infer(*args) == 1 and b'stage' in lib.vgr_last_error()
	args[20] = 2
	assert lib.vgr_foam_infer(*args) == 1 and b'null scene pointer' in lib.vgr_last_error()
	with pytest.raises(RuntimeError, match='trace'):
		_lib.call('vgr_foam_infer_traced', *args[:-1], None, 0, None)
	# grid: geometry is validated before any launch; the work size is a closed form
	f3, i3 = (ctypes.c_float * 3), (ctypes.c_int32 * 3)
	assert lib.vgr_grid_work_size(100, 5000) == 100 + 5000 + 2 + 1
	rc = lib.vgr_grid_nearest(None, 1, 3, f3(0, 0, 0), f3(1, 1, 1), i3(0, 1, 1), None, None, None, 5, None, None)
	assert rc == 1 and b'res[0]' in lib.vgr_last_error()
	rc = lib.vgr_grid_build(None, 1, 3, f3(0, 0, 0), f3(1, 1, -1), i3(1, 1, 1), None, None, None, None)
	assert rc == 1 and b'cell edge 2' in lib.vgr_last_error()
	assert lib.vgr_grid_nearest(None, 1, 3, f3(0, 0, 0), f3(1, 1, 1), i3(1, 1, 1), None, None, None, 0, None, None) == 0
	# the cell-ordered copy and the queries over it: sizes, pointers and alignment checked on the host
	assert lib.vgr_grid_cell_points(None, -1, 3, None, None, None) == 1 and b'n_sites' in lib.vgr_last_error()
	assert lib.vgr_grid_cell_points(None, 10, 2, None, None, None) == 1 and b'stride' in lib.vgr_last_error()
	assert lib.vgr_grid_cell_points(None, 10, 3, None, None, None) == 1 and b'null pointer' in lib.vgr_last_error()
	fake = ctypes.c_void_p(1 << 20)
	rc = lib.vgr_grid_cell_points(fake, 10, 3, fake, ctypes.c_void_p((1 << 20) + 8), None)
	assert rc == 1 and b'16-byte aligned' in lib.vgr_last_error()
	assert lib.vgr_grid_cell_points(None, 0, 3, None, None, None) == 0
	rc = lib.vgr_grid_nearest_points(None, 1, f3(0, 0, 0), f3(1, 1, 1), i3(0, 1, 1), None, None, 5, None, None, None)
	assert rc == 1 and b'res[0]' in lib.vgr_last_error()
	rc = lib.vgr_grid_nearest_points(None, 1, f3(0, 0, 0), f3(1, 1, 1), i3(1, 1, 1), None, None, 5, None, None, None)
	assert rc == 1 and b'null pointer' in lib.vgr_last_error()
	assert lib.vgr_grid_nearest_points(None, 1, f3(0, 0, 0), f3(1, 1, 1), i3(1, 1, 1), None, None, 0, None, None,
									   None) == 0
	# march: one line-aligned block per site in the caller's work buffer (record + SH: 128 B up to sh_deg 1, else
	# 256 B), checked before the pack launch
	assert lib.vgr_march_work_size(0, 3) == 0 and lib.vgr_march_work_size(1000, 4) == 0
	assert [lib.vgr_march_work_size(1000, g) for g in range(4)] == [128000, 128000, 256000, 256000]
	fake = ctypes.c_void_p(1 << 20)
	margs = [fake, 1000, fake, fake, 15000, fake, fake, fake, fake, 3, fake, fake, fake, fake, fake, fake, 8, 0.01, 64,
			 1e-4, 1e-4, fake, fake, fake, fake, None, 0, None, 0, None]
	assert lib.vgr_march_forward(*margs) == 1 and b'work must hold 256000 bytes' in lib.vgr_last_error()
	margs[27], margs[28] = ctypes.c_void_p((1 << 20) + 128), 256000
	assert lib.vgr_march_forward(*margs) == 1 and b'256-byte aligned' in lib.vgr_last_error()
	margs[16] = 0  # no rays: nothing to check or launch
	assert lib.vgr_march_forward(*margs) == 0
	# the layout argument and the training entries' workspaces are checked before any launch
	margs[16] = 8
	largs = margs[:27] + [None, 8] + margs[27:]
	assert lib.vgr_march_forward_lanes(*largs) == 1 and b'lanes_per_ray' in lib.vgr_last_error()
	assert lib.vgr_march_backward_work_size(1000, 3) == 256000 + 256000
	assert lib.vgr_foam_work_size(1000, 1) == 128000 + 256000
	fargs = [fake, 1000, fake, fake, 15000, fake, fake, fake, fake, 3, fake, fake, fake, fake, fake, 8, 1e-4, 1e-4,
			 fake, fake, fake, fake, None, 0, fake, 1000, None]
	assert lib.vgr_foam_forward(*fargs) == 1 and b'work must hold 512000 bytes' in lib.vgr_last_error()
	fargs[9] = 5
	assert lib.vgr_foam_forward(*fargs) == 1 and b'sh_deg' in lib.vgr_last_error()
	# field records: 64 bytes per site
	assert lib.vgr_field_work_size(0) == 0 and lib.vgr_field_work_size(1000) == 64000


def test_indexed_records_arguments_without_a_gpu():
	"""vgr_foam_index_pack and vgr_foam_infer_indexed validate their sizes and record pointers on the host; an empty
	pack launches nothing."""
	from vgr import _lib
	lib = _lib.load()
	pack = lambda n, e: lib.vgr_foam_index_pack(None, None, None, None, n, e, None, None, None)  # noqa: E731
	assert pack(-1, 0) == 1 and b'n_sites' in lib.vgr_last_error()
	assert pack(10, 5) == 1 and b'n_edges' in lib.vgr_last_error()
	assert pack(10, 20) == 1 and b'null pointer' in lib.vgr_last_error()
	assert pack(0, 0) == 0
	args = [None, 10, None, None, None, 10, None, None, 0, 3, None, None, None, None, None, 5, 1e-4, 1e-4, 1e30, 2, 2,
			None, None, None, None, None, None, None, 0, None, 0, None, None, None, None, 16, None]
	assert lib.vgr_foam_infer_indexed(*args) == 1 and b'edge_i and attr_i' in lib.vgr_last_error()
	args[27], args[28] = 1, 0  # a trace sink without a capacity
	assert lib.vgr_foam_infer_indexed(*args) == 1 and b'trace_cap' in lib.vgr_last_error()
	# site blocks (row_floats 64) must sit on 256-byte boundaries, 64-byte rows on 64-byte ones
	args[27], args[28] = None, 0
	args[31], args[32], args[34], args[35] = 4096, 8192, 64, 64
	assert lib.vgr_foam_infer_indexed(*args) == 1 and b'256-byte aligned' in lib.vgr_last_error()
	args[34], args[35] = 64 + 32, 16
	assert lib.vgr_foam_infer_indexed(*args) == 1 and b'64-byte aligned' in lib.vgr_last_error()


def test_slot_table_arguments_without_a_gpu():
	"""vgr_foam_slot_table validates its sizes, pointers and the table's alignment on the host; an empty pack
	launches nothing."""
	from vgr import _lib
	lib = _lib.load()
	assert lib.vgr_foam_slot_table(None, None, -1, 0, None, None) == 1 and b'n_sites' in lib.vgr_last_error()
	assert lib.vgr_foam_slot_table(None, None, 10, 5, None, None) == 1 and b'n_edges' in lib.vgr_last_error()
	assert lib.vgr_foam_slot_table(None, None, 10, 20, None, None) == 1 and b'null pointer' in lib.vgr_last_error()
	assert lib.vgr_foam_slot_table(8, 8, 10, 20, 4, None) == 1 and b'aligned' in lib.vgr_last_error()
	assert lib.vgr_foam_slot_table(None, None, 0, 0, None, None) == 0


def test_ray_order_arguments_without_a_gpu():
	"""vgr_ray_order validates its bin and key-width arguments on the host; an empty batch launches nothing."""
	from vgr import _lib
	lib = _lib.load()
	assert lib.vgr_ray_order(None, None, 10, 0, 7, None, None, 0, None) == 1 and b'dir_res' in lib.vgr_last_error()
	assert lib.vgr_ray_order(None, None, 10, 8, 11, None, None, 0, None) == 1 and b'pos_bits' in lib.vgr_last_error()
	assert lib.vgr_ray_order(None, None, 10, 64, 7, None, None, 0, None) == 1 and b'key bits' in lib.vgr_last_error()
	assert lib.vgr_ray_order(None, None, 0, 8, 7, None, None, 0, None) == 0
	assert lib.vgr_ray_order_work_size(0) == 0 and lib.vgr_ray_order_work_size(1000) >= 3 * 4000
