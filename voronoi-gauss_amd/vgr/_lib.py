"""ctypes binding of libvgr.so (the C ABI declared in include/vgr.h).

torch is imported first so that libvgr.so binds to the HIP runtime torch already loaded (both carry the
soname libamdhip64.so.7): device pointers, streams and the current device are then shared with torch.
There is no fallback: a missing or unloadable library raises."""

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime libvgr.so links against)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'libvgr.so')

_P, _I32, _I64, _F64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_double

# argument types of every entry point of include/vgr.h, in declaration order
SIGNATURES = {
	'vgr_foam_infer': [_P, _I64, _P, _P, _P, _I64, _P, _P, _I32, _I64, _P, _P, _P, _P, _P, _I64, _F64, _F64, _F64,
					   _I64, _I64, _P, _P, _P, _P, _P, _P, _P],
	'vgr_foam_infer_traced': [_P, _I64, _P, _P, _P, _I64, _P, _P, _I32, _I64, _P, _P, _P, _P, _P, _I64, _F64, _F64,
							  _F64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _I64, _P],
	'vgr_foam_infer_lanes': [_P, _I64, _P, _P, _P, _I64, _P, _P, _I32, _I64, _P, _P, _P, _P, _P, _I64, _F64, _F64,
							 _F64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _P, _P],
	'vgr_march_forward': [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _I64, _F64, _I64,
						  _F64, _F64, _P, _P, _P, _P, _P, _I64, _P, _I64, _P],
	'vgr_march_work_size': [_I64, _I64],
	'vgr_march_backward_work_size': [_I64, _I64],
	'vgr_foam_work_size': [_I64, _I64],
	'vgr_foam_forward': [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _F64, _F64, _P, _P,
						 _P, _P, _P, _I64, _P, _I64, _P],
	'vgr_foam_backward': [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _F64, _F64, _P, _P,
						  _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _P, _I64, _P],
	'vgr_march_forward_lanes': [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _I64, _F64,
								_I64, _F64, _F64, _P, _P, _P, _P, _P, _I64, _P, _I64, _P, _I64, _P],
	'vgr_march_backward': [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _I64, _F64, _I64,
						   _F64, _F64, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _P, _I64, _P],
	'vgr_foam_traverse_faces': [_P, _I64, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _I64, _I64,
								_P],
	'vgr_walk': [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _I64, _I64, _P, _P, _P],
	'vgr_density_forward': [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _F64, _P, _P, _I64, _P],
	'vgr_color_forward': [_P, _I64, _P, _P, _I64, _P, _P, _P, _I64, _P, _P, _P, _I64, _P, _P, _I64, _P],
	'vgr_field_work_size': [_I64],
	'vgr_density_backward_work_size': [_I64, _I64],
	'vgr_density_backward': [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _P],
	'vgr_color_backward_work_size': [_I64, _I64],
	'vgr_color_backward': [_P, _I64, _P, _P, _I64, _P, _P, _P, _I64, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _I64,
						   _P],
	'vgr_conic_backward': [_P, _P, _I64, _F64, _P, _P, _P, _P],
	'vgr_pack_work_size': [_I64],
	'vgr_morton_work_size': [_I64],
	'vgr_morton_codes': [_P, _I64, _I32, _P, _P, _I64, _P],
	'vgr_bake_colors': [_P, _P, _I64, _I64, _F64, _F64, _F64, _P, _P],
	'vgr_pack_foam': [_P, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _F64, _F64, _P, _P, _P, _P, _P, _P, _P, _P,
					  _I64, _P],
	'vgr_conic_forward': [_P, _P, _I64, _F64, _P, _P],
	'vgr_grid_work_size': [_I64, _I64],
	'vgr_grid_build': [_P, _I64, _I32, _P, _P, _P, _P, _P, _P, _P],
	'vgr_ray_order_work_size': [_I64],
	'vgr_ray_order': [_P, _P, _I64, _I32, _I32, _P, _P, _I64, _P],
	'vgr_foam_index_pack': [_P, _P, _P, _P, _I64, _I64, _P, _P, _P],
	'vgr_foam_infer_indexed': [_P, _I64, _P, _P, _P, _I64, _P, _P, _I32, _I64, _P, _P, _P, _P, _P, _I64, _F64,
							   _F64, _F64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _P, _P, _P, _P, _I64,
							   _P],
	'vgr_foam_slot_table': [_P, _P, _I64, _I64, _P, _P],
	'vgr_grid_build_noalloc': [_P, _I64, _I32, _P, _P, _P, _P, _P, _P],
	'vgr_grid_nearest': [_P, _I64, _I32, _P, _P, _P, _P, _P, _P, _I64, _P, _P],
	'vgr_grid_cell_points': [_P, _I64, _I32, _P, _P, _P],
	'vgr_grid_nearest_points': [_P, _I64, _P, _P, _P, _P, _P, _I64, _P, _P, _P],
	'vgr_abi_version': [],
	'vgr_last_error': [],
}

ABI_VERSION = 27
_lib = None


def load():
	"""The loaded library (loaded once); raises RuntimeError when it is missing or out of date."""
	global _lib
	if _lib is None:
		if not os.path.exists(LIB_PATH):
			raise RuntimeError(f'{LIB_PATH} is not built: run __graft_entry__.build() (hipcc, gfx950) first')
		lib = ctypes.CDLL(LIB_PATH)
		for name, argtypes in SIGNATURES.items():
			fn = getattr(lib, name)
			fn.argtypes = argtypes
			fn.restype = ctypes.c_int
		lib.vgr_last_error.restype = ctypes.c_char_p
		lib.vgr_grid_work_size.restype = ctypes.c_int64
		lib.vgr_march_work_size.restype = ctypes.c_int64
		lib.vgr_march_backward_work_size.restype = ctypes.c_int64
		lib.vgr_foam_work_size.restype = ctypes.c_int64
		lib.vgr_field_work_size.restype = ctypes.c_int64
		lib.vgr_color_backward_work_size.restype = ctypes.c_int64
		lib.vgr_density_backward_work_size.restype = ctypes.c_int64
		lib.vgr_pack_work_size.restype = ctypes.c_int64
		lib.vgr_morton_work_size.restype = ctypes.c_int64
		lib.vgr_ray_order_work_size.restype = ctypes.c_int64
		if lib.vgr_abi_version() != ABI_VERSION:
			raise RuntimeError(f'{LIB_PATH} has ABI {lib.vgr_abi_version()}, expected {ABI_VERSION}: rebuild it')
		_lib = lib
	return _lib


def call(name, *args):
	"""Calls an entry point and raises RuntimeError with vgr_last_error() when it fails."""
	lib = load()
	rc = getattr(lib, name)(*args)
	if rc != 0:
		raise RuntimeError(f'{name[4:]}: {lib.vgr_last_error().decode()}')


def ptr(t):
	"""Device address of a tensor (None -> NULL)."""
	return None if t is None else t.data_ptr()


def stream_of(device):
	return torch.cuda.current_stream(device).cuda_stream
