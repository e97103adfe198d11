"""Builds libvgr.so (all HIP kernels + the C ABI) for gfx950 with hipcc, in place next to this file.

Each source compiles to its own object in parallel (one hipcc process per file), then hipcc links them."""

import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), 'csrc')
SOURCES = ['abi.hip', 'foam_infer.hip', 'foam_faces.hip', 'field_grad.hip', 'pack.hip', 'march.hip', 'field.hip', 'grid.hip',
		   'order.hip']
LIB = os.path.join(HERE, 'libvgr.so')

# -ffp-contract=off: traversal arithmetic rounds exactly as written (bit-exact walks against the CPU oracle).
# -packed-fp32-ops: no packed fp32 VALU ops are generated.
HIPCC_FLAGS = ['--offload-arch=gfx950', '-O3', '-std=c++17', '-fPIC', '-shared', '-ffp-contract=off',
			   '-mcode-object-version=5', '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops', '-Wall']
COMPILE_FLAGS = [f for f in HIPCC_FLAGS if f != '-shared']


def hipcc():
	rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
	return os.path.join(rocm, 'bin', 'hipcc')


def _run(cmd):
	res = subprocess.run(cmd, capture_output=True, text=True)
	msgs = '\n'.join(line for line in (res.stdout + res.stderr).splitlines() if 'packed-fp32-ops' not in line)
	if res.returncode != 0:
		raise RuntimeError(f'hipcc failed ({res.returncode}):\n{" ".join(cmd)}\n{msgs}')
	return msgs


def build_library(verbose=False, jobs=None):
	"""Compiles every source of csrc/ into libvgr.so (always recompiles); raises on failure."""
	jobs = jobs or min(len(SOURCES), max(1, min(16, os.cpu_count() or 1)))
	tmpdir = tempfile.mkdtemp(prefix='vgr_build_')
	try:
		objs = [os.path.join(tmpdir, os.path.splitext(s)[0] + '.o') for s in SOURCES]
		cmds = [[hipcc(), *COMPILE_FLAGS, '-c', '-o', obj, os.path.join(CSRC, src)] for src, obj in zip(SOURCES, objs)]
		with ThreadPoolExecutor(max_workers=jobs) as pool:
			msgs = list(pool.map(_run, cmds))
		tmp = LIB + '.tmp'
		msgs.append(_run([hipcc(), *HIPCC_FLAGS, '-o', tmp, *objs]))
	finally:
		shutil.rmtree(tmpdir, ignore_errors=True)
	text = '\n'.join(m for m in msgs if m.strip())
	if verbose and text.strip():
		print(text)
	os.replace(tmp, LIB)
	return LIB


if __name__ == '__main__':
	print(build_library(verbose=True))
