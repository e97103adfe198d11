"""Builds libvgr.so (all HIP kernels + the C ABI) for gfx950 with hipcc, in place next to this file."""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), 'csrc')
SOURCES = ['abi.hip', 'foam_infer.hip', 'foam_faces.hip', 'field_grad.hip', 'pack.hip', 'march.hip', 'field.hip', 'grid.hip',
		   'order.hip']
LIB = os.path.join(HERE, 'libvgr.so')

# -ffp-contract=off: traversal arithmetic rounds exactly as written (bit-exact walks against the CPU oracle).
# -packed-fp32-ops: no packed fp32 VALU ops are generated.
HIPCC_FLAGS = ['--offload-arch=gfx950', '-O3', '-std=c++17', '-fPIC', '-shared', '-ffp-contract=off',
			   '-mcode-object-version=5', '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops', '-Wall']


def hipcc():
	rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
	return os.path.join(rocm, 'bin', 'hipcc')


def build_library(verbose=False):
	"""Compiles every source of csrc/ into libvgr.so (always recompiles); raises on failure."""
	tmp = LIB + '.tmp'
	cmd = [hipcc(), *HIPCC_FLAGS, '-o', tmp, *[os.path.join(CSRC, s) for s in SOURCES]]
	res = subprocess.run(cmd, capture_output=True, text=True)
	msgs = '\n'.join(line for line in (res.stdout + res.stderr).splitlines() if 'packed-fp32-ops' not in line)
	if res.returncode != 0:
		raise RuntimeError(f'hipcc failed ({res.returncode}):\n{" ".join(cmd)}\n{msgs}')
	if verbose and msgs.strip():
		print(msgs)
	os.replace(tmp, LIB)
	return LIB


if __name__ == '__main__':
	print(build_library(verbose=True))
