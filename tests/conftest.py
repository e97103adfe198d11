"""pytest configuration: import paths (the product package, the oracle), the `gpu` marker, the guard that keeps GPU
tests honest (the HIP library must be built and load; no silent fallback), and the background triangulation of
the full-size benchmark scenes that the stated-size GPU tests need."""

import os
import subprocess
import sys
import time

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, 'voronoi-gauss_amd')
for p in (PKG, os.path.join(ROOT, 'oracle'), os.path.join(ROOT, 'tests')):
	if p not in sys.path:
		sys.path.insert(0, p)

STATED_SIZE_TESTS = 'test_gpu_stated_sizes'
_BUILDS = {}


def stated_configs():
	"""Benchmark configurations the stated-size tests cover: VGR_STATED_CONFIGS (comma-separated), default 2-5."""
	env = os.environ.get('VGR_STATED_CONFIGS', '2,3,4,5')
	return [int(c) for c in env.split(',') if c.strip()]


def pytest_configure(config):
	config.addinivalue_line('markers', 'gpu: needs an MI355X (gfx950) and the built libvgr.so')


def pytest_collection_finish(session):
	"""When stated-size tests are selected, triangulate their scenes (Qhull, single-threaded: about 50 s for 2M
	sites on the GPU box's host) in one child process per configuration, so that they run in parallel with each
	other and with the tests before them. Started before any test touches the GPU."""
	if session.config.option.collectonly or not any(STATED_SIZE_TESTS in item.nodeid for item in session.items):
		return
	from vgr import scenes
	os.makedirs(scenes.DEFAULT_CACHE, exist_ok=True)
	env = dict(os.environ, PYTHONPATH=PKG + os.pathsep + os.environ.get('PYTHONPATH', ''))
	for c in stated_configs():
		n = scenes.SITE_COUNTS[c]
		if os.path.exists(os.path.join(scenes.DEFAULT_CACHE, f'c{c}_s{scenes.SEEDS[c]}_n{n}_adj.npy')):
			continue
		log = open(os.path.join(scenes.DEFAULT_CACHE, f'build_c{c}.log'), 'w')
		_BUILDS[c] = (subprocess.Popen([sys.executable, '-m', 'vgr.scenes', '--geometry', str(c)], env=env,
										stdout=log, stderr=subprocess.STDOUT, cwd=ROOT), log.name, time.time())


def pytest_sessionfinish(session, exitstatus):
	for proc, _, _ in _BUILDS.values():
		if proc.poll() is None:
			proc.kill()
			proc.wait()


def progress(msg):
	"""A progress line on stdout and in stated_sizes_progress.log under the run's output folder: a wait of minutes
	for Qhull then still shows activity when pytest captures the output."""
	print(msg, flush=True)
	out = os.path.join(ROOT, 'gpurun_out')
	os.makedirs(out, exist_ok=True)
	with open(os.path.join(out, 'stated_sizes_progress.log'), 'a') as f:
		f.write(msg + '\n')


def wait_for_geometry(config, timeout=900):
	"""Blocks until the background triangulation of `config` (if one was started) has finished, reporting progress
	every 20 s; raises with its log when it failed or took longer than `timeout` seconds from its start."""
	if config not in _BUILDS:
		return
	proc, log, t0 = _BUILDS[config]
	while proc.poll() is None:
		if time.time() - t0 > timeout:
			proc.kill()
			proc.wait()
			raise RuntimeError(f'triangulation of config {config} did not finish in {timeout} s')
		progress(f'[stated sizes] waiting for the config-{config} triangulation ({time.time() - t0:.0f} s)')
		try:
			proc.wait(timeout=20)
		except subprocess.TimeoutExpired:
			pass
	if proc.returncode != 0:
		raise RuntimeError(f'triangulation of config {config} failed ({proc.returncode}):\n' + open(log).read()[-4000:])
	progress(f'[stated sizes] config {config} geometry ready {time.time() - t0:.0f} s after its build started')


@pytest.fixture(scope='session')
def oracle_lib():
	import oracle
	oracle.build()
	return oracle


@pytest.fixture(scope='session')
def gpu():
	"""The CUDA (HIP) device for GPU tests; fails (not skips) when there is none, since GPU tests only run where
	one is expected."""
	import torch
	if not torch.cuda.is_available():
		pytest.fail('GPU test run without a visible GPU')
	from vgr import _lib
	_lib.load()
	return torch.device('cuda:0')
