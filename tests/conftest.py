"""pytest configuration: import paths (the product package, the oracle), the `gpu` marker, and the guard that
keeps GPU tests honest (the HIP library must be built and load; no silent fallback)."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, 'voronoi-gauss_amd'), os.path.join(ROOT, 'oracle'), os.path.join(ROOT, 'tests')):
	if p not in sys.path:
		sys.path.insert(0, p)


def pytest_configure(config):
	config.addinivalue_line('markers', 'gpu: needs an MI355X (gfx950) and the built libvgr.so')


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
