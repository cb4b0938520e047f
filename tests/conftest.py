"""Shared fixtures: package loader, seeded weight packs, oracle binding."""
import importlib.util
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / 'tests' / 'golden'
PACK_CACHE = Path(os.environ.get('QWEN_GPU_PACK_CACHE', '/tmp/qwen_gpu_packs'))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X GPU')


def load_package():
    """Import fpga-qwen_amd/ (a directory name Python cannot import directly)."""
    if 'fpga_qwen_amd' in sys.modules:
        return sys.modules['fpga_qwen_amd']
    package_dir = ROOT / 'fpga-qwen_amd'
    spec = importlib.util.spec_from_file_location('fpga_qwen_amd', package_dir / '__init__.py',
                                                  submodule_search_locations=[str(package_dir)])
    module = importlib.util.module_from_spec(spec)
    sys.modules['fpga_qwen_amd'] = module
    spec.loader.exec_module(module)
    return module


@pytest.fixture(scope='session')
def qpkg():
    return load_package()


@pytest.fixture(scope='session')
def pack0(qpkg):
    """QWCPU01 pack with seed 0 (all matrices N(0, 0.02) FP16, norm gains 1.0)."""
    return qpkg.ensure_random_pack(PACK_CACHE / 'seed0', seed=0)


@pytest.fixture(scope='session')
def oracle_lib():
    sys.path.insert(0, str(ROOT / 'tests'))
    from oracle_binding import OracleLib
    return OracleLib()
