"""The C-ABI boundary: library loads, exports exactly what include/qwen_gpu.h
declares, and both public headers compile on their own (CPU only; no
compute call is made)."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / 'include' / 'qwen_gpu.h'


def declared_functions():
    text = re.sub(r'/\*.*?\*/', '', HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r'\b(qwen_gpu_[a-z0-9_]+)\s*\(', text)))


def test_header_symbols_exported(qpkg):
    names = declared_functions()
    assert len(names) >= 20
    lib = ctypes.CDLL(str(qpkg.LIBRARY_PATH))
    for name in names:
        assert hasattr(lib, name), f'{name} declared but not exported'
    assert set(names) == set(qpkg.SIGNATURES), 'Python binding out of sync with the header'


def test_exported_symbols_declared(qpkg):
    out = subprocess.run(['nm', '-D', '--defined-only', str(qpkg.LIBRARY_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if ' T qwen_gpu_' in line}
    assert exported == set(declared_functions())


def test_c_header_is_plain_c(tmp_path):
    src = tmp_path / 'use.c'
    src.write_text('#include "qwen_gpu.h"\nint main(void){qwen_gpu_options o={12,6,4096};(void)o;'
                   'return QWEN_GPU_VOCABULARY==151936?0:1;}\n')
    subprocess.run(['gcc', '-std=c99', '-Wall', '-Werror', '-pedantic', '-fsyntax-only', f'-I{ROOT / "include"}',
                    str(src)], check=True)


def test_cpp_facade_compiles(tmp_path):
    src = tmp_path / 'use.cpp'
    src.write_text('#include "qwen_gpu.hpp"\n'
                   'int run(qwen_gpu::Model& m){m.reset();m.prefill({1,2});m.step(3);'
                   'auto r=m.verify_two(4,5);m.commit_verified(1);'
                   'return int(m.logits().size()+m.hidden().size()+r.logits.size())+m.position();}\n')
    subprocess.run(['g++', '-std=c++20', '-Wall', '-Werror', '-fsyntax-only', f'-I{ROOT / "include"}', str(src)],
                   check=True)


def test_create_errors_are_reported(qpkg, pack0):
    with pytest.raises(RuntimeError, match='Cannot open weights'):
        qpkg.Model('/nonexistent/weights.bin')
    with pytest.raises(RuntimeError, match='Context must be in 1..4096'):
        qpkg.Model(pack0, context=0)
    try:
        model = qpkg.Model(pack0, context=8)
    except RuntimeError as error:  # CPU-only host: validated pack, then no device
        assert 'No HIP device available' in str(error)
    else:
        model.close()
        pytest.skip('a GPU is present')


@pytest.mark.parametrize('name', ['gemm', 'gemm_static'])
def test_gemm_shapes_checked_before_the_device(qpkg, name):
    """The GEMM wrappers reject operands the kernel's whole-tile reads and
    writes would overrun before any device buffer exists (so on a host
    without a GPU too)."""
    call = getattr(qpkg, name)
    a = np.zeros((4, 64), np.float32)
    for w, c, message in ((np.zeros((128, 128), np.float16), None, 'w must be'),
                          (np.zeros((100, 64), np.float16), None, 'w must be'),
                          (np.zeros((128, 64), np.float16), np.zeros((4, 100), np.float32), 'c must be'),
                          (np.zeros(128, np.float16), None, 'matrices')):
        with pytest.raises(ValueError, match=message):
            call(a, w, c)
    with pytest.raises(ValueError, match='w must be'):
        call(np.zeros((4, 96), np.float32), np.zeros((128, 96), np.float16))
