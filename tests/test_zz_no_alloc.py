"""The GEMM entry point that allocates nothing (qwen_gpu_op_gemm_static)
against qwen_gpu_op_gemm, which allocates its operand planes per call: the
same kernels on the same inputs, so results must be bit-identical. Two calls
in a row, the second smaller (it reuses the shared static planes the first
filled), accumulate mode, and a clear error past the planes' capacity."""
import numpy as np
import pytest


@pytest.mark.gpu
def test_gemm_static_matches_gemm(qpkg):
    rng = np.random.default_rng(31)
    # 512 x 2048 fills the static planes exactly (1048576 elements).
    for m, n, k in ((512, 2048, 2048), (37, 1024, 1024)):
        a = rng.standard_normal((m, k), dtype=np.float32) * 3
        w = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float16)
        expected = qpkg.gemm(a, w)
        got = qpkg.gemm_static(a, w)
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), (m, n, k)
        base = rng.standard_normal((m, n)).astype(np.float32)
        assert np.array_equal(qpkg.gemm_static(a, w, base).view(np.uint32),
                              qpkg.gemm(a, w, base).view(np.uint32)), (m, n, k)


@pytest.mark.gpu
def test_gemm_static_rejects_oversize(qpkg):
    a = np.zeros((1025, 1024), np.float32)
    w = np.zeros((128, 1024), np.float16)
    with pytest.raises(RuntimeError, match='exceeds the 1048576 operand elements'):
        qpkg.gemm_static(a, w)
