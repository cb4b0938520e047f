"""GEMV parity on the GPU at the decode projection shapes (batch-1 FP16
weights, FP32 activations, FP32 accumulation; seed 1).

The HIP kernel owns one FP32 chain per thread and must reproduce the
reference dot order (engine/core.cpp:119-147) bit for bit, so the bar is
exact equality with the oracle's restatement, not a tolerance.
"""
import numpy as np
import pytest

SHAPES = [(1024, 2048), (1024, 1024), (2048, 1024), (1024, 3072), (3072, 1024), (1024, 151936)]


@pytest.mark.gpu
@pytest.mark.parametrize('n_in,n_out', SHAPES)
def test_gemv_bit_exact(qpkg, oracle_lib, n_in, n_out):
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((n_out, n_in), dtype=np.float32) * 0.02).astype(np.float16)
    x = rng.standard_normal(n_in, dtype=np.float32)
    expected = oracle_lib.gemv(w, x, threads=16)
    got = qpkg.gemv(qpkg.tile_matrix(w), x, n_out)
    mismatch = np.flatnonzero(got.view(np.uint32) != expected.view(np.uint32))
    assert mismatch.size == 0, f'{mismatch.size} rows differ, first {mismatch[:5]}: {got[mismatch[:5]]} vs {expected[mismatch[:5]]}'
    # Independent sanity: FP64 dot within the FP32 accumulation bound.
    ref = w.astype(np.float64) @ x.astype(np.float64)
    bound = 1e-5 * (np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))) + 1e-6
    assert np.all(np.abs(got - ref) <= bound)


@pytest.mark.gpu
def test_tile_interleaved_matches_plain(qpkg):
    """Gate/up interleaving: tile T holds 4 rows of each matrix."""
    rng = np.random.default_rng(5)
    g = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float16)
    u = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float16)
    x = rng.standard_normal(1024).astype(np.float32)
    both = qpkg.gemv(qpkg.tile_matrix(g, u), x, 128)
    yg = qpkg.gemv(qpkg.tile_matrix(g), x, 64)
    yu = qpkg.gemv(qpkg.tile_matrix(u), x, 64)
    interleaved = np.empty(128, np.float32)
    for t in range(16):
        interleaved[8 * t:8 * t + 4] = yg[4 * t:4 * t + 4]
        interleaved[8 * t + 4:8 * t + 8] = yu[4 * t:4 * t + 4]
    assert np.array_equal(both.view(np.uint32), interleaved.view(np.uint32))
