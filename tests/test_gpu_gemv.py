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


# ---- the fused decode projections, as a step runs them ----

def _fold_parts(x, parts):
    """x + the 16 per-query-head O partials in the engine's fixed tree order
    (FP32 throughout): ((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7)) then the same over
    p8..p15. A plausible slip (another order, a dropped partial) changes the
    bits of some entries at these magnitudes, so equality pins the order."""
    p = np.asarray(parts, np.float32)
    lo = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]))
    hi = ((p[8] + p[9]) + (p[10] + p[11])) + ((p[12] + p[13]) + (p[14] + p[15]))
    return np.asarray(x, np.float32) + (lo + hi)


def _decode_inputs(seed, rows, cols):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols), dtype=np.float32) * 0.02).astype(np.float16)
    x = rng.standard_normal(1024, dtype=np.float32)
    norm_w = (1.0 + 0.1 * rng.standard_normal(1024, dtype=np.float32)).astype(np.float32)
    parts = (0.05 * rng.standard_normal((16, 1024), dtype=np.float32)).astype(np.float32)
    return rng, w, x, norm_w, parts


def _assert_same_bits(got, expected, what):
    got, expected = np.asarray(got, np.float32), np.asarray(expected, np.float32)
    mismatch = np.flatnonzero(got.view(np.uint32) != expected.view(np.uint32))
    assert mismatch.size == 0, (f'{what}: {mismatch.size} entries differ, first {mismatch[:5]}: '
                                f'{got[mismatch[:5]]} vs {expected[mismatch[:5]]}')


@pytest.mark.gpu
def test_norm_qkv_bit_exact(qpkg, oracle_lib):
    """QKV with the RMSNorm prologue (engine/core.cpp:384-386): the oracle's
    norm then its chain-ordered GEMV over the stacked q/k/v rows."""
    _, w, x, norm_w, _ = _decode_inputs(11, 4096, 1024)
    got = qpkg.norm_qkv(qpkg.tile_matrix(w), norm_w, x)
    expected = oracle_lib.gemv(w, oracle_lib.norm(x, norm_w), threads=16)
    _assert_same_bits(got, expected, 'qkv')


@pytest.mark.gpu
@pytest.mark.parametrize('with_parts', [False, True])
def test_norm_gate_up_bit_exact(qpkg, oracle_lib, with_parts):
    """Gate/up with the O-partial fold and RMSNorm prologue (engine/core.cpp:
    625-635): the dot products are the oracle's bit for bit; the SwiGLU
    epilogue (636-639) on those same values is within the few-ulp spread of
    two tanhf implementations (GPU libm vs glibc)."""
    rng, w, x, norm_w, parts = _decode_inputs(12 + with_parts, 3072, 1024)
    up = (rng.standard_normal((3072, 1024), dtype=np.float32) * 0.02).astype(np.float16)
    act, gate_rows, up_rows = qpkg.norm_gate_up(qpkg.tile_matrix(w, up), norm_w, x,
                                                parts if with_parts else None)
    h = oracle_lib.norm(_fold_parts(x, parts) if with_parts else x, norm_w)
    _assert_same_bits(gate_rows, oracle_lib.gemv(w, h, threads=16), 'gate rows')
    _assert_same_bits(up_rows, oracle_lib.gemv(up, h, threads=16), 'up rows')
    expected = oracle_lib.swiglu(gate_rows, up_rows)
    # A tanhf result t off by k ulp moves g (0.5 + 0.5 t) u by 0.5 |g u| k ulp(t).
    g, u = gate_rows.astype(np.float64), up_rows.astype(np.float64)
    bound = 0.5 * np.abs(g * u) * 2 * 2.0 ** -23 + 4 * np.spacing(np.abs(expected)).astype(np.float64)
    err = np.abs(act.astype(np.float64) - expected.astype(np.float64))
    assert (err <= bound).all(), float((err / bound).max())
    exact = np.mean(act.view(np.uint32) == expected.view(np.uint32))
    print('swiglu entries bit-equal to the oracle:', exact)
    # And against the closed form g sigmoid(g) u in FP64 (a sign or a dropped
    # half in the epilogue fails this).
    ref = g / (1.0 + np.exp(-g)) * u
    assert np.allclose(act, ref, rtol=1e-5, atol=1e-7)


@pytest.mark.gpu
@pytest.mark.parametrize('with_parts', [False, True])
def test_down_residual_bit_exact(qpkg, oracle_lib, with_parts):
    """Down projection + residual (engine/core.cpp:640-641) on two-segment
    chains, with and without the pending O partials folded into the
    residual entry first."""
    rng, w, x, _, parts = _decode_inputs(14 + with_parts, 1024, 3072)
    act = (0.3 * rng.standard_normal(3072, dtype=np.float32)).astype(np.float32)
    got = qpkg.down_residual(qpkg.tile_matrix(w), act, x, parts if with_parts else None)
    base = _fold_parts(x, parts) if with_parts else x
    expected = base + oracle_lib.gemv(w, act, threads=16)
    _assert_same_bits(got, expected, 'x')


def _fold_slices(xm, d):
    """xm + the 8 per-slice down products in the engine's fixed tree order
    ((d0+d1)+(d2+d3))+((d4+d5)+(d6+d7)), FP32 throughout."""
    d = np.asarray(d, np.float32)
    return np.asarray(xm, np.float32) + (((d[0] + d[1]) + (d[2] + d[3])) + ((d[4] + d[5]) + (d[6] + d[7])))


@pytest.mark.gpu
@pytest.mark.parametrize('with_parts', [False, True])
def test_fused_ffn_slices_bit_exact(qpkg, oracle_lib, with_parts):
    """The fused FFN kernel (norm + gate/up + SwiGLU + down in one launch,
    engine/core.cpp:625-641 with the down projection split into 8 column
    slices exchanged inside each XCD): xm is x plus the folded O partials bit
    for bit; the activations it exchanges are the norm+gate/up kernel's bit
    for bit; slice g's down product is the oracle's chain-ordered dot over
    columns 384g .. 384g + 383 bit for bit; and the folded slices lie within
    the FP32 accumulation bound of the whole product in FP64 (a slice taken
    from the wrong columns or rows fails all three). Two calls in a row
    reuse the exchange with a new tag."""
    rng, gate, x, norm_w, parts = _decode_inputs(16 + with_parts, 3072, 1024)
    up = (rng.standard_normal((3072, 1024), dtype=np.float32) * 0.02).astype(np.float16)
    down = (rng.standard_normal((1024, 3072), dtype=np.float32) * 0.02).astype(np.float16)
    gu_t, down_t = qpkg.tile_matrix(gate, up), qpkg.tile_matrix(down)
    ffn = qpkg.FusedFfn()
    p = parts if with_parts else None
    act_ref, _, _ = qpkg.norm_gate_up(gu_t, norm_w, x, p)
    for call in range(2):
        xm, dparts, act, stalled = ffn(gu_t, down_t, norm_w, x, p)
        assert stalled == 0
        _assert_same_bits(xm, _fold_parts(x, parts if with_parts else np.zeros((16, 1024), np.float32)), 'xm')
        _assert_same_bits(act, act_ref, 'act')
        for g in range(8):
            cols = slice(384 * g, 384 * (g + 1))
            expected = oracle_lib.gemv(np.ascontiguousarray(down[:, cols]), np.ascontiguousarray(act[cols]), threads=16)
            _assert_same_bits(dparts[g], expected, f'down slice {g}')
        total = _fold_slices(np.zeros(1024, np.float32), dparts).astype(np.float64)
        ref = down.astype(np.float64) @ act.astype(np.float64)
        bound = 1e-5 * (np.abs(down.astype(np.float64)) @ np.abs(act.astype(np.float64))) + 1e-7
        assert np.all(np.abs(total - ref) <= bound), float((np.abs(total - ref) / bound).max())


@pytest.mark.gpu
def test_norm_qkv_folded_bit_exact(qpkg, oracle_lib):
    """QKV after a fused FFN layer: the residual is xm plus the 8 down slices
    in the fixed tree order (written out bit for bit), then the oracle's norm
    and chain-ordered GEMV over the stacked q/k/v rows (engine/core.cpp:641,
    384-386)."""
    rng, w, xm, norm_w, _ = _decode_inputs(18, 4096, 1024)
    d = (0.05 * rng.standard_normal((8, 1024), dtype=np.float32)).astype(np.float32)
    x, qkv = qpkg.norm_qkv_folded(qpkg.tile_matrix(w), norm_w, xm, d)
    xf = _fold_slices(xm, d)
    _assert_same_bits(x, xf, 'x')
    _assert_same_bits(qkv, oracle_lib.gemv(w, oracle_lib.norm(xf, norm_w), threads=16), 'qkv')
