"""Batched prefill on the matrix cores (engine/core.cpp:292-294, 353-646).

The reference multiplies FP32 activations by FP32-widened weights
(cblas_sgemm, closed source, summation order unknown: parity unpinned
bitwise, held to tolerance). The GPU GEMM splits each activation exactly into
FP16 hi + lo and accumulates in FP32; it is checked against an FP64 product
with a bound proportional to sum |a||w|, for row independence from the
chunk size (needed for exact canonical prefix reuse), and end to end through
the oracle gate and the reuse-equals-fresh invariant
(tools/check_native_cpu_prefix.py).
"""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle_binding import compare_logits

PROMPTS = json.loads((Path(__file__).parent / 'golden' / 'prompts.json').read_text())


@pytest.mark.gpu
@pytest.mark.parametrize('m,n,k', [(1, 1024, 1024), (37, 4096, 1024), (85, 1024, 2048), (512, 6144, 1024),
                                   (129, 1024, 3072), (1000, 4096, 1024), (1100, 6144, 1024),
                                   (1024, 6144, 1024), (2500, 4096, 1024)])
def test_gemm_against_fp64(qpkg, m, n, k):
    """Row counts cover each tile-to-XCD mapping of 128-row tiles: 1000 /
    1024 rows (4 XCDs pool their row tiles), 1100 (2 XCDs pool 2 row tiles
    each), 2500 (2 XCDs pool 3 each), plus the narrower 32 / 64-row tiles."""
    rng = np.random.default_rng(21)
    a = rng.standard_normal((m, k), dtype=np.float32) * 3
    w = (rng.standard_normal((n, k), dtype=np.float32) * 0.02).astype(np.float16)
    got = qpkg.gemm(a, w)
    ref = a.astype(np.float64) @ w.astype(np.float64).T
    bound = 4e-6 * (np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T) + 1e-7
    err = np.abs(got - ref)
    assert np.all(err <= bound), float((err / bound).max())
    base = rng.standard_normal((m, n)).astype(np.float32)
    acc = qpkg.gemm(a, w, base)
    assert np.array_equal(acc, (base + got).astype(np.float32))


@pytest.mark.gpu
def test_gemm_range_guard(qpkg):
    """Rows holding values far beyond FP16's range (up to 3e6; FP16 ends at
    65504) are split as a * 2^-e and scaled back (engine/core.cpp:292-294
    multiplies FP32 activations): within the FP64 bound, while rows that fit
    FP16 keep the bits they have in a call where no row is scaled, through
    the allocating and the static entry points."""
    rng = np.random.default_rng(31)
    a = rng.standard_normal((300, 1024), dtype=np.float32)
    big = np.arange(0, 300, 7)
    a[big, 5] = 3e6
    a[big[::2], 900] = -7e4
    a[11, :] *= 40000.0
    w = (rng.standard_normal((1024, 1024), dtype=np.float32) * 0.02).astype(np.float16)
    ref = a.astype(np.float64) @ w.astype(np.float64).T
    bound = 4e-6 * (np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T) + 1e-7
    fits = np.setdiff1d(np.arange(300), np.r_[big, 11])
    alone = qpkg.gemm(a[fits], w)
    for got in (qpkg.gemm(a, w), qpkg.gemm_static(a, w)):
        assert np.isfinite(got).all()
        err = np.abs(got - ref)
        assert np.all(err <= bound), float((err / bound).max())
        assert np.array_equal(got[fits].view(np.uint32), alone.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize('m,amp', [(1024, 1.0), (100, 1.0), (3968, 1.0), (1024, 200.0), (100, 200.0)])
def test_gemm_swiglu_against_fp64(qpkg, m, amp):
    """The gate/up GEMM with its SwiGLU epilogue (engine/core.cpp:630-639 at
    batch > 1). 1024 rows take 128 x 192 tiles (256 workgroups in one round),
    100 rows narrower 32- or 64-row tiles and 3968 rows 128 x 256 tiles, so
    each epilogue's gate/up column mapping is exercised. Against FP64:
    g sigmoid(g) u with g, u the exact products, the GEMM error bound
    propagated through the activation's partial derivatives, plus the FP16
    hi + lo rounding of the stored result. With amp = 200 many activations
    lie beyond FP16's range: their groups of 8 carry exponents (the others
    keep 0, and so does every group at amp = 1)."""
    rng = np.random.default_rng(23 + m)
    a = rng.standard_normal((m, 1024), dtype=np.float32) * np.float32(amp)
    w = (rng.standard_normal((6144, 1024), dtype=np.float32) * 0.02).astype(np.float16)
    # Every column, every third row plus the last (the FP64 products of all
    # 3968 rows would dominate the test's time).
    rows = np.r_[0:m:3, m - 1]
    got, exps = qpkg.gemm_swiglu(a, w, exponents=True)
    got = got.astype(np.float64)[rows]
    if amp == 1.0:
        assert not exps.any()
    else:
        assert 0.005 < (exps > 0).mean() < 0.995, float((exps > 0).mean())
        assert np.isfinite(got).all()
    a64, w64 = a[rows].astype(np.float64), w.astype(np.float64)
    g, u = a64 @ w64[:3072].T, a64 @ w64[3072:].T
    sig = 1.0 / (1.0 + np.exp(-g))
    ref = g * sig * u
    bg = 4e-6 * (np.abs(a64) @ np.abs(w64[:3072]).T) + 1e-7
    bu = 4e-6 * (np.abs(a64) @ np.abs(w64[3072:]).T) + 1e-7
    # The last terms: the FP32 formula's own rounding, including 0.5 + 0.5 t
    # for t near -1 (tanhf saturates to -1 below g ~ -17, where FP64 still
    # has g sigmoid(g) u ~ 1e-8 g u): 2^-23 |g u| covers it.
    bound = (np.abs(sig * (1.0 + g * (1.0 - sig)) * u) * bg + np.abs(g * sig) * bu
             + 1e-6 * np.abs(ref) + 2.0 ** -23 * np.abs(g * u) + 1e-8)
    # The epilogue itself: the plain GEMM accumulates every element in the
    # same K order, so its g and u are the ones the SwiGLU epilogue saw. The
    # activation must be the reference formula evaluated in FP32 on them, up
    # to the spread of two tanhf implementations and what FP16 hi + lo holds
    # (2^-22 relative, half of FP16's subnormal spacing absolute). A hi / lo
    # pair rounded from two different values misses this by an FP16 ulp.
    plain = qpkg.gemm(a, w)[rows]
    g32, u32 = plain[:, :3072], plain[:, 3072:]
    t32 = np.tanh(np.float32(0.5) * g32).astype(np.float32)
    emu = (g32 * (np.float32(0.5) + np.float32(0.5) * t32) * u32).astype(np.float64)
    tol = (np.abs(g32.astype(np.float64) * u32) * 2.0 ** -23 + 4 * np.spacing(np.abs(emu).astype(np.float32))
           + 2.0 ** -21 * np.abs(emu) + 2.0 ** -24)
    assert np.all(np.abs(got - emu) <= tol), float((np.abs(got - emu) / tol).max())
    err = np.abs(got - ref)
    worst = np.unravel_index(np.argmax(err / bound), err.shape)
    assert np.all(err <= bound), dict(ratio=float((err / bound).max()), row=int(rows[worst[0]]), col=int(worst[1]),
                                      g=float(g[worst]), u=float(u[worst]), got=float(got[worst]),
                                      ref=float(ref[worst]), bound=float(bound[worst]))


def causal_attention_fp64(q, keys, values, pos0):
    """softmax(q k^T / sqrt(128)) v per query head over positions 0..pos0 + i,
    query head h reading KV head h // 2 (engine/core.cpp:407-605), in FP64."""
    rows = q.shape[0]
    out = np.empty((rows, 16, 128))
    k64, v64 = keys.astype(np.float64), values.astype(np.float64)
    for i in range(rows):
        n = pos0 + i + 1
        for h in range(16):
            s = k64[h // 2, :n] @ q[i, h].astype(np.float64) / np.sqrt(128.0)
            p = np.exp(s - s.max())
            out[i, h] = (p @ v64[h // 2, :n]) / p.sum()
    return out.reshape(rows, 2048)


@pytest.mark.gpu
@pytest.mark.parametrize('rows,pos0,boost', [(1, 0, False), (45, 0, True), (130, 200, True), (300, 37, False),
                                             (300, 37, True)])
def test_attention_prefill_against_fp64(qpkg, rows, pos0, boost):
    """The prefill attention kernel against an FP64 causal softmax. With
    `boost`, keys at positions 40, 97, 170 and 300 align with a direction
    every query shares, so their scores beat all earlier ones by about 14, 28,
    42 and 56 (natural log units), far past the kernel's lazy-rescale margin.
    Keys 170 and 300 lie in the second and third tiles of key split 1 (tiles
    of 32 keys, split = tile % 4), so the cases past 170 positions rescale a
    running output and sum mid-sequence: a CPU emulation of the kernel's
    order without that rescale misses these two cases by 3.6 and 4.5."""
    rng = np.random.default_rng(rows + pos0)
    context = pos0 + rows + 7
    u = rng.standard_normal(128)
    u *= 4.0 / np.linalg.norm(u)
    q = (u + 0.5 * rng.standard_normal((rows, 16, 128))).astype(np.float32)
    keys = (0.3 * rng.standard_normal((8, context, 128))).astype(np.float16)
    values = rng.standard_normal((8, context, 128)).astype(np.float16)
    if boost:
        for t, alpha in ((40, 10.0), (97, 20.0), (170, 30.0), (300, 40.0)):
            if t < pos0 + rows:
                keys[:, t] = (alpha * u).astype(np.float16)
    qkv = np.zeros((rows, 4096), np.float32)
    qkv[:, :2048] = q.reshape(rows, 2048)
    got = qpkg.attention_prefill(qkv, keys, values, pos0)
    ref = causal_attention_fp64(q, keys, values, pos0)
    err = np.abs(got - ref)
    assert np.all(err <= 1e-4 + 1e-4 * np.abs(ref)), float(err.max())


@pytest.mark.gpu
def test_attention_prefill_range_guard(qpkg):
    """Queries with a channel far beyond FP16's range (4e6 before the
    kernel's scale * log2(e), against keys that are 0 in that channel, so the
    scores stay moderate): the kernel splits such a query as q * 2^-e and
    scales its scores back, within the same FP64 tolerance as plain
    queries."""
    rng = np.random.default_rng(77)
    rows, pos0 = 70, 30
    context = pos0 + rows
    q = rng.standard_normal((rows, 16, 128)).astype(np.float32)
    q[::3, :, 17] = 4e6
    q[1::5, 2, 90] = -9e5
    keys = (0.3 * rng.standard_normal((8, context, 128))).astype(np.float16)
    keys[:, :, 17] = 0
    keys[:, :, 90] = 0
    values = rng.standard_normal((8, context, 128)).astype(np.float16)
    qkv = np.zeros((rows, 4096), np.float32)
    qkv[:, :2048] = q.reshape(rows, 2048)
    got = qpkg.attention_prefill(qkv, keys, values, pos0)
    ref = causal_attention_fp64(q, keys, values, pos0)
    err = np.abs(got - ref)
    assert np.all(err <= 1e-4 + 1e-4 * np.abs(ref)), float(err.max())


@pytest.mark.gpu
def test_gemm_rows_independent_of_chunk(qpkg):
    """Row results do not depend on M, on the row's position in a tile or on
    the tile height chosen for the launch (128-row tiles for 1200 x 4096,
    64-row tiles for the smaller calls)."""
    rng = np.random.default_rng(22)
    a = rng.standard_normal((1200, 1024), dtype=np.float32)
    w = (rng.standard_normal((4096, 1024), dtype=np.float32) * 0.02).astype(np.float16)
    full = qpkg.gemm(a, w)
    for rows in (slice(0, 37), slice(100, 101), slice(300, 512), slice(1100, 1200)):
        part = qpkg.gemm(a[rows], w)
        assert np.array_equal(part.view(np.uint32), full[rows].view(np.uint32))


@pytest.mark.gpu
def test_prefill_1024_matches_oracle(qpkg, pack0, oracle_lib):
    """The 1024-token prompt (seed 2): two full 512-row chunks."""
    prompt = PROMPTS['prefill_1024']
    with qpkg.Model(pack0) as gpu:
        oracle = oracle_lib.model(pack0, 16, 16, 4096)
        try:
            gpu.prefill(prompt)
            oracle.prefill(prompt)
            result = compare_logits(gpu.logits(), oracle.logits())
            print(result)
            assert result['passed'], result
            for _ in range(3):
                token = gpu.greedy()
                gpu.step(token)
                oracle.step(token)
                result = compare_logits(gpu.logits(), oracle.logits())
                assert result['passed'], result
        finally:
            oracle.close()


@pytest.mark.gpu
def test_canonical_prefix_reuse_equals_fresh(qpkg, pack0):
    """Rewind to a 512 boundary and prefill the rest == one fresh prefill
    (chunk shapes match; INTERFACE.md:94-111, tools/check_native_cpu_prefix.py)."""
    prompt = PROMPTS['long_3968'][:1100]
    with qpkg.Model(pack0) as m:
        m.prefill(prompt)
        fresh = (m.logits(), m.hidden())
        m.step(7)
        m.truncate(512)
        m.prefill(prompt[512:])
        assert np.array_equal(m.logits().view(np.uint32), fresh[0].view(np.uint32))
        assert np.array_equal(m.hidden().view(np.uint32), fresh[1].view(np.uint32))
        m.reset()
        m.prefill(prompt[:1024])
        m.truncate(1024)
        m.prefill(prompt[1024:])
        assert np.array_equal(m.logits().view(np.uint32), fresh[0].view(np.uint32))


@pytest.mark.gpu
def test_prefill_rows_independent_of_grouping(qpkg, pack0):
    """A call runs its consecutive 512-row chunks as one batched pass; that is
    only legal because every batched row is computed alone. Any split of a
    prompt into calls of two or more rows must give the same bits, and a
    trailing one-row chunk takes the batch-1 path like a step
    (engine/core.cpp:712)."""
    prompt = PROMPTS['long_3968'][:1025]
    with qpkg.Model(pack0) as m:
        m.prefill(prompt[:700])
        whole = m.logits().view(np.uint32).copy()
        m.reset()
        m.prefill(prompt[:300])
        m.prefill(prompt[300:700])
        assert np.array_equal(m.logits().view(np.uint32), whole)
        m.reset()
        m.prefill(prompt)  # 1024 batched rows + one batch-1 row
        tail = m.logits().view(np.uint32).copy()
        m.reset()
        m.prefill(prompt[:1024])
        m.step(prompt[1024])
        assert np.array_equal(m.logits().view(np.uint32), tail)
