"""Batched decode of several sequences that share the weights (the
prefix-reuse workload: a canonical prefix rewound and reused, distinct
suffixes, greedy decode as a batch on one GPU).

The reference is single-stream, so parity is per sequence: every sequence
of a batched step must match the same sequence stepped alone (Model::step,
engine/core.cpp:707-714) and the oracle trajectory, under the gate of
tools/check_native_saved_oracle.py:36 (max-abs 1e-2, RMS 2e-3, greedy
identity). The batched projections run on the matrix cores (FP32
activations as FP16 hi + lo), so they are held to that gate and to an FP64
bound, not to bit equality with the batch-1 GEMVs.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle_binding import compare_logits

PROMPTS = json.loads((Path(__file__).parent / 'golden' / 'prompts.json').read_text())


@pytest.mark.gpu
@pytest.mark.parametrize('rows,cols', [(4096, 1024), (1024, 2048), (1024, 3072), (6144, 1024)])
@pytest.mark.parametrize('batch', [1, 3, 8])
def test_bgemv_against_fp64(qpkg, rows, cols, batch):
    """The batched projection against FP64. For 3 and 8 sequences, sequence
    1 holds values beyond FP16's range (split as x * 2^-e, products scaled
    back); the other sequences keep the bits of a call without it."""
    rng = np.random.default_rng(1000 + rows + cols + batch)
    w = (rng.standard_normal((rows, cols), dtype=np.float32) * 0.02).astype(np.float16)
    x = rng.standard_normal((batch, cols), dtype=np.float32)
    if batch > 1:
        plain = qpkg.bgemv(w, np.delete(x, 1, axis=0))
        x[1, ::97] = 2e6
    y = qpkg.bgemv(w, x)
    if batch > 1:
        assert np.array_equal(np.delete(y, 1, axis=0).view(np.uint32), plain.view(np.uint32))
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    ref = x64 @ w64.T
    bound = 4e-6 * (np.abs(x64) @ np.abs(w64).T) + 1e-7
    err = np.abs(y.astype(np.float64) - ref)
    assert (err <= bound).all(), float((err / bound).max())


def _seed_sequences(qpkg, pack0):
    """A base model with a 300-token prefix; three sequences reuse it with
    suffixes of 20, 37 and 5 tokens, a fourth runs its own 600-token prompt
    (past 512 positions). Returns (base, batch sequences, twins stepped alone)."""
    prompt = PROMPTS['long_3968']
    base = qpkg.Model(pack0, context=4096)
    base.prefill(prompt[:300])
    batch, alone = [], []
    for suffix in (prompt[300:320], prompt[300:337], prompt[1000:1005]):
        for group in (batch, alone):
            m = base.share()
            m.copy_prefix(base, 300)
            m.prefill(suffix)
            group.append(m)
    for group in (batch, alone):
        m = base.share()
        m.prefill(prompt[2000:2600])
        group.append(m)
    return base, batch, alone


@pytest.mark.gpu
def test_step_batch_equals_single_steps(qpkg, pack0):
    base, batch, alone = _seed_sequences(qpkg, pack0)
    try:
        tokens = [m.greedy() for m in batch]
        assert tokens == [m.greedy() for m in alone]
        worst = 0.0
        for _ in range(6):
            qpkg.step_batch(batch, tokens)
            for m, t in zip(alone, tokens):
                m.step(t)
            for b, a in zip(batch, alone):
                assert b.position() == a.position()
                result = compare_logits(b.logits(), a.logits())
                assert result['passed'], result
                worst = max(worst, result['max_abs'])
                assert np.array_equal(b.hidden().shape, (1024,))
            tokens = [m.greedy() for m in batch]
            assert tokens == [m.greedy() for m in alone]
        print('max_abs batched vs alone', worst)
    finally:
        for m in batch + alone + [base]:
            m.close()


@pytest.mark.gpu
def test_step_batch_matches_oracle(qpkg, pack0, oracle_lib):
    prompt = PROMPTS['long_3968']
    base = qpkg.Model(pack0, context=4096)
    other = base.share()
    oracle = oracle_lib.model(pack0, 16, 16, 4096)
    try:
        base.prefill(prompt[:85])
        other.prefill(prompt[500:530])
        oracle.prefill(prompt[:85])
        tokens = [base.greedy(), other.greedy()]
        for _ in range(8):
            qpkg.step_batch([base, other], tokens)
            oracle.step(tokens[0])
            result = compare_logits(base.logits(), oracle.logits())
            assert result['passed'], result
            tokens = [base.greedy(), other.greedy()]
    finally:
        oracle.close()
        other.close()
        base.close()


@pytest.mark.gpu
def test_copy_prefix_equals_truncate(qpkg, pack0):
    prompt = PROMPTS['long_3968']
    with qpkg.Model(pack0) as a:
        b = a.share(context=1024)
        try:
            a.prefill(prompt[:700])
            b.copy_prefix(a, 512)
            assert b.position() == 512 and b.logits().size == 0
            b.prefill(prompt[512:800])
            a.truncate(512)
            a.prefill(prompt[512:800])
            assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))
            with pytest.raises(RuntimeError, match='Rewind position out of range'):
                b.copy_prefix(a, 801)
        finally:
            b.close()


def _prefix_family(qpkg, pack0):
    """A base sequence and six sequences built from copies of its rows:
    copies of 700 and 520 rows, a 650-row copy rewound to 200 and refilled
    with other tokens, a copy of the first copy (600 rows), a 640-row copy
    with a larger cache than the copy it reads its rows from (another row
    stride), and a copy taken after the base was rewound to 100 and refilled
    (its rows 100.. differ)."""
    prompt = PROMPTS['long_3968']
    base = qpkg.Model(pack0, context=4096)
    base.prefill(prompt[:700])
    seqs = []
    for source_index, rows, rewind, suffix, context in ((None, 700, None, prompt[1000:1010], 2048),
                                                        (None, 520, None, prompt[1100:1150], 2048),
                                                        (None, 650, 200, prompt[1200:1500], 2048),
                                                        (0, 600, None, prompt[1300:1330], 2048),
                                                        (None, 640, None, prompt[1400:1420], 3000)):
        m = base.share(context=context)
        m.copy_prefix(base if source_index is None else seqs[source_index], rows)
        if rewind is not None:
            m.truncate(rewind)
        m.prefill(suffix)
        seqs.append(m)
    base.truncate(100)
    base.prefill(prompt[2000:2500])
    m = base.share()
    m.copy_prefix(base, 450)
    m.prefill(prompt[2600:2620])
    seqs.append(m)
    return seqs + [base]


@pytest.mark.gpu
def test_shared_prefix_rows_bit_identical(qpkg, pack0, monkeypatch):
    """Sequences of a batched step that hold copies of the same rows read
    them from one cache (whole 64-row blocks up to the shorter copy). The
    rows are equal, so every step's logits must equal, bit for bit, those of
    the same sequences each reading its own cache (QWEN_HIP_SHARED_PREFIX=0
    when they are created). A copy rewound below its prefix, or one of a
    source that was rewound and refilled, would read wrong rows if it were
    still grouped: those sequences' logits would then differ."""
    monkeypatch.setenv('QWEN_HIP_SHARED_PREFIX', '0')
    own = _prefix_family(qpkg, pack0)
    monkeypatch.delenv('QWEN_HIP_SHARED_PREFIX')
    shared = _prefix_family(qpkg, pack0)
    try:
        tokens = [m.greedy() for m in shared]
        assert tokens == [m.greedy() for m in own]
        for _ in range(4):
            qpkg.step_batch(shared, tokens)
            qpkg.step_batch(own, tokens)
            for i, (a, b) in enumerate(zip(shared, own)):
                assert a.position() == b.position()
                assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32)), i
            tokens = [m.greedy() for m in shared]
    finally:
        for m in shared + own:
            m.close()


@pytest.mark.gpu
def test_step_batch_greedy_returns_the_selections(qpkg, pack0):
    """step_batch_greedy = step_batch followed by each model's greedy():
    same selections and bit-identical logits along a 4-step trajectory."""
    base, batch, alone = _seed_sequences(qpkg, pack0)
    try:
        tokens = [m.greedy() for m in batch]
        for _ in range(4):
            nxt = qpkg.step_batch_greedy(batch, tokens)
            qpkg.step_batch(alone, tokens)
            assert nxt == [m.greedy() for m in alone] == [m.greedy() for m in batch]
            for b, a in zip(batch, alone):
                assert np.array_equal(b.logits().view(np.uint32), a.logits().view(np.uint32))
            tokens = nxt
        with pytest.raises(RuntimeError, match='Token ID out of range'):
            qpkg.step_batch_greedy(batch[:2], [1, 151936])
    finally:
        for m in batch + alone + [base]:
            m.close()


@pytest.mark.gpu
def test_step_batch_validates_before_running(qpkg, pack0):
    prompt = PROMPTS['long_3968']
    with qpkg.Model(pack0) as a, qpkg.Model(pack0) as stranger:
        b = a.share()
        try:
            a.prefill(prompt[:10])
            b.prefill(prompt[10:30])
            stranger.prefill(prompt[:5])
            before = (a.position(), b.position(), a.logits().copy())
            for models, tokens, message in (
                    ([a, stranger], [1, 2], 'do not share weights'),
                    ([a, b], [1, 151936], 'Token ID out of range'),
                    ([a, a], [1, 2], 'repeated'),
                    ([a] * 9, [1] * 9, '1..8')):
                with pytest.raises(RuntimeError, match=message):
                    qpkg.step_batch(models, tokens)
                assert (a.position(), b.position()) == before[:2]
            assert np.array_equal(a.logits(), before[2])
            b.verify_two(3, 4)
            with pytest.raises(RuntimeError, match='Commit or discard pending verification'):
                qpkg.step_batch([a, b], [1, 2])
            assert (a.position(), b.position()) == before[:2]
        finally:
            b.close()


@pytest.mark.gpu
def test_prefix_reuse_workload_matches_oracle(qpkg, pack0, oracle_lib):
    """The 8-sequence prefix-reuse workload at its real size
    (engine/INTERFACE.md:94-103, tools/native_cpu_chat.py:198-216): the
    canonical 512-token prefix is prefilled once; 8 sequences take a device
    copy of its K/V (the 512-token rewind), prefill their own 1536-token
    suffix (positions 512..2047) and decode 8 greedy steps together through
    step_batch (contexts 2049..2056: each sequence's 33 blocks of 64
    positions split into 4 pieces per KV head, its first 512 rows read from
    one shared copy). Teacher-forced against the oracle (rewind to 512, prefill
    the suffix, step the same tokens), every sequence's logits after its
    prefill and after each batched step pass the reference gate; then each
    sequence re-steps the same tokens alone from position 2048 (batch-1
    path), and those rows too pass the gate against its batched rows."""
    prefix, suffixes = PROMPTS['prefix_512'], PROMPTS['suffix_1536']
    assert len(prefix) == 512 and len(suffixes) == 8 and all(len(s) == 1536 for s in suffixes)
    steps = 8
    base = qpkg.Model(pack0, context=4096)
    seqs = [base.share(context=2304) for _ in suffixes]
    try:
        base.prefill(prefix)
        for m, suffix in zip(seqs, suffixes):
            m.copy_prefix(base, len(prefix))
            m.prefill(suffix)
        rows = [[(m.logits(), m.greedy())] for m in seqs]
        for _ in range(steps):
            qpkg.step_batch(seqs, [r[-1][1] for r in rows])
            for r, m in zip(rows, seqs):
                r.append((m.logits(), m.greedy()))
        assert all(m.position() == 2048 + steps for m in seqs)
        worst_alone = 0.0
        for r, m in zip(rows, seqs):
            m.truncate(2048)
            for k in range(1, steps + 1):
                m.step(r[k - 1][1])
                result = compare_logits(m.logits(), r[k][0])
                assert result['passed'], ('alone vs batched', k, result)
                worst_alone = max(worst_alone, result['max_abs'])
    finally:
        for m in seqs + [base]:
            m.close()
    oracle = oracle_lib.model(pack0, 16, 16, 4096)
    worst = 0.0
    try:
        oracle.prefill(prefix)
        for i, suffix in enumerate(suffixes):
            oracle.truncate(len(prefix))
            oracle.prefill(suffix)
            for k, (logits, _) in enumerate(rows[i]):
                if k:
                    oracle.step(rows[i][k - 1][1])
                result = compare_logits(logits, oracle.logits())
                assert result['passed'], ('sequence', i, 'row', k, result)
                worst = max(worst, result['max_abs'])
    finally:
        oracle.close()
    print('max_abs vs oracle', worst, 'alone vs batched', worst_alone)


@pytest.mark.gpu
def test_step_batch_long_pieces(qpkg, pack0, oracle_lib):
    """8 sequences at 2,900-3,043 and at 3,884-4,062 positions: each
    sequence's 64-position blocks, split into 4 pieces per KV head, give 12
    and 16 blocks per piece (the batched attention kernel's two largest
    forms, past what the 2,048-position prefix-reuse workload reaches). Every
    batched row passes the reference gate against the same sequence
    re-stepped alone, and sequence 0's rows against the oracle."""
    prompt, other = PROMPTS['long_3968'], PROMPTS['prefill_1024']
    steps = 3
    base = qpkg.Model(pack0, context=4096)
    seqs = [base.share() for _ in range(8)]
    oracle = oracle_lib.model(pack0, 16, 16, 4096)
    worst_alone = worst_oracle = 0.0
    oracle_valid = 0
    try:
        for shared, lengths in ((2816, [2900 + 20 * i for i in range(8)]), (3584, [3884 + 25 * i for i in range(8)])):
            base.reset()
            base.prefill(prompt[:shared])
            starts = []
            for i, (m, n) in enumerate(zip(seqs, lengths)):
                suffix = prompt[shared:n] if i == 0 else other[37 * i:37 * i + n - shared]
                assert len(suffix) == n - shared
                m.copy_prefix(base, shared)
                m.prefill(suffix)
                starts.append(m.position())
            rows = [[(m.logits(), m.greedy())] for m in seqs]
            for _ in range(steps):
                qpkg.step_batch(seqs, [r[-1][1] for r in rows])
                for r, m in zip(rows, seqs):
                    r.append((m.logits(), m.greedy()))
            for r, m, start in zip(rows, seqs, starts):
                m.truncate(start)
                for k in range(1, steps + 1):
                    m.step(r[k - 1][1])
                    result = compare_logits(m.logits(), r[k][0])
                    assert result['passed'], ('alone vs batched', start, k, result)
                    worst_alone = max(worst_alone, result['max_abs'])
            oracle.truncate(min(oracle_valid, lengths[0]))
            oracle.prefill(prompt[min(oracle_valid, lengths[0]):lengths[0]])
            for k, (logits, _) in enumerate(rows[0]):
                if k:
                    oracle.step(rows[0][k - 1][1])
                result = compare_logits(logits, oracle.logits())
                assert result['passed'], ('sequence 0', lengths[0], k, result)
                worst_oracle = max(worst_oracle, result['max_abs'])
            oracle_valid = lengths[0]
    finally:
        for m in seqs + [base]:
            m.close()
        oracle.close()
    print('max_abs vs oracle', worst_oracle, 'alone vs batched', worst_alone)
