"""Whole-model parity and lifecycle invariants of the GPU engine.

Parity follows the reference's oracle pipeline (tools/check_native_logits.py):
the GPU trajectory's consumed ids are replayed through the oracle and every
position's full-vocabulary logits must pass max-abs 1e-2, RMS 2e-3 and greedy
identity (tools/check_native_saved_oracle.py:36). Lifecycle invariants follow
tools/native_verify_check.cpp and tools/check_native_cpu_robustness.py:
bit-identical repeats, verify == two steps, validation before mutation.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle_binding import compare_logits

PROMPTS = json.loads((Path(__file__).parent / 'golden' / 'prompts.json').read_text())
V = 151936


@pytest.fixture(scope='module')
def gpu_model(qpkg, pack0):
    model = qpkg.Model(pack0, context=4096)
    yield model
    model.close()


@pytest.fixture(scope='module')
def oracle_model(oracle_lib, pack0):
    model = oracle_lib.model(pack0, 16, 16, 4096)
    yield model
    model.close()


def greedy_trajectory(model, prompt, steps):
    model.reset()
    model.prefill(prompt)
    rows = []
    token = model.greedy()
    rows.append((model.logits(), token))
    for _ in range(steps - 1):
        model.step(token)
        token = model.greedy()
        rows.append((model.logits(), token))
    return rows


@pytest.mark.gpu
def test_decode_85_matches_oracle(gpu_model, oracle_model):
    """85-token prompt (seed 0) + 32 greedy tokens: every position in the gate."""
    prompt = PROMPTS['decode_85']
    rows = greedy_trajectory(gpu_model, prompt, 32)
    assert gpu_model.position() == 85 + 31
    oracle_model.reset()
    oracle_model.prefill(prompt)
    worst = dict(max_abs=0.0, rms=0.0)
    for i, (logits, token) in enumerate(rows):
        if i:
            oracle_model.step(rows[i - 1][1])
        assert token == int(np.argmax(logits)), 'device greedy disagrees with the logits'
        result = compare_logits(logits, oracle_model.logits())
        worst = dict(max_abs=max(worst['max_abs'], result['max_abs']), rms=max(worst['rms'], result['rms']))
        assert result['passed'], (i, result)
    print('worst', worst)


@pytest.mark.gpu
def test_repeat_is_bit_identical(gpu_model):
    prompt = PROMPTS['decode_85'][:20]
    a = greedy_trajectory(gpu_model, prompt, 4)
    b = greedy_trajectory(gpu_model, prompt, 4)
    for (la, ta), (lb, tb) in zip(a, b):
        assert ta == tb
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize('switch', ['QWEN_HIP_FUSED_FFN', 'QWEN_HIP_FUSED_ATTENTION'])
def test_fused_kernels_match_separate_kernels(qpkg, pack0, gpu_model, monkeypatch, switch):
    """The step's two fused kernels against the separate kernels they
    replace. QWEN_HIP_FUSED_FFN=0: norm+gate/up, then down as the reference's
    dot over all 3072 columns, instead of 8 column slices added by the next
    layer. QWEN_HIP_FUSED_ATTENTION=0: the QKV kernel and the fused (up to 512
    positions) or split + merge attention kernels, instead of one kernel whose
    workgroups attend over 64-position passes and merge their partials. Along
    greedy trajectories after the 85-, 200-, 1100- and 3000-token prompts
    (the 200-token one crosses from 3 to 4 passes of the FULL form and on to
    the split form at 257 positions) both paths choose the same tokens and their logits
    agree to 1e-4: the different summation orders move outputs by a few FP32
    ulps, nothing more (a wrong slice, row, head, pass or fold moves them by
    ~1e-1)."""
    monkeypatch.setenv(switch, '0')
    plain = qpkg.Model(pack0, context=4096)
    monkeypatch.delenv(switch)
    try:
        for prompt, steps in ((PROMPTS['decode_85'], 12), (PROMPTS['long_3968'][:190], 70),
                              (PROMPTS['long_3968'][:1100], 12), (PROMPTS['long_3968'][:3000], 12)):
            fused_rows = greedy_trajectory(gpu_model, prompt, steps)
            plain_rows = greedy_trajectory(plain, prompt, steps)
            worst = 0.0
            for (lf, tf), (lp, tp) in zip(fused_rows, plain_rows):
                assert tf == tp
                worst = max(worst, float(np.max(np.abs(lf - lp))))
            print(f'{switch}=0, prompt {len(prompt)}: max |d logit| against the fused kernels {worst:.3e}')
            assert worst <= 1e-4
    finally:
        plain.close()


@pytest.mark.gpu
def test_token_kernel_equals_two_kernel_path(qpkg, pack0, gpu_model, monkeypatch):
    """The one-launch step (all 28 layers in one persistent kernel, weights
    streamed into LDS a layer ahead, residual folds across XCDs inside the
    launch) against the two fused kernels per layer it replaces
    (QWEN_HIP_TOKEN_KERNEL=0): the same dots, norms, folds and attention
    order, so the logits of every step must be bit-identical. Contexts cover
    the FULL attention form with 1, 2, 3 and 4 passes and the split form with
    one and two passes per workgroup."""
    monkeypatch.setenv('QWEN_HIP_TOKEN_KERNEL', '0')
    plain = qpkg.Model(pack0, context=4096)
    monkeypatch.delenv('QWEN_HIP_TOKEN_KERNEL')
    try:
        assert gpu_model.decode_kernels() == 2 and plain.decode_kernels() == 1
        for length in (20, 85, 150, 200, 300, 2100, 3000):
            prompt = (PROMPTS['decode_85'] if length <= 85 else PROMPTS['long_3968'])[:length]
            fused_rows = greedy_trajectory(gpu_model, prompt, 3)
            plain_rows = greedy_trajectory(plain, prompt, 3)
            for (lt, tt), (lp, tp) in zip(fused_rows, plain_rows):
                assert tt == tp
                assert np.array_equal(lt.view(np.uint32), lp.view(np.uint32)), length
    finally:
        plain.close()


@pytest.mark.gpu
def test_stalled_step_is_reported_and_rolled_back(qpkg, pack0, monkeypatch):
    """A decode launch whose exchange cannot complete fails cleanly instead
    of hanging. A test-only knob makes workgroup 5 withhold its q/k/v rows in
    layer 0 of the next launch, and a short poll limit (2048 rounds) makes
    the workgroups waiting for them give up; their give-up raises the step's
    stall word, which ends every other workgroup's polls, so the launch
    exits. The step raises 'Decode step stalled' and leaves the model at its
    position before the call, without logits; the next step (the knob acts
    once) is bit-identical to the same step on a clean model, and so are the
    steps after it (engine/core.cpp:740; engine/main.cpp:190-193)."""
    monkeypatch.setenv('QWEN_HIP_TEST_WITHHOLD', '5')
    monkeypatch.setenv('QWEN_HIP_TEST_SPINS', '2048')
    m = qpkg.Model(pack0, context=512)
    monkeypatch.delenv('QWEN_HIP_TEST_WITHHOLD')
    monkeypatch.delenv('QWEN_HIP_TEST_SPINS')
    clean = qpkg.Model(pack0, context=512)
    try:
        assert m.decode_kernels() == 2
        prompt = PROMPTS['decode_85'][:40]
        m.prefill(prompt)
        clean.prefill(prompt)
        token = clean.greedy()
        with pytest.raises(RuntimeError, match='Decode step stalled'):
            m.step(token)
        assert m.position() == 40 and m.logits().size == 0
        for _ in range(3):
            m.step(token)
            clean.step(token)
            assert np.array_equal(m.logits().view(np.uint32), clean.logits().view(np.uint32))
            token = clean.greedy()
    finally:
        m.close()
        clean.close()


@pytest.mark.gpu
def test_separate_kernels_when_placement_cannot_be_assumed(qpkg, pack0, gpu_model, tmp_path):
    """When the placement probe fails (forced here in a fresh process) the
    engine runs the separate kernels, which exchange nothing inside a launch:
    the same greedy tokens and logits within 1e-4 of the one-launch step, and
    the batched step, which needs the placement, is refused."""
    import os
    import subprocess
    import sys
    out = tmp_path / 'logits.npy'
    code = f"""
import sys, numpy as np
sys.path.insert(0, {str(Path(__file__).parent)!r})
from conftest import load_package
q = load_package()
m = q.Model({str(pack0)!r}, context=512)
assert m.decode_kernels() == 0, m.decode_kernels()
m.prefill({PROMPTS['decode_85'][:60]!r})
rows = [m.logits()]
for _ in range(3):
    m.step(m.greedy())
    rows.append(m.logits())
np.save({str(out)!r}, np.stack(rows))
b = m.share()
try:
    q.step_batch([m, b], [1, 2])
except RuntimeError as error:
    assert 'round-robin' in str(error), error
else:
    raise AssertionError('batched step ran without the placement')
print('separate kernels ok', flush=True)
"""
    env = {**os.environ, 'QWEN_HIP_ASSUME_NO_PLACEMENT': '1'}
    subprocess.run([sys.executable, '-c', code], env=env, check=True, timeout=300)
    separate = np.load(out)
    rows = greedy_trajectory(gpu_model, PROMPTS['decode_85'][:60], 4)
    for (logits, _), other in zip(rows, separate):
        assert int(np.argmax(logits)) == int(np.argmax(other))
        assert float(np.max(np.abs(logits - other))) <= 1e-4


@pytest.mark.gpu
def test_models_stepped_from_two_threads(qpkg, pack0):
    """Two independent models (own weights, caches and streams) decoding at
    the same time from two host threads: the library runs their decode
    launches one after another (each needs every CU), so no step stalls and
    each trajectory is bit-identical to the same model run alone."""
    import threading
    prompt = PROMPTS['decode_85']
    models = [qpkg.Model(pack0, context=512) for _ in range(2)]
    try:
        lengths = (40, 60)
        expected = [greedy_trajectory(m, prompt[:n], 30) for m, n in zip(models, lengths)]
        got, errors = [None, None], []

        def run(i):
            try:
                got[i] = greedy_trajectory(models[i], prompt[:lengths[i]], 30)
            except Exception as error:  # reported by the main thread
                errors.append(error)

        threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=100)
        assert not any(t.is_alive() for t in threads), 'a decode thread did not finish'
        assert not errors, errors
        for exp, rows in zip(expected, got):
            for (le, te), (lg, tg) in zip(exp, rows):
                assert te == tg
                assert np.array_equal(le.view(np.uint32), lg.view(np.uint32))
    finally:
        for m in models:
            m.close()


@pytest.mark.gpu
def test_prefill_equals_steps_and_truncate(gpu_model):
    """Token-at-a-time equivalence and rewind: KV before the cut is retained."""
    prompt = PROMPTS['decode_85'][:12]
    gpu_model.reset()
    gpu_model.prefill(prompt)
    full = gpu_model.logits()
    gpu_model.truncate(7)
    assert gpu_model.position() == 7 and gpu_model.logits().size == 0
    with pytest.raises(RuntimeError, match='No current hidden state'):
        gpu_model.hidden()
    gpu_model.prefill(prompt[7:])
    assert np.array_equal(gpu_model.logits().view(np.uint32), full.view(np.uint32))


VERIFY_IDS = [32 + (i * 37) % 1000 for i in range(700)]


class OraclePrefix:
    """One oracle model walked to prefixes of VERIFY_IDS: rows below the
    reached prefix always hold those ids, so a test may step past it and a
    later test truncate back or extend forward."""

    def __init__(self, oracle):
        self.oracle, self.valid = oracle, 0
        oracle.reset()

    def at(self, n):
        if n > self.valid:
            self.oracle.truncate(self.valid)
            self.oracle.prefill(VERIFY_IDS[self.valid:n])
        else:
            self.oracle.truncate(n)
        self.valid = n  # the caller's steps overwrite rows from n on
        return self.oracle


@pytest.fixture(scope='module')
def oracle_prefix(oracle_lib, pack0):
    model = oracle_lib.model(pack0, 16, 16, 4096)
    yield OraclePrefix(model)
    model.close()


@pytest.mark.gpu
# Prefixes cover the two-row launch of the token kernel (fused attention:
# 0, 1, 62, 63 where row 1 needs one more 64-position pass than row 0, 254
# with both rows at the fused limit of 256 positions; split attention: 510,
# 511, 513, 700) and the two-step fallback (255: row 0 fused, row 1 split).
@pytest.mark.parametrize('prefix,commit', [(0, 1), (0, 2), (1, 1), (1, 2), (62, 2), (63, 1), (254, 2), (255, 1),
                                           (510, 2), (511, 2), (513, 2), (700, 1)])
def test_verify_two_equals_two_steps(qpkg, pack0, gpu_model, oracle_prefix, prefix, commit):
    """tools/native_verify_check.cpp normal_case, against a second model:
    every row bit-identical to single steps; and both rows (logits and
    hidden) against the oracle's two steps (engine/core.cpp:729-752) under
    the reference gate."""
    ids = VERIFY_IDS[:prefix]
    ref = qpkg.Model(pack0, context=4096)
    try:
        for m in (gpu_model, ref):
            m.reset()
            if prefix:
                m.prefill(ids)
        base_logits = gpu_model.logits()
        for bad in ((-1, 11), (9707, V)):
            with pytest.raises(RuntimeError, match='Token ID out of range'):
                gpu_model.verify_two(*bad)
        with pytest.raises(RuntimeError, match='No verification pending'):
            gpu_model.commit_verified(1)
        rows = gpu_model.verify_two(9707, 11)
        assert rows.base_position == prefix and rows.logits.shape == (2, V) and rows.hidden.shape == (2, 1024)
        assert gpu_model.position() == prefix
        assert np.array_equal(gpu_model.logits().view(np.uint32), base_logits.view(np.uint32))
        ref.step(9707)
        first = (ref.logits(), ref.hidden())
        ref.step(11)
        second = (ref.logits(), ref.hidden())
        for row, (l, h) in enumerate((first, second)):
            assert np.array_equal(rows.logits[row].view(np.uint32), l.view(np.uint32))
            assert np.array_equal(rows.hidden[row].view(np.uint32), h.view(np.uint32))
        oracle = oracle_prefix.at(prefix)
        for row, token in enumerate((9707, 11)):
            oracle.step(token)
            result = compare_logits(rows.logits[row], oracle.logits())
            assert result['passed'], (prefix, row, result)
            hidden_err = float(np.abs(rows.hidden[row] - oracle.hidden()).max())
            assert hidden_err <= 1e-2, (prefix, row, hidden_err)
        assert gpu_model.verify_greedy() == (int(np.argmax(first[0])), int(np.argmax(second[0])))
        for blocked in (lambda: gpu_model.step(12), lambda: gpu_model.prefill([12])):
            with pytest.raises(RuntimeError, match='Commit or discard pending verification'):
                blocked()
        with pytest.raises(RuntimeError, match='Verification already pending'):
            gpu_model.verify_two(12, 13)
        for count in (-1, 0, 3):
            with pytest.raises(RuntimeError, match='Commit count must be one or two'):
                gpu_model.commit_verified(count)
        gpu_model.commit_verified(commit)
        expected = first if commit == 1 else second
        assert gpu_model.position() == prefix + commit
        assert np.array_equal(gpu_model.logits().view(np.uint32), expected[0].view(np.uint32))
        assert np.array_equal(gpu_model.hidden().view(np.uint32), expected[1].view(np.uint32))
        if commit == 1:
            ref.truncate(prefix + 1)
        gpu_model.step(42)
        ref.step(42)
        assert np.array_equal(gpu_model.logits().view(np.uint32), ref.logits().view(np.uint32))
    finally:
        ref.close()


@pytest.mark.gpu
@pytest.mark.parametrize('prefix', [5, 511, 600])
def test_verify_two_greedy_matches_rows(qpkg, pack0, gpu_model, prefix):
    """The no-host-copy verification selects what verify_two's rows give and
    leaves the same pending state."""
    ids = [100 + (i * 53) % 5000 for i in range(prefix)]
    gpu_model.reset()
    gpu_model.prefill(ids)
    rows = gpu_model.verify_two(77, 78)
    expected = (int(np.argmax(rows.logits[0])), int(np.argmax(rows.logits[1])))
    gpu_model.commit_verified(2)
    after = gpu_model.logits()
    gpu_model.truncate(prefix)  # same cache contents, no current logits
    assert gpu_model.verify_two_greedy(77, 78) == expected
    with pytest.raises(RuntimeError, match='Verification already pending'):
        gpu_model.verify_two_greedy(77, 78)
    gpu_model.commit_verified(2)
    assert gpu_model.position() == prefix + 2
    assert np.array_equal(gpu_model.logits().view(np.uint32), after.view(np.uint32))


@pytest.mark.gpu
def test_validation_before_mutation(qpkg, pack0):
    """Capacity/id/range errors leave state unchanged (engine/core.cpp:707-732)."""
    m = qpkg.Model(pack0, context=4)
    try:
        m.prefill([1, 2, 3])
        before = m.logits()
        for call, message in ((lambda: m.prefill([4, 5]), 'Context capacity exceeded'),
                              (lambda: m.step(V), 'Token ID out of range'),
                              (lambda: m.step(-1), 'Token ID out of range'),
                              (lambda: m.prefill([]), 'Empty token input'),
                              (lambda: m.truncate(4), 'Rewind position out of range'),
                              (lambda: m.truncate(-1), 'Rewind position out of range'),
                              (lambda: m.verify_two(1, 2), 'Context capacity exceeded')):
            with pytest.raises(RuntimeError, match=message):
                call()
            assert m.position() == 3
            assert np.array_equal(m.logits().view(np.uint32), before.view(np.uint32))
        m.step(4)
        assert m.position() == 4
        with pytest.raises(RuntimeError, match='Context capacity exceeded'):
            m.step(5)
    finally:
        m.close()
