"""Whole-model pins of the C++ oracle (CPU only).

The NumPy restatement of the reference's independent oracle
(tests/test_full_model.py:40-80; oracle/numpy_ref.py) uses BLAS FP32 sums and
its own norm, so agreement within the reference's gate (max-abs 1e-2, RMS
2e-3, greedy identity; tools/check_native_saved_oracle.py:36) at every
position pins the C++ restatement's wiring: residuals, QK-norm, RoPE, GQA
head mapping, causal KV, SwiGLU and the tied head. A dropped term or a
wrong head index moves logits by O(0.1-1), far outside the gate.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle_binding import compare_logits

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / 'oracle'))
import numpy_ref  # noqa: E402


@pytest.fixture(scope='module')
def numpy_model(pack0):
    return numpy_ref.NumpyQwen(pack0)


@pytest.fixture(scope='module')
def cpu_model(oracle_lib, pack0):
    m = oracle_lib.model(pack0, 8, 8, 64)
    yield m
    m.close()


def test_oracle_matches_numpy_restatement(cpu_model, numpy_model):
    ids = [9707, 11, 1917, 0, 151935, 42]
    cpu_model.reset()
    numpy_model.reset()
    cpu_model.prefill(ids[:3])
    for tok in ids[:2]:
        numpy_model.token(tok, logits=False)
    expected = numpy_model.token(ids[2])
    results = [compare_logits(cpu_model.logits(), expected)]
    for tok in ids[3:]:
        cpu_model.step(tok)
        results.append(compare_logits(cpu_model.logits(), numpy_model.token(tok)))
    for r in results:
        assert r['passed'], r
        # The two restatements differ only in FP32 summation order.
        assert r['max_abs'] < 5e-3


def test_oracle_prefill_equals_steps_and_truncate(cpu_model):
    """Per-row B1 arithmetic: a batched prefill equals token-by-token steps."""
    ids = [5, 6000, 151000, 77, 12, 9]
    cpu_model.reset()
    cpu_model.prefill(ids)
    batched = cpu_model.logits()
    cpu_model.reset()
    for tok in ids:
        cpu_model.step(tok)
    assert np.array_equal(cpu_model.logits().view(np.uint32), batched.view(np.uint32))
    cpu_model.truncate(3)
    assert cpu_model.position() == 3 and cpu_model.logits().size == 0 and cpu_model.hidden() is None
    cpu_model.prefill(ids[3:])
    assert np.array_equal(cpu_model.logits().view(np.uint32), batched.view(np.uint32))


def test_oracle_errors(cpu_model, oracle_lib, pack0):
    cpu_model.reset()
    for call, message in ((lambda: cpu_model.step(151936), 'Token ID out of range'),
                          (lambda: cpu_model.prefill([]), 'Empty token input'),
                          (lambda: cpu_model.prefill([1] * 65), 'Context capacity exceeded'),
                          (lambda: cpu_model.truncate(1), 'Rewind position out of range')):
        with pytest.raises(RuntimeError, match=message):
            call()
    with pytest.raises(RuntimeError, match='Threads must be in 1..64'):
        oracle_lib.model(pack0, 0, 1, 8)
    with pytest.raises(RuntimeError, match='Context must be in 1..4096'):
        oracle_lib.model(pack0, 1, 1, 4097)
