"""Long-context decode parity (the 3968-token workload, seed 3).

Up to 512 cached positions decode attention runs fused with the O
projection (one workgroup per KV head and block of O rows, partial
projections folded into the residual stream by the next kernels); beyond
that it splits the positions into up to 32 chunks of 128 whose partial
softmax statistics a merge kernel combines before the O projection. These tests
cover the switch between the two paths, many splits and the 512-row prefill
chunk boundaries against the oracle's sequential softmax
(engine/core.cpp:606-624), teacher-forced like tools/check_native_logits.py,
under the gate of tools/check_native_saved_oracle.py:36.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle_binding import compare_logits

PROMPTS = json.loads((Path(__file__).parent / 'golden' / 'prompts.json').read_text())


def check_trajectory(gpu, oracle, prompt, steps):
    gpu.reset()
    gpu.prefill(prompt)
    oracle.reset()
    oracle.prefill(prompt)
    results = []
    for i in range(steps):
        logits = gpu.logits()
        token = gpu.greedy()
        result = compare_logits(logits, oracle.logits())
        results.append(result)
        assert result['passed'], (len(prompt) + i, result)
        if i + 1 < steps:
            gpu.step(token)
            oracle.step(token)
    return results


@pytest.mark.gpu
def test_fused_to_split_attention_matches_oracle(qpkg, pack0, oracle_lib):
    # Steps at n = 506 .. 517 cached positions: fused attention + O up to 512,
    # split attention with the O-prologue merge from 513 on.
    gpu = qpkg.Model(pack0, context=4096)
    oracle = oracle_lib.model(pack0, 16, 16, 4096)
    try:
        results = check_trajectory(gpu, oracle, PROMPTS['long_3968'][:505], 13)
        print('max_abs', max(r['max_abs'] for r in results), 'rms', max(r['rms'] for r in results))
    finally:
        gpu.close()
        oracle.close()


@pytest.mark.gpu
def test_context_1100_matches_oracle(qpkg, pack0, oracle_lib):
    gpu = qpkg.Model(pack0, context=4096)
    oracle = oracle_lib.model(pack0, 16, 16, 4096)
    try:
        results = check_trajectory(gpu, oracle, PROMPTS['long_3968'][:1100], 4)
        print('max_abs', max(r['max_abs'] for r in results), 'rms', max(r['rms'] for r in results))
    finally:
        gpu.close()
        oracle.close()


@pytest.mark.gpu
def test_context_3968_matches_oracle(qpkg, pack0, oracle_lib):
    gpu = qpkg.Model(pack0, context=4096)
    oracle = oracle_lib.model(pack0, 16, 16, 4096)
    try:
        results = check_trajectory(gpu, oracle, PROMPTS['long_3968'], 6)
        print('max_abs', max(r['max_abs'] for r in results), 'rms', max(r['rms'] for r in results))
        # Fill the cache to its last slot: capacity then rejects a further step.
        gpu.reset()
        gpu.prefill(PROMPTS['long_3968'])
        gpu.prefill(list(range(128)))
        assert gpu.position() == 4096 and np.isfinite(gpu.logits()).all()
        with pytest.raises(RuntimeError, match='Context capacity exceeded'):
            gpu.step(0)
    finally:
        gpu.close()
        oracle.close()
