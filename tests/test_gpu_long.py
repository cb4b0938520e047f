"""Long-context decode parity (the 3968-token workload, seed 3).

Decode attention runs inside one kernel per layer with the QKV and O
projections. Up to 256 cached positions every workgroup attends its query
head over all positions in 64-position passes (FULL form, 1 to 4 passes);
beyond, the 32 workgroups of a KV head each take passes s and s + 32 and
merge their (output, max, sum) partials in a fixed order. These tests cover
every pass count of the FULL form, the switch to the split form (256 -> 257
positions), many passes, the capacity limit and the 512-row prefill chunk
boundaries against the oracle's sequential softmax
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
def test_full_form_passes_and_split_switch_match_oracle(qpkg, pack0, oracle_lib):
    """Steps at n = 125 .. 264 cached positions: the FULL form with 2, 3 and 4
    passes (switches at 129 and 193 positions), then the split form from 257
    on; every row against the oracle."""
    gpu = qpkg.Model(pack0, context=4096)
    oracle = oracle_lib.model(pack0, 16, 16, 4096)
    try:
        results = check_trajectory(gpu, oracle, PROMPTS['long_3968'][:124], 141)
        assert gpu.position() == 264
        print('max_abs', max(r['max_abs'] for r in results), 'rms', max(r['rms'] for r in results))
    finally:
        gpu.close()
        oracle.close()


@pytest.mark.gpu
def test_fused_to_split_attention_matches_oracle(qpkg, pack0, oracle_lib):
    # Steps at n = 506 .. 517 cached positions (the split form, 8 passes; the
    # separate kernels' switch from attention + O to split + merge at 512/513).
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
def test_context_3968_decode_to_capacity_matches_oracle(qpkg, pack0, oracle_lib):
    """The long-context workload end to end: the 3968-token prompt, then 128
    greedy steps over positions 3968..4095 (up to 32 position splits per KV
    head), every one of the 129 logit rows gated against the oracle
    teacher-forced (tools/check_native_logits.py samples such rows; here all
    are taken). The cache is then full: a further step is rejected."""
    gpu = qpkg.Model(pack0, context=4096)
    oracle = oracle_lib.model(pack0, 16, 16, 4096)
    try:
        results = check_trajectory(gpu, oracle, PROMPTS['long_3968'], 129)
        assert gpu.position() == 4096
        print('max_abs', max(r['max_abs'] for r in results), 'rms', max(r['rms'] for r in results))
        with pytest.raises(RuntimeError, match='Context capacity exceeded'):
            gpu.step(0)
        assert gpu.position() == 4096 and np.isfinite(gpu.logits()).all()
    finally:
        gpu.close()
        oracle.close()


@pytest.mark.gpu
def test_chunk_boundary_prompts_match_oracle(qpkg, pack0, oracle_lib):
    """Prompts of 511, 512 and 513 tokens (one batched pass short of, at, and
    one row past the 512-token chunk, the last row then taking the batch-1
    path as engine/core.cpp:712 splits it) and of 1024 / 1025 tokens, each
    prefilled in one call and gated against the oracle at the same position,
    then 2 greedy steps after the 513- and 1025-token prompts."""
    prompt = PROMPTS['prefill_1024'] + PROMPTS['long_3968'][:1]
    gpu = qpkg.Model(pack0, context=4096)
    oracle = oracle_lib.model(pack0, 16, 16, 4096)
    try:
        for start, lengths in ((510, (511, 512, 513)), (1023, (1024, 1025))):
            oracle.reset()
            oracle.prefill(prompt[:start])
            for n in lengths:
                oracle.step(prompt[n - 1])
                gpu.reset()
                gpu.prefill(prompt[:n])
                assert gpu.position() == n
                result = compare_logits(gpu.logits(), oracle.logits())
                assert result['passed'], (n, result)
            for _ in range(2):
                token = gpu.greedy()
                gpu.step(token)
                oracle.step(token)
                result = compare_logits(gpu.logits(), oracle.logits())
                assert result['passed'], (gpu.position(), result)
    finally:
        gpu.close()
        oracle.close()
