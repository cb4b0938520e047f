"""The chat-sampler oracle (oracle/sampler_ref.py) pinned on the CPU:
the C++ standard's known answer for mt19937_64, agreement with libstdc++'s
std::mt19937_64 / generate_canonical<double, 53> (a small program built with
g++ here), brute-force ordering of the candidates, and the top-p draw on
cases whose answer follows from the rule (engine/main.cpp:51-69).
"""
import shutil
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / 'oracle'))
import sampler_ref  # noqa: E402

V = sampler_ref.V


def test_mt19937_64_known_answer():
    rng = sampler_ref.MT19937_64()
    for _ in range(9999):
        rng()
    assert rng() == 9981545732273789042  # [rand.predef]: mt19937_64, 10000th value


CPP = r'''
#include <cstdio>
#include <random>
int main() {
    std::mt19937_64 a(42), b(7);
    for (int i = 0; i < 700; ++i) std::printf("%llu\n", (unsigned long long)a());
    for (int i = 0; i < 50; ++i) std::printf("%.17g\n", std::generate_canonical<double, 53>(b));
}
'''


@pytest.mark.skipif(shutil.which('g++') is None, reason='needs g++ (libstdc++)')
def test_matches_libstdcxx(tmp_path):
    src = tmp_path / 'mt.cpp'
    src.write_text(CPP)
    exe = tmp_path / 'mt'
    subprocess.run(['g++', '-O1', '-o', str(exe), str(src)], check=True)
    lines = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    a, b = sampler_ref.MT19937_64(42), sampler_ref.MT19937_64(7)
    assert [int(x) for x in lines[:700]] == [a() for _ in range(700)]  # crosses two twists
    assert [float(x) for x in lines[700:]] == [sampler_ref.canonical(b) for _ in range(50)]


def brute_top(logits, seen, k):
    s = [np.float32((np.float32(l) - np.float32(1.5 if f else 0.0)) / np.float32(0.7)) for l, f in zip(logits, seen)]
    return sorted(range(len(s)), key=lambda i: (-float(s[i]), i))[:k], s


def test_candidates_order_ties_and_signed_zero():
    rng = np.random.default_rng(3)
    logits = rng.standard_normal(V).astype(np.float32)
    logits[[10, 20, 30]] = np.float32(9.0)      # exact ties: lower id first
    logits[[40, 41]] = [np.float32(9.0 + 1.5), np.float32(9.0 + 1.5)]  # penalized down onto the tie
    seen = np.zeros(V, dtype=bool)
    seen[[41, 30]] = True
    values, ids = sampler_ref.top_candidates(logits, seen)
    s = sampler_ref.scores(logits, seen)
    expected = sorted(range(V), key=lambda i: (-float(s[i]), i))[:20]
    assert ids.tolist() == expected and np.array_equal(values, s[expected])
    zeros = np.full(64, -5.0, dtype=np.float32)
    zeros[[3, 9]] = [np.float32(-0.0), np.float32(0.0)]
    padded = np.concatenate([zeros, np.full(V - 64, -9.0, dtype=np.float32)])
    _, ids = sampler_ref.top_candidates(padded, np.zeros(V, dtype=bool), k=3)
    assert ids[:2].tolist() == [3, 9]  # -0 and +0 tie; id order decides
    small = rng.standard_normal(50).astype(np.float32)
    order, _ = brute_top(small, [i % 3 == 0 for i in range(50)], 20)
    full = np.full(V, -100.0, dtype=np.float32)
    full[:50] = small
    flags = np.zeros(V, dtype=bool)
    flags[:50:3] = True
    assert sampler_ref.top_candidates(full, flags)[1].tolist() == order


def test_draw_rules():
    rng = sampler_ref.MT19937_64(1)
    dominant = np.array([10.0] + [-30.0] * 19, dtype=np.float32)
    ids = np.arange(100, 120)
    assert all(sampler_ref.draw(dominant, ids, rng) == 100 for _ in range(20))  # prefix of one
    flat = np.zeros(20, dtype=np.float32)  # weights 1: the prefix stops at 16 of 20
    picks = {sampler_ref.draw(flat, ids, rng) for _ in range(400)}
    assert picks == set(range(100, 116))
    two = np.array([0.0, 0.0] + [-50.0] * 18, dtype=np.float32)  # 0.5 + 0.5 covers 0.8
    assert {sampler_ref.draw(two, ids, rng) for _ in range(100)} == {100, 101}
    with pytest.raises(ValueError, match='Nonfinite'):
        sampler_ref.scores(np.full(V, np.nan, dtype=np.float32), np.zeros(V, dtype=bool))
