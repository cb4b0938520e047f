"""ORACLE (test infrastructure only): restatement of the reference's chat
sampler, ``Sampler::select`` in chat mode (engine/main.cpp:40-69), for
checking the engine's device candidates and the protocol's seeded draws.

* ``MT19937_64``: the 64-bit Mersenne Twister of Matsumoto and Nishimura
  (2004) with the parameters C++ fixes for ``std::mt19937_64``
  ([rand.predef]); pinned by the standard's known answer (the 10000th output
  of a default-seeded engine is 9981545732273789042).
* ``canonical``: ``std::generate_canonical<double, 53>`` as libstdc++ computes
  it for a 64-bit engine (one draw u, double(u) / 2^64, values that round to
  1 replaced by the largest double below 1). libc++ computes it differently,
  so seeded chat draws are pinned for libstdc++ builds only.
* ``top_candidates`` / ``chat_select``: scores (logit - (seen ? 1.5 : 0)) / 0.7
  in float32, the 20 best by value descending then id ascending, softmax
  weights exp(double(s_i) - s_0), the smallest prefix holding 0.8 of their
  total (at least one), and a draw over that prefix.

Only tests/ use this module.
"""
import math

import numpy as np

V = 151936
TOP = 20
MASK64 = (1 << 64) - 1


class MT19937_64:
    N, M = 312, 156
    A = 0xB5026F5AA96619E9
    UPPER, LOWER = 0xFFFFFFFF80000000, 0x7FFFFFFF

    def __init__(self, seed=5489):
        self.seed(seed)

    def seed(self, seed):
        x = [seed & MASK64]
        for i in range(1, self.N):
            prev = x[-1]
            x.append((6364136223846793005 * (prev ^ (prev >> 62)) + i) & MASK64)
        self.state, self.index = x, self.N

    def _twist(self):
        s = self.state
        for i in range(self.N):
            y = (s[i] & self.UPPER) | (s[(i + 1) % self.N] & self.LOWER)
            s[i] = s[(i + self.M) % self.N] ^ (y >> 1) ^ (self.A if y & 1 else 0)
        self.index = 0

    def __call__(self):
        if self.index >= self.N:
            self._twist()
        y = self.state[self.index]
        self.index += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        return y & MASK64


def canonical(rng):
    value = float(rng()) / 18446744073709551616.0
    return value if value < 1.0 else math.nextafter(1.0, 0.0)


def scores(logits, seen):
    """float32 (logit - (seen ? 1.5 : 0)) / 0.7 for every id."""
    logits = np.asarray(logits, dtype=np.float32)
    if logits.shape != (V,):
        raise ValueError('No current full-vocabulary logits')
    if not np.isfinite(logits).all():
        raise ValueError('Nonfinite model logits')
    penalty = np.where(np.asarray(seen, dtype=bool), np.float32(1.5), np.float32(0.0))
    return (logits - penalty) / np.float32(0.7)


def top_candidates(logits, seen, k=TOP):
    """(values, ids) of the k best scores, value descending then id ascending."""
    s = scores(logits, seen)
    order = np.lexsort((np.arange(V), -s))[:k]
    return s[order], order.astype(np.int32)


def draw(values, ids, rng):
    """The top-p draw over the candidates (engine/main.cpp:62-68)."""
    probabilities, total = [], 0.0
    for v in values:
        p = math.exp(float(v) - float(values[0]))
        probabilities.append(p)
        total += p
    retained, count = 0.0, 0
    while True:
        retained += probabilities[count]
        count += 1
        if not (count < len(values) and retained < 0.8 * total):
            break
    d = canonical(rng) * retained
    for i in range(count):
        d -= probabilities[i]
        if d < 0:
            return int(ids[i])
    return int(ids[count - 1])


def chat_select(logits, seen, rng):
    values, ids = top_candidates(logits, seen)
    return draw(values, ids, rng)
