"""Writes the committed input fixtures of the benchmark workloads.

prompts.json: token ids drawn uniformly from [0, 151936) with
numpy.random.default_rng(seed).integers, one stream per workload:
  decode_85     85 ids, seed 0  (85-token prompt, 32 greedy steps)
  prefill_1024  1024 ids, seed 2 (batched prefill)
  long_3968     3968 ids, seed 3 (long-context decode)
  prefix_512 + suffix_1536[8]: seed 4, prefix first, then the 8 suffixes in order.
pack_seed0.json: size and sha256 of the seed-0 QWCPU01 pack written by
write_random_pack (so a change of the generator is noticed).
Run: python tests/golden/make_fixtures.py [--pack PATH]
"""
import argparse
import hashlib
import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
VOCABULARY = 151936


def prompts():
    out = {}
    out['decode_85'] = np.random.default_rng(0).integers(0, VOCABULARY, 85).tolist()
    out['prefill_1024'] = np.random.default_rng(2).integers(0, VOCABULARY, 1024).tolist()
    out['long_3968'] = np.random.default_rng(3).integers(0, VOCABULARY, 3968).tolist()
    rng = np.random.default_rng(4)
    out['prefix_512'] = rng.integers(0, VOCABULARY, 512).tolist()
    out['suffix_1536'] = [rng.integers(0, VOCABULARY, 1536).tolist() for _ in range(8)]
    return out


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument('--pack', type=Path, help='seed-0 pack to digest')
    args = parser.parse_args()
    (HERE / 'prompts.json').write_text(json.dumps(prompts(), separators=(',', ':')) + '\n')
    if args.pack:
        digest = hashlib.sha256()
        with args.pack.open('rb') as f:
            for block in iter(lambda: f.read(1 << 24), b''):
                digest.update(block)
        (HERE / 'pack_seed0.json').write_text(json.dumps(dict(
            seed=0, stddev=0.02, bytes=args.pack.stat().st_size, sha256=digest.hexdigest()), indent=2) + '\n')


if __name__ == '__main__':
    main()
