"""Device chat sampler (engine/main.cpp:40-69) against the oracle's
restatement (oracle/sampler_ref.py): the GPU candidates (top scores with the
presence penalty, value descending then id ascending) must equal the
oracle's bit for bit, and the protocol's seeded chat draws, replayed by the
oracle from the logits the process dumps, must pick the same tokens."""
import sys
from pathlib import Path

import numpy as np
import pytest

from test_gpu_protocol import Cli

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / 'oracle'))
import sampler_ref  # noqa: E402

V = sampler_ref.V


@pytest.fixture(scope='module')
def model(qpkg, pack0):
    m = qpkg.Model(pack0, context=4096)
    yield m
    m.close()


@pytest.mark.gpu
def test_top_scores_match_oracle(model):
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, V, 40).tolist()
    model.reset()
    model.update_penalized(clear=True)
    model.prefill(prompt)
    seen = np.zeros(V, dtype=bool)
    for penalty, temperature, k in ((1.5, 0.7, 20), (0.0, 1.0, 32), (3.0, 0.25, 1)):
        values, ids = model.top_scores(penalty, temperature, k)
        s = (model.logits() - np.where(seen, np.float32(penalty), np.float32(0))) / np.float32(temperature)
        order = np.lexsort((np.arange(V), -s))[:k]
        assert ids.tolist() == order.tolist()
        assert np.array_equal(values.view(np.uint32), s[order].view(np.uint32))
    # Penalize the prompt and this step's best candidates, as the sampler
    # does with consumed ids, and compare with the oracle's candidates.
    model.update_penalized(prompt)
    seen[prompt] = True
    for step in range(4):
        values, ids = model.top_scores()
        ref_values, ref_ids = sampler_ref.top_candidates(model.logits(), seen)
        assert ids.tolist() == ref_ids.tolist()
        assert np.array_equal(values.view(np.uint32), ref_values.view(np.uint32))
        token = int(ids[step % 3])
        model.update_penalized([token])
        seen[token] = True
        model.step(token)
    model.update_penalized(clear=True)
    values, ids = model.top_scores()
    ref_values, ref_ids = sampler_ref.top_candidates(model.logits(), np.zeros(V, dtype=bool))
    assert ids.tolist() == ref_ids.tolist() and np.array_equal(values, ref_values)


@pytest.mark.gpu
def test_top_scores_errors(qpkg, pack0):
    m = qpkg.Model(pack0, context=16)
    try:
        with pytest.raises(RuntimeError, match='No current full-vocabulary logits'):
            m.top_scores()
        m.prefill([1, 2, 3])
        for kwargs, message in ((dict(k=0), 'k must be 1..32'), (dict(k=33), 'k must be 1..32'),
                                (dict(temperature=0.0), 'temperature positive'),
                                (dict(penalty=float('nan')), 'must be finite')):
            with pytest.raises(RuntimeError, match=message):
                m.top_scores(**kwargs)
        for bad in ([V], [-1]):
            with pytest.raises(RuntimeError, match='Token ID out of range'):
                m.update_penalized(bad)
        assert m.top_scores(k=5)[1].size == 5
    finally:
        m.close()


@pytest.mark.gpu
def test_protocol_chat_draws_match_oracle(qpkg, pack0, tmp_path):
    """Seeded chat through the process: every sampled token equals the
    oracle's draw over the dumped logits, with the presence set following
    consumed ids across prefill, step, rewind and reset."""
    cli = Cli(qpkg, pack0)
    rng_ids = np.random.default_rng(12)
    try:
        for seed in (42, 7):
            cli('reset')
            assert cli(f'mode chat {seed}') == {'ok': True}
            rng = sampler_ref.MT19937_64(seed)
            history = []

            def check(command, ids):
                out = cli(command)
                history.extend(ids)
                dump = tmp_path / 'logits.f32'
                assert cli(f'dump {dump}')['count'] == V
                logits = np.fromfile(dump, dtype=np.float32)
                seen = np.zeros(V, dtype=bool)
                seen[history] = True
                assert out['token'] == sampler_ref.chat_select(logits, seen, rng), command
                return out['token']

            prompt = rng_ids.integers(0, V, 30).tolist()
            token = check('prefill ' + ' '.join(map(str, prompt)), prompt)
            for _ in range(6):
                token = check(f'step {token}', [token])
            assert cli('rewind 20')['position'] == 20
            del history[20:]
            tail = rng_ids.integers(0, V, 5).tolist()
            token = check('prefill ' + ' '.join(map(str, tail)), tail)
            check(f'step {token}', [token])
    finally:
        cli.close()
