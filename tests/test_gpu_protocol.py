"""Protocol v1 of the qwen_gpu process (engine/INTERFACE.md:40-90), checked
the way the reference checks its CLI: tools/check_native_cpu_interface.py
(seeded chat repeat, capacity/invalid-id error + reset at --context 3) and
tools/check_native_cpu_robustness.py (bit-identical logits across worker
settings and repeats, dump metadata)."""
import json
import subprocess

import numpy as np
import pytest

V = 151936


class Cli:
    def __init__(self, qpkg, pack, threads=12, prefill_threads=6, context=4096):
        self.p = subprocess.Popen([str(qpkg.CLI_PATH), '--weights', str(pack), '--threads', str(threads),
                                   '--prefill-threads', str(prefill_threads), '--context', str(context)],
                                  stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
        self.ready = self.read()

    def read(self):
        line = self.p.stdout.readline()
        assert line, self.p.stderr.read()
        return json.loads(line)

    def __call__(self, command):
        self.p.stdin.write(command + '\n')
        self.p.stdin.flush()
        return self.read()

    def close(self):
        if self.p.poll() is None:
            self.p.stdin.write('quit\n')
            self.p.stdin.flush()
            assert self.read() == {'ok': True}
            assert self.p.wait(timeout=30) == 0


@pytest.mark.gpu
def test_handshake_and_commands(qpkg, pack0, tmp_path):
    cli = Cli(qpkg, pack0)
    try:
        r = cli.ready
        expected = dict(ready=True, protocol=1, position=0, decode_threads=12, prefill_threads=6, context=4096,
                        lossless_bf16_decode_cache_bytes=0, gpu=True, pytorch=False, weight_precision='f16',
                        norm_precision='f32', norm_accumulator_precision='f64', activation_precision='f32',
                        kv_precision='f16', prefix_reuse=True, prefix_reuse_chunk=512, suffix_drafting=False,
                        verify_greedy_b2=True, max_verified_draft=1)
        assert r == expected
        assert cli('reset') == {'ok': True, 'position': 0}
        assert cli('mode greedy') == {'ok': True}
        first = cli('prefill 9707 11 1917')
        assert first['position'] == 3 and 0 <= first['token'] < V and first['seconds'] > 0
        dump = tmp_path / 'logits with space.f32'
        assert cli(f'dump {dump}') == {'ok': True, 'count': V, 'position': 3}
        logits = np.fromfile(dump, '<f4')
        assert logits.shape == (V,) and int(np.argmax(logits)) == first['token']
        hidden = tmp_path / 'hidden.f32'
        assert cli(f'dump-hidden {hidden}') == {'ok': True, 'count': 1024, 'position': 3, 'format': 'f32le'}
        assert np.fromfile(hidden, '<f4').shape == (1024,)
        # The C ABI on the same ids gives the same bits.
        with qpkg.Model(pack0) as m:
            m.prefill([9707, 11, 1917])
            assert np.array_equal(m.logits().view(np.uint32), logits.view(np.uint32))
            assert np.array_equal(m.hidden().view(np.uint32), np.fromfile(hidden, '<f4').view(np.uint32))
        step = cli(f'step {first["token"]}')
        assert step['position'] == 4
        assert cli('rewind 2') == {'ok': True, 'position': 2}
        again = cli('prefill 1917')
        assert again['token'] == first['token'] and again['position'] == 3
        assert cli('stats')['position'] == 3
        # verify-greedy: pending = the predicted token, draft = the model's own next prediction.
        nxt = cli(f'step {first["token"]}')
        cli('rewind 3')
        v = cli(f'verify-greedy {first["token"]} {nxt["token"]}')
        assert v['accepted'] == 1 and v['committed_inputs'] == 2 and v['verified_positions'] == 2
        assert v['tokens'][0] == nxt['token'] and v['position'] == 5 and len(v['tokens']) == 2
        bad = cli(f'verify-greedy {first["token"]} {(nxt["token"] + 1) % V}')
        assert bad['accepted'] == 0 and bad['committed_inputs'] == 1 and bad['position'] == 6
        # Errors reset everything and report position 0 (engine/main.cpp:190-193).
        for command in ('bogus', 'rewind 99', 'step', 'step 1 2', f'prefill {V}', 'mode chat', 'dump'):
            out = cli(command)
            assert 'error' in out and out['position'] == 0, (command, out)
            assert cli('stats')['position'] == 0
        cli('mode chat 7')
        out = cli('verify-greedy 1 2')
        assert 'error' in out and 'chat mode' in out['error']
    finally:
        cli.close()


@pytest.mark.gpu
def test_seeded_chat_and_capacity(qpkg, pack0):
    """tools/check_native_cpu_interface.py:28-33 and :54-63."""
    cli = Cli(qpkg, pack0)
    try:
        samples = []
        for _ in range(2):
            cli('reset')
            cli('mode chat 42')
            samples.append(cli('prefill 9707 11 1917')['token'])
        assert samples[0] == samples[1]
    finally:
        cli.close()
    commands = 'prefill 9707 11 1917\nstep 0\nstats\nprefill 151936\nstats\nprefill 9707\nquit\n'
    result = subprocess.run([str(qpkg.CLI_PATH), '--weights', str(pack0), '--threads', '2', '--prefill-threads',
                             '2', '--context', '3'], input=commands, text=True, capture_output=True, timeout=120,
                            check=True)
    rows = [json.loads(line) for line in result.stdout.splitlines()]
    assert len(rows) == 8 and rows[1]['position'] == 3
    assert 'error' in rows[2] and rows[3]['position'] == 0
    assert 'error' in rows[4] and rows[5]['position'] == 0
    assert rows[6]['position'] == 1 and rows[7] == {'ok': True}


@pytest.mark.gpu
def test_worker_settings_do_not_change_bits(qpkg, pack0, tmp_path):
    """tools/check_native_cpu_robustness.py:187-229: 1 vs 64 workers, repeats."""
    reference = None
    for workers in (1, 64):
        cli = Cli(qpkg, pack0, threads=workers, prefill_threads=workers, context=8)
        try:
            for repetition in range(2):
                cli('reset')
                cli('mode greedy')
                tokens, dumps = [], []
                for k, command in enumerate(('prefill 9707 11', 'step 1917', 'step 0')):
                    out = cli(command)
                    assert out['position'] == k + 2
                    path = tmp_path / f'w{workers}-r{repetition}-{k}.f32'
                    assert cli(f'dump {path}')['count'] == V
                    tokens.append(out['token'])
                    dumps.append(path.read_bytes())
                if reference is None:
                    reference = (tokens, dumps)
                assert (tokens, dumps) == reference
        finally:
            cli.close()
