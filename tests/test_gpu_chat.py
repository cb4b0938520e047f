"""The chat client of the engine process (fpga-qwen_amd/gpu_chat.py).

CPU cases drive the client's real start/command/stream code against a
scripted transport that answers like the engine would (no inference):
protocol transactions, token accounting, reuse bookkeeping and the drafter.
GPU cases run the real engine process: greedy tokens equal the library's,
and a cancellation while a command is in flight ends and reaps the process,
after which a restarted process answers again
(tools/check_native_cpu_interface.py:36-57).

The transaction rules are the reference adapter's contract
(tools/native_cpu_chat.py:144-304; regression cases of
tests/test_native_suffix_adapter.py): only committed inputs are consumed,
EOS is never consumed, rewinds keep whole 512-token chunks of an earlier
prompt prefill only, and any violation closes the process.
"""
import importlib.util
import json
import os
import threading
from pathlib import Path
from types import SimpleNamespace

import pytest

ROOT = Path(__file__).resolve().parents[1]
spec = importlib.util.spec_from_file_location('gpu_chat', ROOT / 'fpga-qwen_amd' / 'gpu_chat.py')
gpu_chat = importlib.util.module_from_spec(spec)
spec.loader.exec_module(gpu_chat)
PROMPTS = json.loads((Path(__file__).parent / 'golden' / 'prompts.json').read_text())
TEXT = SimpleNamespace(tokenizer=SimpleNamespace(decode=lambda ids, **kw: str(ids)))


class ScriptedLink:
    """Stands in for the engine process: prefill answers token 8, step its
    input + 1, verify-greedy the scripted row."""

    def __init__(self, log, verification=None, capable=True):
        self.log, self.verification, self.capable = log, verification, capable
        self.position, self.open = 0, True

    def alive(self):
        return self.open

    def receive(self, cancel, timeout):  # the handshake
        return dict(gpu_chat.HANDSHAKE, decode_threads=12, prefill_threads=6, prefix_reuse=True,
                    prefix_reuse_chunk=512, verify_greedy_b2=self.capable, max_verified_draft=1)

    def exchange(self, line, cancel, timeout=None):
        self.log.append(line)
        op, *args = line.split()
        if op == 'reset':
            self.position = 0
            return dict(ok=True, position=0)
        if op == 'rewind':
            self.position = int(args[0])
            return dict(ok=True, position=self.position)
        if op == 'mode':
            return dict(ok=True)
        if op == 'prefill':
            self.position += len(args)
            return dict(token=8, position=self.position)
        if op == 'step':
            self.position += 1
            return dict(token=int(args[0]) + 1, position=self.position)
        if op == 'verify-greedy':
            row = dict(self.verification)
            self.position += row['committed_inputs']
            row.setdefault('position', self.position)
            row.setdefault('verified_positions', 2)
            row.setdefault('finish_reason', 'eos' if row['tokens'][-1] in gpu_chat.EOS else None)
            return row
        raise AssertionError(line)

    def shutdown(self):
        self.open = False


@pytest.fixture
def pack_files(tmp_path):
    """Files the client checks before starting (a stub binary and pack)."""
    binary = tmp_path / 'qwen_gpu'
    binary.write_text('#!/bin/sh\n')
    binary.chmod(0o755)
    weights = tmp_path / 'weights.bin'
    for p in (weights, Path(f'{weights}.index')):
        p.write_bytes(b'')
    Path(f'{weights}.manifest.json').write_text(json.dumps(dict(format='QWCPU01', completed=True)))
    return binary, weights


def scripted(pack_files, verification=None, capable=True, **kwargs):
    calls, links = [], []

    def factory():
        links.append(ScriptedLink(calls, verification, capable))
        return links[-1]

    adapter = gpu_chat.GPUChatAdapter(TEXT, binary=pack_files[0], weights=pack_files[1], link_factory=factory,
                                      **kwargs)
    adapter.calls, adapter.links = calls, links
    return adapter


def request(ids=(7, 8, 9, 7), max_new=3, max_draft=1, decoding='greedy', session='s'):
    return SimpleNamespace(ids=list(ids), max_new=max_new, max_draft=max_draft, decoding=decoding,
                           session=session, seed=42)


def run(adapter, req=None, cancel=None):
    return list(adapter.stream(req or request(), cancel or threading.Event()))


def reference_rule(context, count, min_match=2, max_match=12, history=()):
    """The drafting rule written out as a brute-force search over all
    occurrences (tools/suffix.py:4-29 states it): longest tail first, the
    context before the history (newest first), the occurrence nearest the
    end that has a following token."""
    context = list(context)
    for n in range(min(max_match, len(context)), min_match - 1, -1):
        tail = context[-n:]
        for seq in [context] + [list(h) for h in reversed(history)]:
            hits = [s for s in range(len(seq) - n) if seq[s:s + n] == tail]
            if hits:
                return seq[max(hits) + n:max(hits) + n + count]
    return []


def test_drafter_hand_cases():
    d = gpu_chat.NGramDrafter()
    assert d.propose([7, 8, 9, 7, 8], 1) == [9]               # tail (7, 8) seen before, then 9
    assert d.propose([1, 2, 3], 1) == []                       # nothing repeats
    assert d.propose([5, 6, 1, 5, 6, 2, 5, 6], 2) == [2, 5]   # the latest occurrence wins
    assert d.propose([4, 4, 4], 1) == [4]
    assert d.propose([4, 4, 4], 0) == [] and d.propose([], 3) == []
    h = gpu_chat.NGramDrafter(history=[[3, 9, 9, 11]])
    assert h.propose([1, 9, 9], 1) == [11]                     # falls back to the history
    with pytest.raises(ValueError):
        gpu_chat.NGramDrafter(min_match=3, max_match=2)
    with pytest.raises(ValueError):
        d.propose([1, 2], -1)


def test_drafter_equals_brute_force_rule():
    import random
    rnd = random.Random(3)
    for _ in range(400):
        alphabet = rnd.randint(2, 5)
        context = [rnd.randrange(alphabet) for _ in range(rnd.randint(0, 40))]
        history = [[rnd.randrange(alphabet) for _ in range(rnd.randint(0, 15))] for _ in range(rnd.randint(0, 3))]
        count = rnd.randint(0, 3)
        lo = rnd.randint(1, 3)
        hi = rnd.randint(lo, 6)
        got = gpu_chat.NGramDrafter(lo, hi, history=history).propose(context, count)
        assert got == (reference_rule(context, count, lo, hi, history) if count else []), (context, history)


def test_accepted_draft_consumes_only_committed_inputs(pack_files):
    adapter = scripted(pack_files, dict(tokens=[9, 10], accepted=1, committed_inputs=2))
    done = run(adapter)[-1]
    assert done['token_ids'] == [8, 9, 10]
    assert adapter.ledger.ids == [7, 8, 9, 7, 8, 9] and adapter.ledger.canonical == 0
    m = done['metrics']
    assert (m['rounds'], m['accepted_tokens'], m['rejected_tokens'], m['verification_calls'],
            m['verified_positions']) == (2, 1, 0, 1, 2)
    assert m['suffix_enabled'] and adapter.calls[-1] == 'verify-greedy 8 9'


def test_rejected_draft_continues_from_the_correction(pack_files):
    adapter = scripted(pack_files, dict(tokens=[15], accepted=0, committed_inputs=1))
    done = run(adapter)[-1]
    assert done['token_ids'] == [8, 15, 16]
    assert adapter.ledger.ids[-2:] == [8, 15] and adapter.calls[-1] == 'step 15'


@pytest.mark.parametrize('tokens, accepted, committed, expected', [
    ([151645], 0, 1, [8]), ([9, 151645], 1, 2, [8, 9])])
def test_eos_is_emitted_last_and_never_consumed(pack_files, tokens, accepted, committed, expected):
    adapter = scripted(pack_files, dict(tokens=tokens, accepted=accepted, committed_inputs=committed))
    done = run(adapter)[-1]
    assert done['token_ids'] == expected and done['finish_reason'] == 'eos'
    assert 151645 not in adapter.ledger.ids


def test_matching_eos_draft_commits_only_the_pending_token(pack_files):
    adapter = scripted(pack_files, dict(tokens=[151645], accepted=1, committed_inputs=1))
    done = run(adapter, request(ids=(7, 8, 151645, 7)))[-1]
    assert done['token_ids'] == [8]
    assert adapter.ledger.ids == [7, 8, 151645, 7, 8] and adapter.calls[-1] == 'verify-greedy 8 151645'


@pytest.mark.parametrize('case', ['incapable', 'no_draft', 'small_budget', 'no_match', 'no_drafter'])
def test_steps_when_drafting_is_unavailable(pack_files, case):
    adapter = scripted(pack_files, capable=case != 'incapable',
                       **({'drafter_factory': None} if case == 'no_drafter' else {}))
    req = dict(no_draft=request(max_draft=0), small_budget=request(max_new=2),
               no_match=request(ids=(1, 2, 3))).get(case, request())
    done = run(adapter, req)[-1]
    assert not any(c.startswith('verify-greedy') for c in adapter.calls)
    assert done['token_ids'] == [8, 9, 10][:req.max_new]


def test_zero_budget_emits_nothing(pack_files):
    adapter = scripted(pack_files)
    done = run(adapter, request(max_new=0))[-1]
    assert done['token_ids'] == [] and done['finish_reason'] == 'length' and done['metrics']['rounds'] == 0


def test_reuse_ceiling_is_the_prompt_prefill(pack_files):
    adapter = scripted(pack_files, dict(tokens=[9, 10], accepted=1, committed_inputs=2))
    run(adapter, request(ids=[1] * 508 + [7, 8, 9, 7]))
    assert adapter.ledger.canonical == 512 and len(adapter.ledger.ids) == 514


def test_rewind_keeps_whole_chunks_of_the_same_session(pack_files):
    adapter = scripted(pack_files)
    first = list(range(1, 1101))
    run(adapter, request(ids=first, max_draft=0))
    assert adapter.ledger.canonical == 1024
    second = first[:1030] + [5] * 70
    events = run(adapter, request(ids=second, max_draft=0))
    assert 'rewind 1024' in adapter.calls
    assert events[1]['metrics']['reused_prefix_tokens'] == 1024
    assert adapter.calls[adapter.calls.index('rewind 1024') + 2].split()[1:] == list(map(str, second[1024:]))
    adapter.calls.clear()
    run(adapter, request(ids=second, max_draft=0, session='other'))
    assert adapter.calls[0] == 'reset'
    adapter.calls.clear()
    run(adapter, request(ids=second[:512], max_draft=0, session='other'))  # never the whole prompt
    assert adapter.calls[0] == 'reset'


def test_cancel_closes_and_forgets(pack_files):
    adapter = scripted(pack_files, dict(tokens=[9, 10], accepted=1, committed_inputs=2))
    cancel, events = threading.Event(), []
    for event in adapter.stream(request(), cancel):
        events.append(event)
        if event['type'] == 'update' and event['token_ids'] == [8, 9]:
            cancel.set()
    assert events[-1]['finish_reason'] == 'stopped' and events[-1]['token_ids'] == [8, 9]
    assert adapter.link is None and not adapter.links[-1].alive() and adapter.ledger.ids == []


@pytest.mark.parametrize('row, what', [
    (dict(tokens=[9, 10], accepted=0, committed_inputs=2), 'accepted'),
    (dict(tokens=[9], accepted=1, committed_inputs=2), 'one prediction'),
    (dict(tokens=[9, 10], accepted=1, committed_inputs=2, position=3), 'position'),
    (dict(tokens=[9, 10], accepted=1, committed_inputs=2, verified_positions=1), 'verified_positions')])
def test_invalid_verification_closes(pack_files, row, what):
    adapter = scripted(pack_files, row)
    with pytest.raises(RuntimeError, match=f'verification response: {what}'):
        run(adapter)
    assert adapter.link is None and adapter.ledger.ids == []


def test_handshake_must_match(pack_files):
    adapter = scripted(pack_files)
    adapter.threads = 3  # the scripted engine reports 12 decode workers
    with pytest.raises(RuntimeError, match='handshake differs from this client in: decode_threads'):
        adapter.start(threading.Event())
    assert adapter.link is None


def test_sampled_drafting_is_rejected_before_any_command(pack_files):
    adapter = scripted(pack_files)
    with pytest.raises(ValueError, match='greedy'):
        run(adapter, request(decoding='chat'))
    assert adapter.calls == []


@pytest.mark.gpu
def test_real_process_matches_engine_greedy(qpkg, pack0):
    """The engine process behind the client (handshake with "gpu": true,
    prefix reuse, B2 drafting) yields the same greedy tokens as the library."""
    prompt = PROMPTS['decode_85']
    with qpkg.Model(pack0) as m:
        m.prefill(prompt)
        expected = []
        for _ in range(12):
            token = m.greedy()
            if token in gpu_chat.EOS:
                break
            expected.append(token)
            m.step(token)
    chat = gpu_chat.GPUChatAdapter(TEXT, binary=qpkg.CLI_PATH, weights=pack0)
    try:
        done = run(chat, request(ids=prompt, max_new=len(expected), max_draft=1))[-1]
        assert chat.ready['gpu'] is True
        assert done['token_ids'] == expected, (done['token_ids'], expected)
        assert done['finish_reason'] == 'length'
        again = run(chat, request(ids=prompt + expected[:2] + [5] * 600, max_new=3, max_draft=0))
        assert again[1]['metrics']['reused_prefix_tokens'] == 0  # 85-token prompt: no whole chunk to keep
    finally:
        chat.close()


@pytest.mark.gpu
def test_real_process_cancellation_in_flight(qpkg, pack0, tmp_path):
    """A command that has not answered when the cancel event is set: the
    client ends the process, reaps it and forgets the context; a restarted
    process answers like a fresh one. The command kept in flight is a logits
    dump into a FIFO nobody reads (the engine blocks opening it), so the
    cancellation is certain to find it unanswered."""
    with qpkg.Model(pack0) as m:
        m.prefill([9707])
        expected = m.greedy()
    chat = gpu_chat.GPUChatAdapter(TEXT, binary=qpkg.CLI_PATH, weights=pack0)
    cancel = threading.Event()
    try:
        chat.start(cancel)
        assert chat.command('prefill 9707 11', cancel)['position'] == 2
        fifo = tmp_path / 'logits.fifo'
        os.mkfifo(fifo)
        process = chat.link.proc
        timer = threading.Timer(0.5, cancel.set)
        timer.start()
        try:
            with pytest.raises(gpu_chat.Cancelled):
                chat.command(f'dump {fifo}', cancel)
        finally:
            timer.cancel()
            timer.join()
        assert process.poll() is not None and chat.link is None and chat.ledger.ids == []
        cancel.clear()
        chat.start(cancel)
        assert chat.command('mode greedy', cancel)['ok'] is True
        reply = chat.command('prefill 9707', cancel)
        assert reply['token'] == expected and reply['position'] == 1
    finally:
        chat.close()
