"""The chat-side process driver (fpga-qwen_amd/gpu_chat.py): protocol
transactions and token accounting against a fake engine (no inference, CPU),
the n-gram drafter on hand cases, and one real run of the engine process on
the GPU whose greedy tokens must equal the engine's own greedy generation.

The transaction rules follow the reference adapter's contract
(tools/native_cpu_chat.py:144-304; regression cases of
tests/test_native_suffix_adapter.py): only committed inputs are consumed,
EOS is never consumed, rewinds keep whole 512-token chunks of an earlier
prompt prefill only, and any violation closes the process.
"""
import importlib.util
import json
import threading
from pathlib import Path
from types import SimpleNamespace

import pytest

ROOT = Path(__file__).resolve().parents[1]
spec = importlib.util.spec_from_file_location('gpu_chat', ROOT / 'fpga-qwen_amd' / 'gpu_chat.py')
gpu_chat = importlib.util.module_from_spec(spec)
spec.loader.exec_module(gpu_chat)
PROMPTS = json.loads((Path(__file__).parent / 'golden' / 'prompts.json').read_text())


class ScriptedEngine(gpu_chat.NativeGPUChat):
    """Answers commands like the engine would, with a scripted verify-greedy
    result; prefill answers token 8 and step answers its input + 1."""

    def __init__(self, verification=None, capable=True, **kwargs):
        super().__init__(SimpleNamespace(tokenizer=SimpleNamespace(decode=lambda ids, **kw: str(ids))), **kwargs)
        self.verification, self.capable = verification, capable
        self.calls, self.position, self.closed = [], 0, False

    def start(self, cancel):
        self.process = SimpleNamespace(poll=lambda: None)
        self.ready = dict(prefix_reuse=True, prefix_reuse_chunk=512, verify_greedy_b2=self.capable,
                          max_verified_draft=1)

    def close(self):
        self.closed = True
        self.process = self.ready = None
        self._forget()

    def command(self, command, cancel, *, preserve_cache=False):
        self.calls.append(command)
        op, *args = command.split()
        if op == 'reset':
            self._forget()
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
        raise AssertionError(command)


def request(ids=(7, 8, 9, 7), max_new=3, max_draft=1, decoding='greedy', session='s'):
    return SimpleNamespace(ids=list(ids), max_new=max_new, max_draft=max_draft, decoding=decoding,
                           session=session, seed=42)


def run(engine, req=None, cancel=None):
    return list(engine.stream(req or request(), cancel or threading.Event()))


def test_drafter_longest_latest_match():
    d = gpu_chat.LongestMatchDrafter()
    assert d.propose([7, 8, 9, 7, 8], 1) == [9]          # suffix (7, 8) seen before, then 9
    assert d.propose([1, 2, 3], 1) == []                  # nothing repeats
    assert d.propose([5, 6, 1, 5, 6, 2, 5, 6], 2) == [2, 5]  # latest occurrence wins
    assert d.propose([4, 4, 4], 1) == [4]
    h = gpu_chat.LongestMatchDrafter(history=[[3, 9, 9, 11]])
    assert h.propose([1, 9, 9], 1) == [11]               # falls back to history
    with pytest.raises(ValueError):
        gpu_chat.LongestMatchDrafter(min_match=3, max_match=2)


def test_accepted_draft_consumes_only_committed_inputs():
    engine = ScriptedEngine(dict(tokens=[9, 10], accepted=1, committed_inputs=2))
    done = run(engine)[-1]
    assert done['token_ids'] == [8, 9, 10]
    assert engine.cache_ids == [7, 8, 9, 7, 8, 9]
    assert engine.canonical_reusable_tokens == 0
    m = done['metrics']
    assert (m['rounds'], m['accepted_tokens'], m['rejected_tokens'], m['verification_calls'],
            m['verified_positions']) == (2, 1, 0, 1, 2)
    assert m['suffix_enabled'] and engine.calls[-1] == 'verify-greedy 8 9'


def test_rejected_draft_continues_from_the_correction():
    engine = ScriptedEngine(dict(tokens=[15], accepted=0, committed_inputs=1))
    done = run(engine)[-1]
    assert done['token_ids'] == [8, 15, 16]
    assert engine.cache_ids[-2:] == [8, 15] and engine.calls[-1] == 'step 15'


@pytest.mark.parametrize('tokens, accepted, committed, expected', [
    ([151645], 0, 1, [8]), ([9, 151645], 1, 2, [8, 9])])
def test_eos_is_emitted_last_and_never_consumed(tokens, accepted, committed, expected):
    engine = ScriptedEngine(dict(tokens=tokens, accepted=accepted, committed_inputs=committed))
    done = run(engine)[-1]
    assert done['token_ids'] == expected and done['finish_reason'] == 'eos'
    assert 151645 not in engine.cache_ids


def test_matching_eos_draft_commits_only_the_pending_token():
    engine = ScriptedEngine(dict(tokens=[151645], accepted=1, committed_inputs=1))
    done = run(engine, request(ids=(7, 8, 151645, 7)))[-1]
    assert done['token_ids'] == [8]
    assert engine.cache_ids == [7, 8, 151645, 7, 8] and engine.calls[-1] == 'verify-greedy 8 151645'


@pytest.mark.parametrize('engine, req', [
    (ScriptedEngine(capable=False), request()), (ScriptedEngine(), request(max_draft=0)),
    (ScriptedEngine(), request(max_new=2)), (ScriptedEngine(), request(ids=(1, 2, 3))),
    (ScriptedEngine(drafter_factory=None), request())])
def test_steps_when_drafting_is_unavailable(engine, req):
    done = run(engine, req)[-1]
    assert not any(c.startswith('verify-greedy') for c in engine.calls)
    assert done['token_ids'] == [8, 9, 10][:req.max_new]


def test_reuse_ceiling_is_the_prompt_prefill():
    engine = ScriptedEngine(dict(tokens=[9, 10], accepted=1, committed_inputs=2))
    run(engine, request(ids=[1] * 508 + [7, 8, 9, 7]))
    assert engine.canonical_reusable_tokens == 512 and len(engine.cache_ids) == 514


def test_rewind_keeps_whole_chunks_of_the_same_session():
    engine = ScriptedEngine()
    first = list(range(1, 1101))
    run(engine, request(ids=first, max_draft=0))
    assert engine.canonical_reusable_tokens == 1024
    second = first[:1030] + [5] * 70
    events = run(engine, request(ids=second, max_draft=0))
    assert 'rewind 1024' in engine.calls
    assert events[1]['metrics']['reused_prefix_tokens'] == 1024
    assert engine.calls[engine.calls.index('rewind 1024') + 2].split()[1:] == list(map(str, second[1024:]))
    engine.calls.clear()
    run(engine, request(ids=second, max_draft=0, session='other'))
    assert engine.calls[0] == 'reset'
    engine.calls.clear()
    run(engine, request(ids=second[:512], max_draft=0, session='other'))  # never the whole prompt
    assert engine.calls[0] == 'reset'


def test_cancel_closes_and_forgets():
    engine = ScriptedEngine(dict(tokens=[9, 10], accepted=1, committed_inputs=2))
    cancel, events = threading.Event(), []
    for event in engine.stream(request(), cancel):
        events.append(event)
        if event['type'] == 'update' and event['token_ids'] == [8, 9]:
            cancel.set()
    assert events[-1]['finish_reason'] == 'stopped' and events[-1]['token_ids'] == [8, 9]
    assert engine.closed and engine.cache_ids == []


def test_invalid_verification_closes():
    engine = ScriptedEngine(dict(tokens=[9, 10], accepted=0, committed_inputs=2))
    with pytest.raises(RuntimeError, match='verification response'):
        run(engine)
    assert engine.closed and engine.cache_ids == []


def test_sampled_drafting_is_rejected_before_any_command():
    engine = ScriptedEngine()
    with pytest.raises(ValueError, match='greedy'):
        run(engine, request(decoding='chat'))
    assert engine.calls == []


@pytest.mark.gpu
def test_real_process_matches_engine_greedy(qpkg, pack0):
    """The engine process behind the adapter (handshake with "gpu": true,
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
    chat = gpu_chat.NativeGPUChat(SimpleNamespace(tokenizer=SimpleNamespace(decode=lambda ids, **kw: str(ids))),
                                  binary=qpkg.CLI_PATH, weights=pack0)
    try:
        done = run(chat, request(ids=prompt, max_new=len(expected), max_draft=1))[-1]
        assert chat.ready['gpu'] is True
        assert done['token_ids'] == expected, (done['token_ids'], expected)
        assert done['finish_reason'] == 'length'
        again = run(chat, request(ids=prompt + expected[:2] + [5] * 600, max_new=3, max_draft=0))
        assert again[1]['metrics']['reused_prefix_tokens'] == 0  # 85-token prompt: no whole chunk to keep
    finally:
        chat.close()
