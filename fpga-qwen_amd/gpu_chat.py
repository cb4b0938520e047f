"""Chat client of the MI355X engine process (``build/qwen_gpu``, protocol v1 of
engine/INTERFACE.md:40-90).

A front end hands it one request at a time (prompt token ids, an output
budget, greedy or seeded chat decoding, optional one-token drafting) and
receives the events a chat page consumes: ``loading``, ``start``,
``prefill``, one ``update`` per emitted token and ``done``, each carrying the
running metrics. Tokenization and text belong to the caller
(``protocol.tokenizer.decode``).

The rules it keeps are the reference adapter's contract
(tools/native_cpu_chat.py:144-304, engine/INTERFACE.md:91-120); the code is
this project's own:

* the engine consumes only committed inputs; an EOS prediction is reported,
  never fed back;
* a new request of the same session reuses its common prefix with what the
  engine holds, but only whole 512-token chunks that came from a prompt
  prefill, and never the whole prompt (the last prompt token is always
  prefilled, its logits give the first output); anything else starts from
  ``reset``;
* drafting (greedy only, opt-in per request) proposes one token after the
  pending one and checks both with ``verify-greedy``; only what the engine
  committed enters the context;
* an error object, a malformed or inconsistent response, a time-out or a
  cancellation ends the process and forgets the context.

It differs where this engine does: the handshake reports ``"gpu": true``.
"""
import json
import os
import queue
import secrets
import subprocess
import threading
import time
from dataclasses import asdict, dataclass, field
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
EOS = frozenset((151643, 151645))
VOCABULARY = 151936
CONTEXT = 4096
CHUNK = 512
REPLY_TIMEOUT = 180.0

# What the engine's ready line must state (exact values and JSON types).
HANDSHAKE = dict(ready=True, protocol=1, gpu=True, pytorch=False, weight_precision='f16', kv_precision='f16',
                 norm_precision='f32', activation_precision='f32', context=CONTEXT)


class Cancelled(Exception):
    """The caller's cancel event was set while a request was running."""


class EngineError(RuntimeError):
    """The engine answered with an error, broke the protocol or went away."""


def _is_token(value):
    return type(value) is int and 0 <= value < VOCABULARY


# ---------------------------------------------------------------- drafting

class NGramDrafter:
    """Proposes what followed an earlier occurrence of the context's tail.

    Tails of max_match down to min_match tokens are tried, longest first; for
    each tail the current context is searched first, then the history
    sequences from the newest; within a sequence the occurrence closest to its
    end that still has a following token wins. That is the reference
    drafter's rule (tools/suffix.py:4-29); the search here walks the
    occurrences of the tail's last token, indexed once per sequence.
    """

    def __init__(self, min_match=2, max_match=12, max_context=CONTEXT, history=()):
        if not (1 <= min_match <= max_match) or max_context < max_match:
            raise ValueError('Drafter limits need 1 <= min_match <= max_match <= max_context')
        self.min_match, self.max_match, self.max_context = min_match, max_match, max_context
        self.history = [list(seq) for seq in history]

    @staticmethod
    def _ends(seq):
        """token -> end positions (exclusive) that have a following token, newest first."""
        ends = {}
        for end in range(len(seq) - 1, 0, -1):
            ends.setdefault(seq[end - 1], []).append(end)
        return ends

    def propose(self, context, count):
        if count < 0:
            raise ValueError('Cannot propose a negative number of tokens')
        context = list(context)[-self.max_context:]
        if count == 0 or not context:
            return []
        sources = [context] + self.history[::-1]
        indexes = [self._ends(seq) for seq in sources]
        for length in range(min(self.max_match, len(context)), self.min_match - 1, -1):
            tail = context[-length:]
            for seq, ends in zip(sources, indexes):
                for end in ends.get(tail[-1], ()):
                    if end >= length and seq[end - length:end] == tail:
                        return seq[end:end + count]
        return []


# ---------------------------------------------------------------- transport

_CLOSED = object()


class ProcessLink:
    """One engine process. Commands are written to its stdin; a reader thread
    cuts its stdout into lines and queues them, so waiting for a reply can
    watch the cancel event and a deadline at the same time."""

    MAX_LINE = 1 << 20

    def __init__(self, argv, log):
        self.proc = subprocess.Popen(argv, stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=log, bufsize=0)
        self.lines = queue.Queue()
        self.reader = threading.Thread(target=self._read_lines, daemon=True)
        self.reader.start()

    def _read_lines(self):
        pending = bytearray()
        try:
            while True:
                block = os.read(self.proc.stdout.fileno(), 1 << 16)
                if not block:
                    break
                pending += block
                while (cut := pending.find(b'\n')) >= 0:
                    self.lines.put(bytes(pending[:cut]))
                    del pending[:cut + 1]
                if len(pending) > self.MAX_LINE:
                    self.lines.put(b'oversized')
                    break
        except OSError:
            pass
        finally:
            self.lines.put(_CLOSED)

    def alive(self):
        return self.proc.poll() is None

    def send(self, line):
        data = (line + '\n').encode()
        written = 0
        while written < len(data):
            n = self.proc.stdin.write(data[written:])
            if not n:
                raise EngineError('Engine stdin closed')
            written += n

    def receive(self, cancel, timeout):
        """The next reply as a dict; Cancelled, EngineError or TimeoutError."""
        deadline = time.monotonic() + timeout
        while True:
            if cancel.is_set():
                raise Cancelled()
            try:
                line = self.lines.get(timeout=0.02)
            except queue.Empty:
                if time.monotonic() > deadline:
                    raise TimeoutError('No engine reply before the deadline')
                continue
            if line is _CLOSED:
                raise EngineError('Engine process ended; see its chat.log')
            try:
                reply = json.loads(line)
            except ValueError:
                raise EngineError(f'Engine wrote a line that is not JSON: {line[:120]!r}') from None
            if not isinstance(reply, dict):
                raise EngineError(f'Engine reply is not an object: {reply!r}')
            if 'error' in reply:
                raise EngineError(f'Engine error: {reply["error"]}')
            return reply

    def exchange(self, line, cancel, timeout=REPLY_TIMEOUT):
        self.send(line)
        return self.receive(cancel, timeout)

    def shutdown(self):
        if self.proc.poll() is None:
            self.proc.terminate()
            try:
                self.proc.wait(timeout=2)
            except subprocess.TimeoutExpired:
                self.proc.kill()
                self.proc.wait(timeout=5)
        for pipe in (self.proc.stdin, self.proc.stdout):
            try:
                pipe.close()
            except OSError:
                pass
        self.reader.join(timeout=2)


# ---------------------------------------------------------------- context bookkeeping

class ContextLedger:
    """What the engine holds: the ids it consumed, in order, the session they
    belong to, and how many leading ids are whole 512-token chunks of a prompt
    prefill (the only part a later request may keep)."""

    def __init__(self):
        self.clear()

    def clear(self):
        self.ids, self.session, self.canonical = [], None, 0

    def reusable(self, session, prompt):
        """Leading prompt tokens a rewind may keep (a multiple of 512)."""
        if session != self.session:
            return 0
        limit = min(self.canonical, len(prompt) - 1, len(self.ids))
        common = 0
        while common < limit and self.ids[common] == prompt[common]:
            common += 1
        return common - common % CHUNK

    def prefilled(self, session, prompt):
        self.ids, self.session = list(prompt), session
        self.canonical = len(prompt) - len(prompt) % CHUNK


@dataclass
class RequestMetrics:
    """The running numbers each event carries (names as the chat page reads them)."""
    prompt_tokens: int = 0
    reused_prefix_tokens: int = 0
    evaluated_prompt_tokens: int = 0
    output_tokens: int = 0
    rounds: int = 0
    proposed_tokens: int = 0
    accepted_tokens: int = 0
    rejected_tokens: int = 0
    tokens_per_round: float = 0
    suffix_enabled: bool = False
    verification_calls: int = 0
    verified_positions: int = 0
    decode_tokens_per_second: float = 0
    first_token_ms: float = None
    elapsed_seconds: float = 0
    kv_tokens: int = 0
    context_limit: int = CONTEXT


@dataclass
class _Run:
    request: object
    began: float = field(default_factory=time.perf_counter)
    tokens: list = field(default_factory=list)
    text: str = ''
    first_at: float = None
    reason: str = 'length'
    metrics: RequestMetrics = field(default_factory=RequestMetrics)

    def event(self, kind, **extra):
        self.metrics.elapsed_seconds = time.perf_counter() - self.began
        return dict(type=kind, **extra, metrics=asdict(self.metrics))

    def emit(self, token, decode):
        now = time.perf_counter()
        self.tokens.append(token)
        if self.first_at is None:
            self.first_at = now
            self.metrics.first_token_ms = (now - self.began) * 1e3
        self.text = decode(self.tokens, skip_special_tokens=True)
        m = self.metrics
        m.output_tokens = len(self.tokens)
        m.tokens_per_round = m.output_tokens / m.rounds
        m.decode_tokens_per_second = (len(self.tokens) - 1) / (now - self.first_at) if now > self.first_at else 0
        return self.event('update', text=self.text, token_ids=list(self.tokens))

    def done(self):
        m = self.metrics
        m.tokens_per_round = len(self.tokens) / m.rounds if m.rounds else 0
        return self.event('done', text=self.text, token_ids=list(self.tokens), finish_reason=self.reason)


def _checked_verification(reply, draft, budget, base):
    """(tokens, accepted, committed) of a verify-greedy reply, after checking it
    against engine/INTERFACE.md:63-72 and the request's output budget."""
    def fail(what):
        raise EngineError(f'Invalid engine B2 verification response: {what}')

    tokens = reply.get('tokens')
    if not (isinstance(tokens, list) and 1 <= len(tokens) <= 2 and all(map(_is_token, tokens))):
        fail('tokens')
    accepted = reply.get('accepted')
    if type(accepted) is not int or accepted != int(tokens[0] == draft):
        fail('accepted')
    committed = reply.get('committed_inputs')
    if type(committed) is not int or committed != (2 if accepted and tokens[0] not in EOS else 1):
        fail('committed_inputs')
    if len(tokens) != committed:
        fail('one prediction per committed input')
    if len(tokens) > budget:
        fail('more predictions than the output budget')
    if tokens[0] in EOS and len(tokens) > 1:
        fail('prediction after EOS')
    position = reply.get('position')
    if type(position) is not int or position != base + committed:
        fail('position')
    if type(reply.get('verified_positions')) is not int or reply['verified_positions'] != 2:
        fail('verified_positions')
    if reply.get('finish_reason') != ('eos' if tokens[-1] in EOS else None):
        fail('finish_reason')
    return tokens, accepted, committed


# ---------------------------------------------------------------- the client

class GPUChatAdapter:
    def __init__(self, protocol, binary=None, weights=None, threads=12, prefill_threads=6, reuse_prefix=True,
                 drafter_factory=NGramDrafter, link_factory=None):
        if not isinstance(reuse_prefix, bool):
            raise ValueError('reuse_prefix must be True or False')
        self.protocol = protocol
        self.binary = Path(binary or PACKAGE_DIR / 'build' / 'qwen_gpu')
        self.weights = Path(weights or PACKAGE_DIR / 'build' / 'weights.bin')
        self.threads, self.prefill_threads = threads, prefill_threads
        self.reuse_prefix = reuse_prefix
        self.drafter_factory = drafter_factory
        self.link_factory = link_factory or self._spawn
        self.link = None
        self.ready = None
        self.ledger = ContextLedger()
        self._log = None

    # -- capabilities the running engine advertised
    def _advertises(self, key, value=True):
        ready = self.ready or {}
        return (self.link is not None and self.link.alive() and type(ready.get(key)) is type(value)
                and ready.get(key) == value)

    def prefix_reuse_supported(self):
        return self._advertises('prefix_reuse') and self._advertises('prefix_reuse_chunk', CHUNK)

    def suffix_supported(self):
        return self._advertises('verify_greedy_b2') and self._advertises('max_verified_draft', 1)

    def available(self):
        files = [self.binary, self.weights, Path(f'{self.weights}.index'), Path(f'{self.weights}.manifest.json')]
        return all(p.is_file() for p in files) and os.access(self.binary, os.X_OK)

    def status(self):
        reuse, suffix = self.prefix_reuse_supported(), self.suffix_supported()
        return dict(model='Qwen3-0.6B', device='gpu', gpu_inference=True, pytorch_loaded=False,
                    precision='FP16 matrices / FP32 norm weights / FP16 KV', context_limit=CONTEXT,
                    decode_workers=self.threads, prefill_workers=self.prefill_threads,
                    cached_tokens=len(self.ledger.ids) if reuse else 0,
                    prefix_reuse_supported=reuse, prefix_reuse_enabled=reuse and self.reuse_prefix,
                    canonical_reusable_tokens=self.ledger.canonical if reuse else 0,
                    canonical_prefix_policy='native_f16_prefill512_v1' if reuse else None,
                    suffix_supported=suffix, suffix_greedy_only=True, max_verified_draft=int(suffix))

    # -- process lifetime
    def _spawn(self):
        if self._log is None:
            self._log = (self.binary.parent / 'chat.log').open('ab')
        return ProcessLink([str(self.binary), '--weights', str(self.weights), '--threads', str(self.threads),
                            '--prefill-threads', str(self.prefill_threads), '--context', str(CONTEXT)], self._log)

    def start(self, cancel):
        """Starts the engine unless it is running, and checks its ready line."""
        if self.link is not None and self.link.alive():
            return
        self.close()
        if not self.available():
            raise EngineError('Build the engine and write a weight pack before selecting this backend')
        manifest = json.loads(Path(f'{self.weights}.manifest.json').read_text())
        if manifest.get('format') != 'QWCPU01' or manifest.get('completed') is not True:
            raise EngineError('The weight pack manifest does not mark a completed QWCPU01 pack')
        try:
            self.link = self.link_factory()
            ready = self.link.receive(cancel, REPLY_TIMEOUT)
            wanted = dict(HANDSHAKE, decode_threads=self.threads, prefill_threads=self.prefill_threads)
            wrong = sorted(k for k, v in wanted.items() if type(ready.get(k)) is not type(v) or ready.get(k) != v)
            if wrong:
                raise EngineError(f'Engine handshake differs from this client in: {", ".join(wrong)}')
            self.ready = ready
        except BaseException:
            self.close()
            raise

    def close(self):
        self.ledger.clear()
        link, self.link, self.ready = self.link, None, None
        if link is not None:
            link.shutdown()
        if self._log is not None:
            self._log.close()
            self._log = None

    def command(self, line, cancel, *, keep_ledger=False):
        """Sends one protocol command and returns its reply. A command that
        changes the engine's context clears the ledger unless the caller
        updates it itself (keep_ledger); any failure ends the process."""
        if '\n' in line or '\r' in line:
            raise ValueError('A protocol command is one line')
        verb = line.split(' ', 1)[0]
        if verb == 'reset' or (not keep_ledger and verb in ('rewind', 'prefill', 'step', 'verify-greedy')):
            self.ledger.clear()
        try:
            if cancel.is_set():
                raise Cancelled()
            if self.link is None:
                raise EngineError('Engine not started')
            return self.link.exchange(line, cancel)
        except BaseException:
            self.close()
            raise

    # -- one request
    def stream(self, request, cancel):
        """Yields the request's events; request has ids, max_new, max_draft,
        decoding ('greedy' or chat), seed and session."""
        run = _Run(request)
        run.metrics.prompt_tokens = len(request.ids)
        try:
            if request.max_draft and request.decoding != 'greedy':
                raise ValueError('One-token drafting needs greedy decoding')
            yield run.event('loading', message='Loading the MI355X engine…')
            self.start(cancel)
            run.metrics.suffix_enabled = bool(request.max_draft > 0 and request.decoding == 'greedy'
                                              and self.suffix_supported())
            kept = self._open_context(request, cancel)
            run.metrics.reused_prefix_tokens = kept
            run.metrics.evaluated_prompt_tokens = len(request.ids) - kept
            run.metrics.kv_tokens = kept
            self._choose_mode(request, cancel)
            yield run.event('start')
            first = self._prefill(request, kept, cancel)
            run.metrics.kv_tokens = len(self.ledger.ids)
            yield run.event('prefill', processed_tokens=len(request.ids) - kept)
            yield from self._decode(run, first, cancel)
            if cancel.is_set():
                raise Cancelled()
        except Cancelled:
            self.close()
            run.reason = 'stopped'
        except BaseException:
            self.close()
            raise
        yield run.done()

    def _open_context(self, request, cancel):
        keep = self.ledger.reusable(request.session, request.ids) if (
            self.reuse_prefix and self.prefix_reuse_supported()) else 0
        if keep:
            reply = self.command(f'rewind {keep}', cancel, keep_ledger=True)
            if reply.get('ok') is not True or reply.get('position') != keep:
                raise EngineError('Engine rewind did not keep the reused prefix')
            self.ledger.ids = self.ledger.ids[:keep]
            self.ledger.canonical = keep
        else:
            reply = self.command('reset', cancel)
            if reply.get('ok') is not True or reply.get('position') != 0:
                raise EngineError('Engine reset did not empty the context')
        return keep

    def _choose_mode(self, request, cancel):
        if request.decoding == 'greedy':
            line = 'mode greedy'
        else:
            line = f'mode chat {request.seed if request.seed is not None else secrets.randbits(32)}'
        if self.command(line, cancel).get('ok') is not True:
            raise EngineError('Engine did not acknowledge the decoding mode')

    def _prefill(self, request, kept, cancel):
        reply = self.command('prefill ' + ' '.join(map(str, request.ids[kept:])), cancel, keep_ledger=True)
        if reply.get('position') != len(request.ids):
            raise EngineError('Engine position after prefill is not the prompt length')
        self.ledger.prefilled(request.session, request.ids)
        if not self.prefix_reuse_supported():
            self.ledger.canonical = 0
        return reply.get('token')

    def _decode(self, run, first, cancel):
        request, decode = run.request, self.protocol.tokenizer.decode
        drafter = self.drafter_factory() if self.drafter_factory else None
        fresh = [first]  # predictions not yet shown; the last shown one is pending
        while len(run.tokens) < request.max_new:
            run.metrics.rounds += 1
            run.metrics.kv_tokens = len(self.ledger.ids)
            for token in fresh:
                if cancel.is_set():
                    raise Cancelled()
                if not _is_token(token):
                    raise EngineError(f'Engine predicted an invalid token: {token!r}')
                if token in EOS:
                    run.reason = 'eos'
                    return
                yield run.emit(token, decode)
            budget = request.max_new - len(run.tokens)
            if budget <= 0:
                return
            fresh = self._advance(run, run.tokens[-1], budget, drafter, cancel)

    def _advance(self, run, pending, budget, drafter, cancel):
        """Feeds the pending token (and a draft after it, when one is
        proposed) and returns the engine's new predictions."""
        draft = []
        if (drafter is not None and run.request.max_draft > 0 and budget >= 2 and self.suffix_supported()
                and len(self.ledger.ids) + 2 <= CONTEXT):
            draft = drafter.propose(self.ledger.ids + [pending], 1)
        if not draft:
            reply = self.command(f'step {pending}', cancel, keep_ledger=True)
            if reply.get('position') != len(self.ledger.ids) + 1:
                raise EngineError('Engine position after a step is not one past the context')
            self.ledger.ids.append(pending)
            return [reply.get('token')]
        m = run.metrics
        m.proposed_tokens += 1
        m.verification_calls += 1
        reply = self.command(f'verify-greedy {pending} {draft[0]}', cancel, keep_ledger=True)
        tokens, accepted, committed = _checked_verification(reply, draft[0], budget, len(self.ledger.ids))
        self.ledger.ids += [pending, draft[0]][:committed]
        m.accepted_tokens += accepted
        m.rejected_tokens += 1 - accepted
        m.verified_positions += 2
        return tokens
