"""Chat-side driver of the MI355X engine process (protocol v1,
engine/INTERFACE.md:40-90): the counterpart of the reference's adapter
tools/native_cpu_chat.py for callers that switch to ``build/qwen_gpu``.

It keeps the adapter's contract (tools/native_cpu_chat.py:144-304) and
differs where the process does: the handshake reports ``"gpu": true``.

* One process per adapter, started lazily; its ready object must report
  protocol 1, ``gpu`` true, ``pytorch`` false, FP16 weights and KV, FP32
  norms and activations, the requested worker counts and a 4096 context.
* Canonical prefix reuse: a request in the same session reuses the longest
  common prefix with the previous prompt, rounded down to a multiple of 512
  and capped by the tokens that came from a fresh prompt prefill (never
  decoded tokens, never the whole prompt), via ``rewind``; otherwise
  ``reset``. Rows of a 512-aligned rewind equal a fresh prefill's.
* Greedy B2 drafting (opt-in per request): when a drafter proposes one token
  after the pending one, ``verify-greedy PENDING DRAFT`` checks both in one
  call and the adapter consumes only what the engine committed.
* Any protocol violation, error object or cancellation closes the process
  and forgets the cached prefix.

Token ids in, token ids out; tokenization and text belong to the caller
(``protocol.tokenizer.decode``).
"""
import json
import os
import secrets
import select
import subprocess
import time
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
EOS = frozenset((151643, 151645))
VOCABULARY = 151936
CONTEXT = 4096
CHUNK = 512


class NativeCancelled(Exception):
    """The request's cancel event was set."""


class LongestMatchDrafter:
    """Proposes the tokens that followed the most recent earlier occurrence
    of the context's longest suffix (min_match..max_match tokens), looking in
    the context first and then in earlier sequences, newest first. The same
    rule as the reference's n-gram drafter (tools/suffix.py:4-33): no model,
    no future tokens."""

    def __init__(self, min_match=2, max_match=12, max_context=CONTEXT, history=()):
        if not 1 <= min_match <= max_match or max_context < max_match:
            raise ValueError('Invalid matching limits')
        self.min_match, self.max_match, self.max_context = min_match, max_match, max_context
        self.history = [tuple(h) for h in history]

    def propose(self, context, count):
        if count < 0:
            raise ValueError('Negative proposal length')
        if count == 0:
            return []
        context = tuple(context[-self.max_context:])
        sources = [context] + self.history[::-1]
        for length in range(min(self.max_match, len(context)), self.min_match - 1, -1):
            suffix = context[-length:]
            for seq in sources:
                # Latest occurrence that still has a next token.
                for start in range(len(seq) - length - 1, -1, -1):
                    if seq[start:start + length] == suffix:
                        return list(seq[start + length:start + length + count])
        return []


class NativeGPUChat:
    def __init__(self, protocol, binary=None, weights=None, threads=12, prefill_threads=6, reuse_prefix=True,
                 drafter_factory=LongestMatchDrafter):
        if type(reuse_prefix) is not bool:
            raise ValueError('reuse_prefix must be boolean')
        self.protocol = protocol
        self.binary = Path(binary or PACKAGE_DIR / 'build' / 'qwen_gpu')
        self.weights = Path(weights or PACKAGE_DIR / 'build' / 'weights.bin')
        self.threads, self.prefill_threads = threads, prefill_threads
        self.reuse_prefix = reuse_prefix
        self.drafter_factory = drafter_factory
        self.process = None
        self.ready = None
        self.log = None
        self._pending = b''
        self._forget()

    # -- cached prefix bookkeeping ---------------------------------------
    def _forget(self):
        self.cache_ids = []           # inputs the engine has consumed, in order
        self.cache_session = None
        self.canonical_reusable_tokens = 0   # prompt tokens a rewind may keep

    def _capable(self, key, value):
        return bool(self.ready and self.ready.get(key) is True and self.process is not None
                    and self.process.poll() is None and value)

    def prefix_reuse_supported(self):
        chunk = (self.ready or {}).get('prefix_reuse_chunk')
        return self._capable('prefix_reuse', type(chunk) is int and chunk == CHUNK)

    def suffix_supported(self):
        draft = (self.ready or {}).get('max_verified_draft')
        return self._capable('verify_greedy_b2', type(draft) is int and draft == 1)

    def available(self):
        return (self.binary.is_file() and os.access(self.binary, os.X_OK) and self.weights.is_file()
                and Path(f'{self.weights}.index').is_file() and Path(f'{self.weights}.manifest.json').is_file())

    def status(self):
        reuse, suffix = self.prefix_reuse_supported(), self.suffix_supported()
        return dict(model='Qwen3-0.6B', device='gpu', gpu_inference=True, pytorch_loaded=False,
                    precision='FP16 matrices / FP32 norm weights / FP16 KV', context_limit=CONTEXT,
                    decode_workers=self.threads, prefill_workers=self.prefill_threads,
                    cached_tokens=len(self.cache_ids) if reuse else 0,
                    prefix_reuse_supported=reuse, prefix_reuse_enabled=self.reuse_prefix and reuse,
                    canonical_reusable_tokens=self.canonical_reusable_tokens if reuse else 0,
                    canonical_prefix_policy='native_f16_prefill512_v1' if reuse else None,
                    suffix_supported=suffix, suffix_greedy_only=True, max_verified_draft=1 if suffix else 0)

    # -- process ---------------------------------------------------------
    def close(self):
        self._forget()
        process, self.process = self.process, None
        if process is not None:
            if process.poll() is None:
                process.terminate()
                try:
                    process.wait(timeout=2)
                except subprocess.TimeoutExpired:
                    process.kill()
                    process.wait(timeout=5)
            for pipe in (process.stdin, process.stdout):
                if pipe:
                    pipe.close()
        if self.log:
            self.log.close()
            self.log = None
        self._pending = b''
        self.ready = None

    def start(self, cancel):
        if self.process is not None and self.process.poll() is None:
            return
        self.close()
        if not self.available():
            raise RuntimeError('Build the engine and export a weight pack before selecting this backend')
        manifest = json.loads(Path(f'{self.weights}.manifest.json').read_text())
        if manifest.get('format') != 'QWCPU01' or manifest.get('completed') is not True:
            raise RuntimeError('Weight pack manifest is incomplete')
        self.log = (self.binary.parent / 'chat.log').open('ab')
        argv = [str(self.binary), '--weights', str(self.weights), '--threads', str(self.threads),
                '--prefill-threads', str(self.prefill_threads), '--context', str(CONTEXT)]
        try:
            self.process = subprocess.Popen(argv, stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=self.log,
                                            bufsize=0)
            ready = self._read(cancel)
            expected = dict(ready=True, protocol=1, gpu=True, pytorch=False, weight_precision='f16',
                            kv_precision='f16', norm_precision='f32', activation_precision='f32',
                            decode_threads=self.threads, prefill_threads=self.prefill_threads, context=CONTEXT)
            if any(ready.get(key) != value or type(ready.get(key)) is not type(value)
                   for key, value in expected.items()):
                raise RuntimeError('Unexpected engine startup handshake')
            self.ready = ready
        except BaseException:
            self.close()
            raise

    def _read(self, cancel, timeout=180):
        deadline = time.monotonic() + timeout
        while True:
            if cancel.is_set():
                self.close()
                raise NativeCancelled()
            line, sep, rest = self._pending.partition(b'\n')
            if sep:
                self._pending = rest
                value = json.loads(line)
                if not isinstance(value, dict) or value.get('error'):
                    raise RuntimeError(f'Engine protocol error: {value}')
                return value
            if self.process is None or self.process.poll() is not None:
                raise RuntimeError('Engine process exited; see its chat.log')
            if time.monotonic() >= deadline:
                raise TimeoutError('Engine response timed out')
            if select.select([self.process.stdout], [], [], 0.05)[0]:
                block = os.read(self.process.stdout.fileno(), 1 << 16)
                if not block:
                    raise RuntimeError('Engine stdout closed')
                self._pending += block
                if len(self._pending) > 1 << 20:
                    raise RuntimeError('Oversized engine protocol response')

    def command(self, command, cancel, *, preserve_cache=False):
        """Sends one command line and returns its JSON response. Commands that
        change the context forget the cached prefix unless the caller keeps
        the bookkeeping itself (preserve_cache)."""
        if '\n' in command or '\r' in command:
            raise ValueError('Engine command must occupy one line')
        op = command.split(' ', 1)[0]
        if op == 'reset' or (not preserve_cache and op in ('rewind', 'prefill', 'step', 'verify-greedy')):
            self._forget()
        try:
            if cancel.is_set():
                raise NativeCancelled()
            data = memoryview((command + '\n').encode())
            while data:
                n = self.process.stdin.write(data)
                if not n:
                    raise RuntimeError('Engine stdin closed')
                data = data[n:]
            self.process.stdin.flush()
            return self._read(cancel)
        except BaseException:
            self.close()
            raise

    # -- one request -----------------------------------------------------
    def _reusable(self, request):
        if not (self.reuse_prefix and self.prefix_reuse_supported() and self.cache_session == request.session):
            return 0
        common = 0
        for a, b in zip(self.cache_ids, request.ids):
            if a != b:
                break
            common += 1
        # Keep whole 512-token chunks of an earlier prompt prefill, and always
        # recompute at least one prompt token so the call yields logits.
        return min(common, self.canonical_reusable_tokens, len(request.ids) - 1) // CHUNK * CHUNK

    def _check_verification(self, response, draft, remaining):
        tokens, accepted, committed = response.get('tokens'), response.get('accepted'), response.get('committed_inputs')
        valid = (isinstance(tokens, list) and tokens and all(type(t) is int and 0 <= t < VOCABULARY for t in tokens)
                 and type(accepted) is int and accepted == int(tokens[0] == draft)
                 and type(committed) is int and committed == (2 if accepted and tokens[0] not in EOS else 1)
                 and len(tokens) == committed and len(tokens) <= remaining
                 and not any(t in EOS for t in tokens[:-1])
                 and type(response.get('position')) is int
                 and response['position'] == len(self.cache_ids) + committed
                 and response.get('verified_positions') == 2 and type(response.get('verified_positions')) is int
                 and response.get('finish_reason') == ('eos' if tokens[-1] in EOS else None))
        if not valid:
            raise RuntimeError('Invalid engine B2 verification response')
        return tokens, accepted, committed

    def stream(self, request, cancel):
        """Yields loading, start, prefill, update* and done events for one
        request (ids, max_new, max_draft, decoding 'greedy' or chat, seed,
        session)."""
        started = time.perf_counter()
        out, text, first, reason = [], '', None, 'length'
        metrics = dict(prompt_tokens=len(request.ids), reused_prefix_tokens=0, output_tokens=0, rounds=0,
                       proposed_tokens=0, accepted_tokens=0, rejected_tokens=0, tokens_per_round=0,
                       suffix_enabled=False, verification_calls=0, verified_positions=0,
                       decode_tokens_per_second=0, first_token_ms=None, elapsed_seconds=0, kv_tokens=0,
                       context_limit=CONTEXT)
        try:
            if request.max_draft and request.decoding != 'greedy':
                raise ValueError('B2 suffix drafting supports greedy decoding only')
            yield dict(type='loading', message='Loading the MI355X engine…')
            self.start(cancel)
            metrics['suffix_enabled'] = bool(request.max_draft > 0 and request.decoding == 'greedy'
                                             and self.suffix_supported())
            reuse = self._reusable(request)
            if reuse:
                ack = self.command(f'rewind {reuse}', cancel, preserve_cache=True)
                if ack.get('ok') is not True or ack.get('position') != reuse:
                    raise RuntimeError('Engine rewind did not keep the reused prefix')
                self.cache_ids = self.cache_ids[:reuse]
                self.canonical_reusable_tokens = reuse
            else:
                ack = self.command('reset', cancel)
                if ack.get('ok') is not True or ack.get('position') != 0:
                    raise RuntimeError('Engine reset did not clear the context')
            metrics.update(reused_prefix_tokens=reuse, evaluated_prompt_tokens=len(request.ids) - reuse,
                           kv_tokens=reuse)
            seed = request.seed if request.seed is not None else secrets.randbits(32)
            mode = 'mode greedy' if request.decoding == 'greedy' else f'mode chat {seed}'
            if self.command(mode, cancel).get('ok') is not True:
                raise RuntimeError('Engine decoding mode was not acknowledged')
            yield dict(type='start', metrics=dict(metrics))
            response = self.command('prefill ' + ' '.join(map(str, request.ids[reuse:])), cancel,
                                    preserve_cache=True)
            if response.get('position') != len(request.ids):
                raise RuntimeError('Engine prefill position differs from the full prompt')
            self.cache_ids, self.cache_session = list(request.ids), request.session
            self.canonical_reusable_tokens = (len(request.ids) // CHUNK * CHUNK
                                              if self.prefix_reuse_supported() else 0)
            metrics.update(elapsed_seconds=time.perf_counter() - started, kv_tokens=len(request.ids))
            yield dict(type='prefill', processed_tokens=len(request.ids) - reuse, metrics=dict(metrics))
            drafter = self.drafter_factory() if self.drafter_factory else None
            produced = [response.get('token')]
            while len(out) < request.max_new:
                metrics['rounds'] += 1
                metrics['kv_tokens'] = len(self.cache_ids)
                for token in produced:
                    if cancel.is_set():
                        raise NativeCancelled()
                    if type(token) is not int or not 0 <= token < VOCABULARY:
                        raise RuntimeError('Invalid engine token')
                    if token in EOS:
                        reason = 'eos'
                        break
                    out.append(token)
                    now = time.perf_counter()
                    if first is None:
                        first = now
                        metrics['first_token_ms'] = (now - started) * 1e3
                    text = self.protocol.tokenizer.decode(out, skip_special_tokens=True)
                    metrics.update(output_tokens=len(out), tokens_per_round=len(out) / metrics['rounds'],
                                   elapsed_seconds=now - started,
                                   decode_tokens_per_second=(len(out) - 1) / (now - first) if now > first else 0)
                    yield dict(type='update', text=text, token_ids=list(out), metrics=dict(metrics))
                if reason == 'eos' or len(out) >= request.max_new:
                    break
                # The last emitted token is pending: it enters cache_ids only
                # once the engine consumes it. The reuse ceiling stays at the
                # prompt prefill.
                pending, remaining = out[-1], request.max_new - len(out)
                draft = []
                if (drafter and request.max_draft > 0 and self.suffix_supported() and remaining >= 2
                        and len(self.cache_ids) + 2 <= CONTEXT):
                    draft = drafter.propose(self.cache_ids + [pending], 1)
                if draft:
                    metrics['proposed_tokens'] += 1
                    metrics['verification_calls'] += 1
                    response = self.command(f'verify-greedy {pending} {draft[0]}', cancel, preserve_cache=True)
                    tokens, accepted, committed = self._check_verification(response, draft[0], remaining)
                    self.cache_ids.extend([pending, draft[0]][:committed])
                    metrics['accepted_tokens'] += accepted
                    metrics['rejected_tokens'] += 1 - accepted
                    metrics['verified_positions'] += 2
                    produced = tokens
                else:
                    response = self.command(f'step {pending}', cancel, preserve_cache=True)
                    if response.get('position') != len(self.cache_ids) + 1:
                        raise RuntimeError('Invalid engine step position')
                    self.cache_ids.append(pending)
                    produced = [response.get('token')]
            if cancel.is_set():
                raise NativeCancelled()
        except NativeCancelled:
            self.close()
            reason = 'stopped'
        except BaseException:
            self.close()
            raise
        metrics['elapsed_seconds'] = time.perf_counter() - started
        metrics['tokens_per_round'] = len(out) / metrics['rounds'] if metrics['rounds'] else 0
        yield dict(type='done', text=text, token_ids=list(out), metrics=dict(metrics), finish_reason=reason)
