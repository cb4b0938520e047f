#!/usr/bin/env python3
"""Batch-1 greedy decode throughput of Qwen3-0.6B FP16 on one MI355X.

Workload (one "step" = one decode token through all 28 layers, the tied
lm_head and the device argmax): seeded random-init FP16 weights (pack seed 0,
N(0, 0.02), norm gains 1.0); after one unscored warm-up request (the prompt
and 100 steps), the 85-token prompt (ids seed 0) prefilled, then W untimed
and K timed greedy steps. Weights, KV cache and activations are
resident in HBM before the timed region. Also reported: TTFT for the 85-,
1024- and 3968-token prompts, per-kernel times, the roofline of the dominant
kernel, and the oracle CPU engine timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / 'tests'))

HBM_PEAK_GBS = 8000.0
# Engine kernel ids (time_kernel). A decode step runs 'token' (all 28 layers
# in one launch) and 'lm_head' (+ the argmax). 'qkv_attention' (norm + QKV +
# attention + O) and 'ffn' (norm + gate/up + SwiGLU + down) are the two
# per-layer kernels of the engine's two-kernel step, and 'qkv', 'attention',
# 'gate_up' and 'down' the separate kernels those replace (timed for
# comparison, not run by a step).
KERNELS = ['qkv', 'attention', 'o', 'gate_up', 'down', 'lm_head', 'ffn', 'qkv_attention', 'token']
# Launches of each kernel per decode token.
PER_TOKEN = {'token': 1, 'lm_head': 1}
# One layer's weights: QKV, O, gate/up, down (FP16).
LAYER_WEIGHT_BYTES = (4096 * 1024 + 1024 * 2048 + 6144 * 1024 + 1024 * 3072) * 2
# Algorithmic bytes per launch: FP16 weights + FP32 vectors read/written.
KERNEL_BYTES = {
    'qkv': 4096 * 1024 * 2 + 1024 * 4 * 2 + 4096 * 4 + 8 * 1024 * 4,  # + the 8 down slices folded in
    'o': 1024 * 2048 * 2 + 2048 * 4 + 1024 * 4 * 2,
    'gate_up': 6144 * 1024 * 2 + 1024 * 4 * 2 + 3072 * 4,
    'down': 1024 * 3072 * 2 + 3072 * 4 + 1024 * 4 * 2,
    'lm_head': 151936 * 1024 * 2 + 1024 * 4 * 2 + 151936 * 4,
    # gate/up + down weights, x, norm weights, 16 O partials, xm and the 8
    # down slices written, the 3072 tagged activations exchanged.
    'ffn': 6144 * 1024 * 2 + 1024 * 3072 * 2 + 1024 * 4 * 3 + 16 * 1024 * 4 + 8 * 1024 * 4 + 3072 * 8,
}


# Contexts up to this many positions run attention and the O projection as
# one kernel (the engine's fused path); beyond it split attention and a
# merge + O kernel. The O projection is never a kernel of its own.
FUSED_ATTENTION_MAX = 512
# Up to this many cached positions every workgroup of the fused QKV +
# attention kernel attends its head over all positions.
FULL_ATTENTION_MAX = 256


def attention_bytes(n):
    """The attention stage (attention + O partials): K and V rows of 8 heads x
    128 FP16 for n positions, q/k/v in, the O weights and the 16 x 1024 FP32
    partial projections written; past the fused range also the split
    partials written and read back by the merge."""
    base = 8 * n * 128 * 2 * 2 + 4096 * 4 + 1024 * 2048 * 2 + 16 * 1024 * 4
    if n <= FUSED_ATTENTION_MAX:
        return base
    splits = (n + 127) // 128
    return base + 2 * 8 * splits * 264 * 4


def kernel_bytes(kernel, n):
    """Algorithmic bytes of one launch with n cached positions."""
    if kernel == 'attention':
        return attention_bytes(n)
    if kernel == 'token':
        # Per layer: the weights, the K/V rows of n positions (one of them
        # written), the two norm weights and the QK-norm weights; once: the
        # embedding row read and the final residual written. The exchange
        # words between workgroups stay in the L2s and are not counted.
        return 28 * (LAYER_WEIGHT_BYTES + 8 * n * 128 * 2 * 2 + 2 * 1024 * 4 + 256 * 4) + 1024 * 2 + 1024 * 4
    if kernel == 'qkv_attention':
        # QKV and O weights, K/V rows, residual (+ the 8 down slices) in and
        # out, norm weights, the 16 partial O projections written.
        return (4096 * 1024 * 2 + 1024 * 2048 * 2 + 8 * n * 128 * 2 * 2 + 1024 * 4 * (2 + 8) + 1024 * 4
                + 16 * 1024 * 4)
    return KERNEL_BYTES[kernel]


def kernel_replays(model, history, iterations=224):
    """Average duration of each decode kernel at the model's position (HIP
    events on the engine stream; layer kernels rotate over the layers, the
    token kernel replays whole steps). Timing an attention kernel or the
    token kernel rewrites cached K/V and resets the model, so the context
    `history` is prefilled again before each of those."""
    kernel_ms = {}
    for which in (0, 6, 3, 4, 5, 1):
        kernel_ms[KERNELS[which]] = model.time_kernel(which, iterations)
    model.prefill(history)
    kernel_ms['qkv_attention'] = model.time_kernel(7, iterations)
    model.prefill(history)
    kernel_ms['token'] = model.time_kernel(8, max(8, iterations // 28))
    return kernel_ms


def measured_traffic(kernel, position):
    """Calibrated HBM bytes per dispatch of a decode kernel with `position`
    cached positions (the step writes position - 1), from the committed
    rocprofv3 counter summary (lines 'traffic KERNEL POSITIONS BYTES').
    Kernels whose traffic does not depend on the context use their one
    measurement. The attention stages read 8 x n x 512 bytes of K/V, so their
    traffic is linear in n on each path (the separate attention kernels:
    fused up to 512 cached positions, split beyond; the fused QKV +
    attention kernel: whole-context workgroups up to 256, passes beyond):
    the line through the two measurements on the same path is evaluated at
    n. Returns (bytes, how) or (None, reason)."""
    path = ROOT / 'profiles' / 'decode_hbm_traffic.txt'
    if not path.exists():
        return None, 'no counter summary'
    points = []
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) == 4 and parts[0] == 'traffic' and parts[1] == kernel:
            points.append((int(parts[2]), float(parts[3])))
    if kernel not in ('attention', 'qkv_attention', 'token'):  # no dependence on the context
        return (points[0][1], f'measured at position {points[0][0]}') if points else (None, 'not measured')
    # Paths: the separate attention kernels switch at 512 cached positions,
    # the fused QKV + attention kernel and the token kernel at 256 (every
    # workgroup attending its head over all positions up to there, passes of
    # 64 positions split over the workgroups beyond).
    limit = FUSED_ATTENTION_MAX if kernel == 'attention' else FULL_ATTENTION_MAX
    same = sorted(p for p in points if (p[0] <= limit) == (position <= limit))
    if any(p[0] == position for p in same):
        return dict(same)[position], f'measured at position {position}'
    if len(same) < 2:
        return None, 'fewer than two measurements on this attention path'
    (p0, b0), (p1, b1) = same[0], same[-1]
    return b0 + (b1 - b0) * (position - p0) / (p1 - p0), f'line through positions {p0} and {p1}'


def _median_ci(values, seed=0, draws=2000):
    """Median and a 95% bootstrap interval of the median."""
    import numpy as np
    v = np.asarray(values, dtype=np.float64)
    rng = np.random.default_rng(seed)
    medians = np.median(rng.choice(v, size=(draws, v.size), replace=True), axis=1)
    return float(np.median(v)), [float(np.percentile(medians, 2.5)), float(np.percentile(medians, 97.5))]


# Prompt, output tokens: the reference's published rows for the 85-, 1024-
# and 3968-token prompts (32 / 128 / 128 outputs).
PROTOCOL_CASES = (('85', 'decode_85', 32), ('1024', 'prefill_1024', 128), ('3968', 'long_3968', 128))


def generation_protocol(model, ids, outputs, warmups=1, repeats=10):
    """The reference's request measurement (tools/benchmark_matched.py:39-48,
    tools/benchmark_native_cpu.py:248-272): per run the model is reset, TTFT
    is prefill -> first greedy token, then N - 1 greedy steps, and decode is
    (N - 1) / (t_last - t_first). One unscored warmup, then `repeats` scored
    runs whose greedy ids must all be the same; medians with 95% bootstrap
    intervals."""
    ttft, decode, expected = [], [], None
    for run in range(warmups + repeats):
        model.reset()
        t0 = time.perf_counter()
        model.prefill(ids)
        token = model.greedy()
        t_first = time.perf_counter()
        produced = [token]
        for _ in range(outputs - 1):
            model.step(token)
            token = model.greedy()
            produced.append(token)
        t_last = time.perf_counter()
        if expected is None:
            expected = produced
        elif produced != expected:
            raise RuntimeError('greedy output changed between runs')
        if run >= warmups:
            ttft.append((t_first - t0) * 1e3)
            decode.append((outputs - 1) / (t_last - t_first))
    ttft_median, ttft_ci = _median_ci(ttft)
    decode_median, decode_ci = _median_ci(decode)
    return dict(prompt_tokens=len(ids), output_tokens=outputs, warmups=warmups, repeats=repeats,
                ttft_ms_median=ttft_median, ttft_ms_ci95=ttft_ci, decode_tok_s_median=decode_median,
                decode_tok_s_ci95=decode_ci, ttft_ms=ttft, decode_tok_s=decode)


def long_context_decode(model, prompt, steps=128):
    """128 greedy steps after the 3968-token prompt (positions 3968..4095),
    then per-kernel times at the full 4096 context."""
    model.reset()
    model.prefill(prompt)
    token = model.greedy()
    history = list(prompt)
    start = time.perf_counter()
    for _ in range(steps):
        model.step(token)
        history.append(token)
        token = model.greedy()
    elapsed = time.perf_counter() - start
    n = model.position()
    assert n == 4096, n
    kernel_ms = kernel_replays(model, history)
    gbs = {k: kernel_bytes(k, n) / (v * 1e-3) / 1e9 for k, v in kernel_ms.items()}
    log(f'long-context decode {steps / elapsed:.1f} tok/s')
    return {'prompt_tokens': 3968, 'steps': steps, 'decode_tok_s': steps / elapsed, 'context_end': n,
            'kernel_ms': kernel_ms, 'kernel_gbs': gbs}


def prefix_reuse_batch(model, prompts, steps=128):
    """Prefix-reuse workload: the canonical 512-token prefix is prefilled once;
    8 sequences on the same weights reuse its K/V (device copy of the rewound
    prefix), prefill their own 1536-token suffix (positions 512..2047) and
    decode 128 greedy tokens each as one batch of 8 (skinny GEMMs on the
    matrix cores; each step returns the 8 selections). Also times one
    sequence stepping alone at that context."""
    prefix, suffixes = prompts['prefix_512'], prompts['suffix_1536']
    base = model.share()
    seqs = [model.share() for _ in suffixes]
    q = sys.modules['fpga_qwen_amd']
    try:
        t0 = time.perf_counter()
        base.prefill(prefix)
        prefix_s = time.perf_counter() - t0
        suffix_s = []
        for m, suffix in zip(seqs, suffixes):
            t0 = time.perf_counter()
            m.copy_prefix(base, len(prefix))
            m.prefill(suffix)
            suffix_s.append(time.perf_counter() - t0)
        tokens = [m.greedy() for m in seqs]
        tokens = q.step_batch_greedy(seqs, tokens)  # warmup step
        start = time.perf_counter()
        for _ in range(steps - 1):
            tokens = q.step_batch_greedy(seqs, tokens)
        elapsed = time.perf_counter() - start
        aggregate = len(seqs) * (steps - 1) / elapsed
        # The same context stepped one sequence at a time (batch-1 path).
        single = seqs[0]
        single.truncate(single.position() - 16)
        token = 0
        t0 = time.perf_counter()
        for _ in range(16):
            single.step(token)
            token = single.greedy()
        single_tps = 16 / (time.perf_counter() - t0)
        context_end = seqs[1].position()
    finally:
        for m in seqs + [base]:
            m.close()
    log(f'prefix reuse: {aggregate:.0f} tok/s aggregate over {len(seqs)} sequences')
    return {'sequences': len(suffixes), 'prefix_tokens': len(prefix), 'suffix_tokens': len(suffixes[0]),
            'steps': steps, 'timed_steps': steps - 1, 'aggregate_tok_s': aggregate,
            'step_ms': elapsed / (steps - 1) * 1e3, 'context_end': context_end,
            'prefix_prefill_ms': prefix_s * 1e3, 'suffix_prefill_ms': sorted(suffix_s)[len(suffix_s) // 2] * 1e3,
            'single_sequence_tok_s': single_tps}


def verification_pairs(model, token, pairs=32):
    """Two-token greedy verification as a drafting loop uses it (the
    protocol's verify-greedy): `pairs` calls of verify_two_greedy, each
    committing both positions, against the same positions stepped one at a
    time. The pair runs both rows in one pass over the weights."""
    start_pos = model.position()
    t0 = time.perf_counter()
    for _ in range(pairs):
        _, token = model.verify_two_greedy(token, token)
        model.commit_verified(2)
    pair_ms = (time.perf_counter() - t0) / pairs * 1e3
    model.truncate(start_pos)
    t0 = time.perf_counter()
    for _ in range(pairs):
        model.step(token)
        model.step(token)
    steps_ms = (time.perf_counter() - t0) / pairs * 1e3
    model.truncate(start_pos)
    log(f'verification pair {pair_ms:.3f} ms vs two steps {steps_ms:.3f} ms')
    return {'positions': [start_pos, start_pos + 2 * pairs], 'pairs': pairs, 'pair_ms': pair_ms,
            'two_steps_ms': steps_ms, 'speedup': steps_ms / pair_ms}


# Decode projection shapes (in, out) of the isolated GEMV microbenchmark.
GEMV_SHAPES = [(1024, 2048), (1024, 1024), (2048, 1024), (1024, 3072), (3072, 1024), (1024, 151936)]


def gemv_microbench(q, seed=1, rotate_bytes=640 << 20):
    """Plain chain-ordered GEMV at each decode shape: W ~ N(0, 0.02) FP16,
    x ~ N(0, 1) FP32 (seed 1), cycling through enough weight copies (at least
    640 MB) that they stream from HBM instead of the Infinity Cache. Bytes
    per call: 2 in out + 4 in + 4 out."""
    import numpy as np
    rng = np.random.default_rng(seed)
    out = {}
    for n_in, n_out in GEMV_SHAPES:
        w = (rng.standard_normal((n_out, n_in), dtype=np.float32) * 0.02).astype(np.float16)
        x = rng.standard_normal(n_in, dtype=np.float32)
        tiled = q.tile_matrix(w)
        del w
        size = n_out * n_in * 2
        copies = max(2, -(-rotate_bytes // size))
        copies_buf = q.DeviceBuffer(size * copies)
        for i in range(copies):
            q.copy_device(tiled, q.DeviceView(copies_buf, i * size), size)
        q.synchronize()
        xd, yd = q.DeviceBuffer.from_array(x), q.DeviceBuffer(n_out * 4)
        iterations = max(copies, 20 if n_out > 100000 else 400)
        ms = q.gemv_time(copies_buf, size, copies, xd, yd, n_out, n_in, iterations)
        nbytes = 2 * n_in * n_out + 4 * n_in + 4 * n_out
        out[f'{n_in}x{n_out}'] = {'us': ms * 1e3, 'gbs': nbytes / (ms * 1e-3) / 1e9, 'copies': copies}
        log(f'gemv {n_in}->{n_out}: {ms * 1e3:.2f} us, {nbytes / (ms * 1e-3) / 1e9:.0f} GB/s')
        del tiled, copies_buf, xd, yd
    return out


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def cpu_baseline(pack, prompt, seconds):
    """Oracle engine (CPU restatement) on this host: 12 decode / 6 prefill workers."""
    from oracle_binding import OracleLib
    cores = os.cpu_count() or 1
    decode_threads, prefill_threads = min(12, cores), min(6, cores)
    oracle = OracleLib().model(pack, decode_threads, prefill_threads, 4096)
    try:
        oracle.prefill(prompt)
        token = int(oracle.logits().argmax())
        oracle.step(token)  # warmup
        token = int(oracle.logits().argmax())
        steps, start = 0, time.perf_counter()
        while time.perf_counter() - start < seconds:
            oracle.step(token)
            token = int(oracle.logits().argmax())
            steps += 1
        elapsed = time.perf_counter() - start
    finally:
        oracle.close()
    return dict(value=steps / elapsed, unit='tok/s', cores=decode_threads, kind='port',
                sample=f'85-token prompt, then {steps} greedy decode steps ({elapsed:.1f} s) with '
                       f'{decode_threads} decode / {prefill_threads} prefill workers on {cores} host cores')


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument('--gpus', type=int, default=1)
    parser.add_argument('--steps', type=int, default=256)
    parser.add_argument('--warmup', type=int, default=16)
    parser.add_argument('--cpu-seconds', type=float, default=12.0)
    parser.add_argument('--no-cpu-baseline', action='store_true')
    parser.add_argument('--no-ttft', action='store_true', help='skip the 1024/3968 prefills and long-context decode')
    parser.add_argument('--no-gemv', action='store_true', help='skip the isolated GEMV microbenchmark')
    parser.add_argument('--no-batch', action='store_true', help='skip the 8-sequence prefix-reuse workload')
    parser.add_argument('--pmc-kernel', choices=KERNELS,
                        help='only replay one decode kernel (28 + 28 layer launches, or 2 + 8 token-kernel '
                             'steps) at one position (hardware-counter passes)')
    parser.add_argument('--pmc-positions', type=int,
                        help='cached positions for --pmc-kernel (default: where the timed region ends)')
    parser.add_argument('--pmc-prefill', type=int, nargs='?', const=1024, choices=(1024, 3968),
                        help='only run one batched prefill of the 1024- (default) or 3968-token prompt '
                             '(hardware-counter passes)')
    parser.add_argument('--pmc-batch', type=int, nargs='?', const=4, metavar='STEPS',
                        help='only set up the 8-sequence prefix-reuse batch and run STEPS (default 4) batched '
                             'decode steps after one warmup step (hardware-counter passes)')
    parser.add_argument('--copy-calibration', type=int, metavar='MIB',
                        help='only run a plain device copy of MIB MiB, 5 times (HBM byte-counter calibration)')
    args = parser.parse_args()
    if args.pmc_kernel:
        # Light run for hardware-counter passes (each profiled dispatch is
        # slow): one batched prefill up to the position the timed region of
        # the default run ends at, then replays of one decode kernel there
        # (the same context the per-kernel timings below use).
        from conftest import GOLDEN, PACK_CACHE, load_package
        q = load_package()
        prompts = json.loads((GOLDEN / 'prompts.json').read_text())
        model = q.Model(q.ensure_random_pack(PACK_CACHE / 'seed0', seed=0), context=4096)
        position = args.pmc_positions or 85 + args.warmup + args.steps
        prompt = (prompts['long_3968'] + prompts['prefill_1024'])[:position]
        model.prefill(prompt)
        which = KERNELS.index(args.pmc_kernel)
        launches = 8 if args.pmc_kernel == 'token' else 28
        ms = model.time_kernel(which, launches)
        model.close()
        warm = 2 if args.pmc_kernel == 'token' else 28
        print(json.dumps({'pmc_kernel': args.pmc_kernel, 'position': position, 'launches': launches + warm,
                          'avg_ms': ms}))
        return 0
    if args.pmc_prefill:
        from conftest import GOLDEN, PACK_CACHE, load_package
        q = load_package()
        prompts = json.loads((GOLDEN / 'prompts.json').read_text())
        model = q.Model(q.ensure_random_pack(PACK_CACHE / 'seed0', seed=0), context=4096)
        name = 'prefill_1024' if args.pmc_prefill == 1024 else 'long_3968'
        t0 = time.perf_counter()
        model.prefill(prompts[name])
        token = model.greedy()
        model.close()
        print(json.dumps({'pmc_prefill': args.pmc_prefill, 'seconds': time.perf_counter() - t0, 'token': token}))
        return 0
    if args.pmc_batch:
        from conftest import GOLDEN, PACK_CACHE, load_package
        q = load_package()
        prompts = json.loads((GOLDEN / 'prompts.json').read_text())
        model = q.Model(q.ensure_random_pack(PACK_CACHE / 'seed0', seed=0), context=4096)
        base = model.share()
        seqs = [model.share() for _ in prompts['suffix_1536']]
        try:
            base.prefill(prompts['prefix_512'])
            for m, suffix in zip(seqs, prompts['suffix_1536']):
                m.copy_prefix(base, len(prompts['prefix_512']))
                m.prefill(suffix)
            tokens = [m.greedy() for m in seqs]
            for _ in range(1 + args.pmc_batch):
                q.step_batch(seqs, tokens)
                tokens = [m.greedy() for m in seqs]
            position = seqs[0].position()
        finally:
            for m in seqs + [base]:
                m.close()
            model.close()
        print(json.dumps({'pmc_batch_steps': args.pmc_batch, 'sequences': len(seqs), 'position': position}))
        return 0
    if args.copy_calibration:
        from conftest import load_package
        q = load_package()
        nbytes = args.copy_calibration << 20
        src, dst = q.DeviceBuffer(nbytes), q.DeviceBuffer(nbytes)
        for _ in range(5):
            q.copy_device(src, dst, nbytes)
        q.synchronize()
        print(json.dumps({'copy_calibration_bytes': nbytes, 'launches': 5}))
        return 0
    if args.gpus != 1:
        print(f'bench.py measures one GPU only (asked for --gpus {args.gpus}); this engine is single-GPU '
              'batch-1 decode and has no multi-GPU path to time.', file=sys.stderr)
        return 2
    if 85 + args.warmup + args.steps > 4096:
        print('warmup + steps exceed the 4096-token context', file=sys.stderr)
        return 2

    from conftest import GOLDEN, PACK_CACHE, load_package
    q = load_package()
    prompts = json.loads((GOLDEN / 'prompts.json').read_text())
    pack = q.ensure_random_pack(PACK_CACHE / 'seed0', seed=0)
    log('pack ready', pack)
    model = q.Model(pack, context=4096)
    prompt = prompts['decode_85']

    # One unscored warm-up request (the prompt and 100 greedy steps) ahead of
    # the measured one, as the reference's benchmark runs one per process
    # before its scored requests (tools/benchmark_native_cpu.py:114,
    # 258-262: "startup and warmup excluded"). After the idle of loading, or
    # any pause of 0.2 s or more, the GPU's first ~25 steps run 7-8 us
    # slower than the same steps once it has been busy.
    model.prefill(prompt)
    token = model.greedy()
    for _ in range(100):
        model.step(token)
        token = model.greedy()
    model.reset()
    log('warm-up request done')

    t0 = time.perf_counter()
    model.prefill(prompt)
    token = model.greedy()
    ttft_85 = time.perf_counter() - t0
    history = list(prompt)  # every id the model has consumed
    for _ in range(args.warmup):
        model.step(token)
        history.append(token)
        token = model.greedy()
    log('warmup done')
    # Timed region: exactly K greedy steps; each step returns after the device
    # has finished (stream synchronized inside the engine).
    start = time.perf_counter()
    for _ in range(args.steps):
        model.step(token)
        history.append(token)
        token = model.greedy()
    elapsed = time.perf_counter() - start
    decode_tps = args.steps / elapsed
    log(f'decode {decode_tps:.1f} tok/s')
    context_end = model.position()
    verification = verification_pairs(model, token)

    # Per-kernel average durations with HIP events on the engine stream, at
    # the context length reached by the timed region.
    kernel_ms = kernel_replays(model, history)
    kernel_ms = {name: kernel_ms.get(name) for name in KERNELS}  # 'o' runs with the attention
    per_token_ms = {k: v * PER_TOKEN[k] for k, v in kernel_ms.items() if v is not None and k in PER_TOKEN}
    dominant = max(per_token_ms, key=per_token_ms.get)
    nbytes = kernel_bytes(dominant, context_end)
    achieved = nbytes / (kernel_ms[dominant] * 1e-3) / 1e9
    # The replays write position context_end - 1 over context_end cached positions.
    traffic, traffic_source = measured_traffic(dominant, context_end)
    log('kernel ms', kernel_ms)

    protocol, long_context = {}, None
    ttft = {'85': ttft_85}
    if not args.no_ttft:
        for key, name, outputs in PROTOCOL_CASES:
            protocol[key] = generation_protocol(model, prompts[name], outputs)
            ttft[key] = protocol[key]['ttft_ms_median'] * 1e-3
            log(f"prompt {key}: TTFT {protocol[key]['ttft_ms_median']:.2f} ms, "
                f"decode {protocol[key]['decode_tok_s_median']:.0f} tok/s (medians of 10)")
        long_context = long_context_decode(model, prompts['long_3968'])
    batch = None if args.no_batch else prefix_reuse_batch(model, prompts)
    model.close()
    gemv = None if args.no_gemv else gemv_microbench(q)

    baseline = None if args.no_cpu_baseline else cpu_baseline(pack, prompt, args.cpu_seconds)
    weight_bytes = 1191968768
    kv_bytes = 114688 * (85 + args.warmup + args.steps / 2)
    result = {
        'metric': 'decode tok/s (batch-1 greedy, Qwen3-0.6B FP16, 85-token prompt)',
        'value': decode_tps,
        'unit': 'tok/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': 1000.0 / decode_tps,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f16 weights/KV, f32 activations and accumulation',
        'data': 'synthetic: random-init FP16 weights N(0,0.02) seed 0; prompt ids uniform seed 0',
        'config': {'workload': 'Qwen3-0.6B FP16 batch-1 greedy decode after an 85-token prompt',
                   'prompt_tokens': 85, 'context': 4096, 'parallelism': 'none (1 GPU)'},
        'ttft_s': ttft,
        'decode_hbm_fraction': (weight_bytes + kv_bytes) * decode_tps / 1e9 / HBM_PEAK_GBS,
        'kernel_ms': kernel_ms,
        'roofline': {'kernel': dominant, 'bound': 'hbm', 'achieved': achieved, 'peak': HBM_PEAK_GBS,
                     'unit': 'GB/s', 'frac': achieved / HBM_PEAK_GBS, 'traffic': traffic,
                     'traffic_source': traffic_source, 'cached_positions': context_end,
                     'bytes_per_launch': nbytes},
        'reference_protocol': protocol,
        'cpu_baseline': baseline,
        'verification_pair': verification,
        'long_context_decode': long_context,
        'prefix_reuse_batch': batch,
        'gemv_microbench': gemv,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
