"""Checkpoint -> QWCPU01 pack export (the counterpart of the reference's
tools/export_native_cpu_weights.py; format engine/INTERFACE.md:6-21).

No Qwen3 checkpoint exists in this environment, so the known answer that
needs one (`prefill 9707` -> 21806, tools/check_native_cpu_interface.py:50-62)
stays out of reach; these tests pin the conversion and every validation on
synthetic BF16 safetensors files instead, and check that a full-shape export
passes the engine's own pack validator.
"""
import importlib.util
import json
import struct
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
spec = importlib.util.spec_from_file_location('export_pack', ROOT / 'fpga-qwen_amd' / 'export_pack.py')
export_pack = importlib.util.module_from_spec(spec)
spec.loader.exec_module(export_pack)

SMALL = {'model.embed_tokens.weight': (8, 4), 'model.norm.weight': (4,),
         'model.layers.0.a.weight': (3, 4), 'model.layers.0.n.weight': (2,)}


def bf16(values):
    """Exact BF16 bit patterns of float32 values that are BF16-representable."""
    bits = np.asarray(values, np.float32).view(np.uint32)
    assert np.all(bits & 0xffff == 0)
    return (bits >> 16).astype('<u2')


def write_checkpoint(path, tensors, order=None, tail=b''):
    """tensors: name -> BF16 uint16 array (with its shape). Writes a
    safetensors file with regions in `order` (default: insertion order)."""
    names = order or list(tensors)
    header, blobs, cursor = {}, [], 0
    for name in names:
        data = tensors[name].astype('<u2').tobytes()
        header[name] = dict(dtype='BF16', shape=list(tensors[name].shape), data_offsets=[cursor, cursor + len(data)])
        blobs.append(data)
        cursor += len(data)
    raw = json.dumps(header).encode()
    path.write_bytes(struct.pack('<Q', len(raw)) + raw + b''.join(blobs) + tail)
    return path


def small_tensors(rng):
    out = {}
    for name, shape in SMALL.items():
        wide = rng.standard_normal(shape).astype(np.float32)
        out[name] = bf16((wide.view(np.uint32) & 0xffff0000).view(np.float32)).reshape(shape)
    out['lm_head.weight'] = out['model.embed_tokens.weight'].copy()
    return out


def test_small_export_layout_and_values(tmp_path):
    rng = np.random.default_rng(5)
    t = small_tensors(rng)
    # BF16 keeps fewer significand bits than FP16, so rounding happens only
    # below FP16's normal range: ties at half the subnormal step go to even
    # (2^-25 -> 0, 3*2^-25 -> 2*2^-24, 5*2^-25 -> 2*2^-24); also the largest
    # BF16 value under FP16's maximum (65280), -0 and normal values.
    special = np.array([2.0 ** -25, 3 * 2.0 ** -25, 5 * 2.0 ** -25, 2.0 ** -24, 65280.0, -0.0, 0.5, -3.0,
                        2.0 ** -14, 1.0, 2.0, 4.0], np.float32)
    t['model.layers.0.a.weight'] = bf16(special).reshape(3, 4)
    ckpt = write_checkpoint(tmp_path / 'model.safetensors', t, order=list(reversed(list(t))))
    manifest = export_pack.write_pack(tmp_path, tmp_path / 'out' / 'weights.bin', table=SMALL)
    pack = (tmp_path / 'out' / 'weights.bin').read_bytes()
    assert pack[:64] == b'QWCPU01' + bytes(57)
    lines = (tmp_path / 'out' / 'weights.bin.index').read_text().splitlines()
    assert lines[0] == 'QWCPU01 4'
    meta = json.loads(manifest.read_text())
    assert meta['format'] == 'QWCPU01' and meta['completed'] is True and meta['tensor_count'] == 4
    assert meta['tied_lm_head_verified'] is True
    for line, (name, shape) in zip(lines[1:], SMALL.items()):
        n, dtype, rows, cols, off, length = line.split()
        assert n == name and int(off) % 64 == 0
        wide = (t[name].astype(np.uint32) << 16).view(np.float32).reshape(-1)
        if len(shape) == 2:
            assert dtype == 'F16' and (int(rows), int(cols)) == shape
            got = np.frombuffer(pack[int(off):int(off) + int(length)], '<f2')
            assert np.array_equal(got.view(np.uint16), wide.astype(np.float16).view(np.uint16))
        else:
            assert dtype == 'F32' and (int(rows), int(cols)) == (shape[0], 1)
            got = np.frombuffer(pack[int(off):int(off) + int(length)], '<f4')
            assert np.array_equal(got.view(np.uint32), wide.view(np.uint32))
    off = int(lines[3].split()[4])
    got = np.frombuffer(pack[off:off + 24], '<u2')
    expected = [0x0000, 0x0002, 0x0002, 0x0001, 0x7BF8, 0x8000, 0x3800, 0xC200, 0x0400, 0x3C00, 0x4000, 0x4400]
    assert got.tolist() == expected
    # Outputs are immutable.
    with pytest.raises(FileExistsError):
        export_pack.write_pack(ckpt, tmp_path / 'out' / 'weights.bin', table=SMALL)


@pytest.mark.parametrize('case, message', [
    ('missing', 'are not the 5 of Qwen3-0.6B: missing'),
    ('extra', 'unexpected'),
    ('dtype', 'expected BF16 \\[4\\], found F32'),
    ('shape', 'expected BF16 \\[3, 4\\], found BF16 \\[4, 3\\]'),
    ('hole', 'a gap or an overlap'),
    ('tail', 'trailing bytes'),
    ('overlap', 'a gap or an overlap'),
    ('untied', 'tied head'),
    ('nan', 'non-finite'),
    ('overflow', 'beyond the FP16 range'),
    ('duplicate', 'repeats the key'),
])
def test_rejections(tmp_path, case, message):
    rng = np.random.default_rng(6)
    t = small_tensors(rng)
    kwargs = {}
    path = tmp_path / 'model.safetensors'
    if case == 'missing':
        del t['model.norm.weight']
    elif case == 'extra':
        t['model.extra.weight'] = bf16(np.ones(2, np.float32))
    elif case == 'untied':
        t['lm_head.weight'] = t['lm_head.weight'].copy()
        t['lm_head.weight'][0, 0] ^= 1
    elif case == 'nan':
        t['model.norm.weight'][1] = 0x7FC0
    elif case == 'overflow':
        t['model.layers.0.a.weight'][0, 0] = 0x4789  # 70144: beyond FP16's range
    elif case == 'tail':
        kwargs['tail'] = b'\0\0'
    if case in ('dtype', 'shape', 'hole', 'overlap', 'duplicate'):
        write_checkpoint(path, t)
        n = struct.unpack('<Q', path.read_bytes()[:8])[0]
        header = json.loads(path.read_bytes()[8:8 + n])
        data = path.read_bytes()[8 + n:]
        if case == 'dtype':
            header['model.norm.weight']['dtype'] = 'F32'
        elif case == 'shape':
            header['model.layers.0.a.weight']['shape'] = [4, 3]
        elif case == 'hole':
            for name in header:
                b, e = header[name]['data_offsets']
                header[name]['data_offsets'] = [b + 2, e + 2]
            data = b'\0\0' + data
        elif case == 'overlap':
            b, e = header['model.norm.weight']['data_offsets']
            header['model.norm.weight']['data_offsets'] = [b - 2, e - 2]
        raw = json.dumps(header).encode()
        if case == 'duplicate':
            raw = raw[:-1] + b', "model.norm.weight": {"dtype": "BF16", "shape": [4], "data_offsets": [0, 8]}}'
        path.write_bytes(struct.pack('<Q', len(raw)) + raw + data)
    else:
        write_checkpoint(path, t, **kwargs)
    with pytest.raises(ValueError, match=message):
        export_pack.write_pack(path, tmp_path / 'out' / 'weights.bin', table=SMALL)
    assert not (tmp_path / 'out' / 'weights.bin').exists()


def write_full_checkpoint(path, seed=7, gains=None):
    """A synthetic BF16 checkpoint with the exact Qwen3-0.6B tensor set: each
    matrix a differently rotated window of one N(0, 0.02) BF16 pattern, norm
    gains 1.0 (gains: {norm name suffix: (channels, value)} overrides them in
    every layer), lm_head a copy of the embedding."""
    shapes = export_pack.qwen3_tensor_table()
    rng = np.random.default_rng(seed)
    wide = rng.standard_normal(1 << 21).astype(np.float32) * 0.02
    pattern = bf16((wide.view(np.uint32) & 0xffff0000).view(np.float32))
    ones = bf16(np.ones(1, np.float32))[0]
    gains = gains or {}
    names = list(shapes) + ['lm_head.weight']
    header, cursor = {}, 0
    for name in names:
        shape = shapes['model.embed_tokens.weight'] if name == 'lm_head.weight' else shapes[name]
        size = 2 * int(np.prod(shape))
        header[name] = dict(dtype='BF16', shape=list(shape), data_offsets=[cursor, cursor + size])
        cursor += size
    raw = json.dumps(header).encode()
    with path.open('wb') as f:
        f.write(struct.pack('<Q', len(raw)) + raw)
        for index, name in enumerate(names):
            tied = name == 'lm_head.weight'
            shape = shapes['model.embed_tokens.weight'] if tied else shapes[name]
            count = int(np.prod(shape))
            if len(shape) == 1:
                norm = np.full(count, ones, '<u2')
                for suffix, (channels, value) in gains.items():
                    if name.endswith(suffix + '.weight'):
                        norm[list(channels)] = bf16(np.float32([value]))[0]
                f.write(norm.tobytes())
                continue
            window = np.roll(pattern, 7919 * (0 if tied else index))
            reps = -(-count // window.size)
            f.write(np.tile(window, reps)[:count].tobytes())
    return path


def test_full_shape_export_passes_engine_validation(tmp_path, qpkg):
    """The exported pack of a full-shape synthetic checkpoint passes the
    engine's own pack checks (qwen_gpu_validate_pack: the checks the engine
    runs before it touches a device, so the test is the same with or
    without one)."""
    path = write_full_checkpoint(tmp_path / 'model.safetensors')
    out = tmp_path / 'pack' / 'weights.bin'
    export_pack.write_pack(path, out)
    index = out.with_name('weights.bin.index').read_text().splitlines()
    assert index[0] == 'QWCPU01 310' and len(index) == 311
    qpkg.validate_pack(out)
    data = bytearray(out.read_bytes()[:64])
    assert data[:7] == b'QWCPU01'
    broken = tmp_path / 'broken' / 'weights.bin'
    broken.parent.mkdir()
    broken.with_name('weights.bin.index').write_text(
        out.with_name('weights.bin.index').read_text().replace('QWCPU01 310', 'QWCPU01 309', 1))
    broken.write_bytes(out.read_bytes())
    with pytest.raises(RuntimeError):
        qpkg.validate_pack(broken)


@pytest.mark.gpu
def test_exported_pack_runs_on_gpu_against_oracle(tmp_path, qpkg, oracle_lib):
    """An exported full-shape pack served by the engine on the GPU: the
    85-token prompt and 4 greedy steps, every position's logits against the
    oracle on the same exported file under the reference gate (max-abs 1e-2,
    RMS 2e-3, greedy identity)."""
    from oracle_binding import compare_logits
    path = write_full_checkpoint(tmp_path / 'model.safetensors')
    out = tmp_path / 'pack' / 'weights.bin'
    export_pack.write_pack(path, out)
    path.unlink()
    prompt = json.loads((ROOT / 'tests' / 'golden' / 'prompts.json').read_text())['decode_85']
    model = qpkg.Model(out, context=256)
    oracle = oracle_lib.model(out, 16, 16, 256)
    try:
        model.prefill(prompt)
        oracle.prefill(prompt)
        for step in range(5):
            result = compare_logits(model.logits(), oracle.logits())
            print('exported pack, position', model.position(), result, flush=True)
            assert result['passed'], (step, result)
            token = model.greedy()
            if step < 4:
                model.step(token)
                oracle.step(token)
    finally:
        model.close()
        oracle.close()


# Norm gains that drive the prefill and batched matrix-core inputs far past
# FP16's range (65504): 32768 in 8 channels of every layer's input and
# post-attention norms.
LARGE_GAINS = {'input_layernorm': ((3, 200, 411, 517, 640, 777, 901, 1013), 32768.0),
               'post_attention_layernorm': ((3, 200, 411, 517, 640, 777, 901, 1013), 32768.0)}


@pytest.mark.gpu
def test_large_activations_against_oracle(tmp_path, qpkg, oracle_lib):
    """FP32 activations beyond FP16's range (engine/core.cpp:292-294 keeps
    them FP32): an exported pack with norm gains of 32768 in 8 channels
    (LARGE_GAINS) makes about a third of the normalized rows exceed 65504 in
    layer 0 already (checked below from the pack's embedding rows), and the
    SwiGLU activations reach the millions. The 1024-token prompt (two
    512-row prefill chunks on the matrix cores, every input split under the
    range guard), 2 decode steps, and one batched step of two sequences
    sharing the weights, every row's logits against the oracle on the same
    file under the reference gate (max-abs 1e-2, RMS 2e-3, greedy
    identity)."""
    from oracle_binding import compare_logits
    path = write_full_checkpoint(tmp_path / 'model.safetensors', gains=LARGE_GAINS)
    out = tmp_path / 'pack' / 'weights.bin'
    export_pack.write_pack(path, out)
    path.unlink()
    prompts = json.loads((ROOT / 'tests' / 'golden' / 'prompts.json').read_text())
    prompt, other = prompts['prefill_1024'], prompts['decode_85']
    # Layer 0's normalized rows: the pack's FP16 embedding rows of the prompt
    # times the input norm gains (FP32 norm of engine/core.cpp:207-215).
    slots = {slot.name: slot for slot in export_pack.plan(export_pack.qwen3_tensor_table())[0]}
    blob = np.memmap(out, np.uint8, 'r')
    emb = slots['model.embed_tokens.weight']
    table = blob[emb.offset:emb.offset + emb.length].view(np.float16).reshape(emb.shape)
    rows = table[prompt].astype(np.float64)
    gain = blob[slots['model.layers.0.input_layernorm.weight'].offset:][:4096].view(np.float32)
    normed = rows / np.sqrt((rows ** 2).mean(axis=1, keepdims=True) + 1e-6) * gain
    share = float((np.abs(normed).max(axis=1) >= 65504).mean())
    print('rows of layer 0 past FP16 range', share, flush=True)
    assert share > 0.1
    del blob, table
    model = qpkg.Model(out, context=1100)
    second = model.share()
    oracle = oracle_lib.model(out, 16, 16, 1100)
    oracle2 = oracle_lib.model(out, 16, 16, 1100)
    try:
        model.prefill(prompt)
        oracle.prefill(prompt)
        second.prefill(other)
        oracle2.prefill(other)
        for step in range(3):
            result = compare_logits(model.logits(), oracle.logits())
            print('large gains, position', model.position(), result, flush=True)
            assert result['passed'], (step, result)
            if step < 2:
                token = model.greedy()
                model.step(token)
                oracle.step(token)
        tokens = [model.greedy(), second.greedy()]
        qpkg.step_batch([model, second], tokens)
        oracle.step(tokens[0])
        oracle2.step(tokens[1])
        for m, o in ((model, oracle), (second, oracle2)):
            result = compare_logits(m.logits(), o.logits())
            print('large gains, batched, position', m.position(), result, flush=True)
            assert result['passed'], result
    finally:
        second.close()
        model.close()
        oracle.close()
        oracle2.close()
