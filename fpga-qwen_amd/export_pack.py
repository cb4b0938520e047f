#!/usr/bin/env python3
"""Real-checkpoint pack writer: a Qwen3-0.6B BF16 ``model.safetensors`` ->
the QWCPU01 pack the engine loads (``weights.bin``, ``.index``,
``.manifest.json``), in the format of engine/INTERFACE.md:6-21 and with the
checks of the reference's exporter (tools/export_native_cpu_weights.py:49-163):

* the safetensors header is read once (8-byte little-endian length, JSON
  without duplicate keys) and must list exactly the 311 expected tensors
  (310 pack tensors plus ``lm_head.weight``), every one BF16 with its exact
  shape and length, the regions tiling the data area with no gaps, overlaps
  or trailing bytes;
* ``lm_head.weight`` must equal the embedding byte for byte and is then
  omitted (the engine ties the output head to the embedding);
* values are widened BF16 -> FP32; 2-D matrices are rounded to FP16
  (round-to-nearest-even), 1-D norms stay FP32; nonfinite inputs and FP16
  overflow are rejected;
* tensors go out in the engine's fixed order at 64-byte aligned offsets
  after a 64-byte ``QWCPU01`` header; the outputs are immutable: existing
  files are never replaced, and the three files appear only once complete
  (hard links from a staging directory, manifest last).

Streams the checkpoint in 1 MiB blocks; needs no GPU and no Torch.

Usage: python export_pack.py --checkpoint DIR_OR_FILE --output weights.bin
"""
import argparse
import hashlib
import json
import os
import struct
import tempfile
from pathlib import Path

import numpy as np

MAGIC = b'QWCPU01'
ALIGN = 64
BLOCK = 1 << 20
ROUNDING = ('BF16 widened to FP32; matrices rounded to FP16 round-to-nearest-even; '
            '1D norms preserved FP32; little endian')


def pack_shapes():
    """Pack tensors in the engine's order (name -> shape); matches
    fpga-qwen_amd/csrc/pack.cpp pack_layout()."""
    shapes = {'model.embed_tokens.weight': (151936, 1024), 'model.norm.weight': (1024,)}
    per_layer = [('input_layernorm', (1024,)), ('post_attention_layernorm', (1024,)),
                 ('self_attn.q_norm', (128,)), ('self_attn.k_norm', (128,)),
                 ('self_attn.q_proj', (2048, 1024)), ('self_attn.k_proj', (1024, 1024)),
                 ('self_attn.v_proj', (1024, 1024)), ('self_attn.o_proj', (1024, 2048)),
                 ('mlp.gate_proj', (3072, 1024)), ('mlp.up_proj', (3072, 1024)),
                 ('mlp.down_proj', (1024, 3072))]
    for layer in range(28):
        for name, shape in per_layer:
            shapes[f'model.layers.{layer}.{name}.weight'] = shape
    return shapes


def _sha256(path):
    digest = hashlib.sha256()
    with open(path, 'rb') as f:
        while True:
            block = f.read(BLOCK)
            if not block:
                return digest.hexdigest()
            digest.update(block)


def _no_duplicates(pairs):
    out = {}
    for key, value in pairs:
        if key in out:
            raise ValueError(f'Duplicate JSON key: {key}')
        out[key] = value
    return out


def read_header(source):
    """(header dict, data start, file size) of a safetensors file."""
    size = source.stat().st_size
    with source.open('rb') as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError('Truncated safetensors header')
        length = struct.unpack('<Q', raw)[0]
        if length < 2 or length > min(64 << 20, size - 8):
            raise ValueError('Invalid safetensors header length')
        header = json.loads(f.read(length), object_pairs_hook=_no_duplicates)
    if not isinstance(header, dict):
        raise ValueError('Invalid safetensors header')
    return header, 8 + length, size


def check_layout(header, data_start, size, shapes):
    """Validates names, dtypes, shapes and the tiling of the data area;
    returns {name: (begin, end)} relative to the data start."""
    expected = dict(shapes)
    expected['lm_head.weight'] = shapes['model.embed_tokens.weight']
    tensors = {k: v for k, v in header.items() if k != '__metadata__'}
    if set(tensors) != set(expected):
        raise ValueError(f'Checkpoint must contain exactly the expected {len(expected)} tensors')
    regions = {}
    for name, shape in expected.items():
        spec = tensors[name]
        if not isinstance(spec, dict) or spec.get('dtype') != 'BF16' or spec.get('shape') != list(shape):
            raise ValueError(f'Unexpected tensor dtype/shape: {name}')
        offsets = spec.get('data_offsets')
        if not isinstance(offsets, list) or len(offsets) != 2 or any(type(v) is not int for v in offsets):
            raise ValueError(f'Invalid offsets: {name}')
        begin, end = offsets
        if begin < 0 or end - begin != 2 * int(np.prod(shape)) or data_start + end > size:
            raise ValueError(f'Tensor bounds/length mismatch: {name}')
        regions[name] = (begin, end)
    spans = sorted(regions.values())
    if spans[0][0] != 0 or data_start + spans[-1][1] != size or any(
            a[1] != b[0] for a, b in zip(spans, spans[1:])):
        raise ValueError('Checkpoint tensor regions overlap, contain holes, or leave trailing bytes')
    return regions


def _same_bytes(path, a, b, length):
    with open(path, 'rb') as fa, open(path, 'rb') as fb:
        fa.seek(a)
        fb.seek(b)
        while length:
            n = min(length, BLOCK)
            if fa.read(n) != fb.read(n):
                return False
            length -= n
    return True


def convert_block(raw, matrix, name):
    """BF16 bytes -> FP16 (matrix) or FP32 (norm) bytes, rejecting nonfinite
    inputs and FP16 overflow."""
    if len(raw) % 2:
        raise ValueError('Truncated tensor during export')
    wide = (np.frombuffer(raw, dtype='<u2').astype(np.uint32) << 16).view('<f4')
    if not np.isfinite(wide).all():
        raise ValueError(f'Nonfinite checkpoint tensor: {name}')
    if not matrix:
        return wide.tobytes()
    with np.errstate(over='ignore'):
        narrow = wide.astype('<f2')
    if not np.isfinite(narrow).all():
        raise ValueError(f'FP16 overflow in tensor: {name}')
    return narrow.tobytes()


def export(checkpoint, output, shapes=None):
    """Writes OUTPUT, OUTPUT.index and OUTPUT.manifest.json; returns the
    manifest path. `shapes` replaces the Qwen3-0.6B table (tests only)."""
    shapes = pack_shapes() if shapes is None else shapes
    checkpoint, output = Path(checkpoint), Path(output)
    source = checkpoint / 'model.safetensors' if checkpoint.is_dir() else checkpoint
    targets = [output, Path(f'{output}.index'), Path(f'{output}.manifest.json')]
    output.parent.mkdir(parents=True, exist_ok=True)
    if any(t.exists() or t.is_symlink() for t in targets):
        raise FileExistsError('Weight pack outputs are immutable; choose a fresh path')
    source_hash = _sha256(source)
    header, data_start, size = read_header(source)
    regions = check_layout(header, data_start, size, shapes)
    head, embed = regions['lm_head.weight'], regions['model.embed_tokens.weight']
    if not _same_bytes(source, data_start + head[0], data_start + embed[0], head[1] - head[0]):
        raise ValueError('lm_head.weight is not bit-identical to the embedding')

    with tempfile.TemporaryDirectory(prefix='.qwen-pack-', dir=output.parent) as staging:
        staging = Path(staging)
        staged = [staging / 'weights.bin', staging / 'weights.bin.index', staging / 'weights.bin.manifest.json']
        records = []
        with source.open('rb') as src, staged[0].open('wb') as dst:
            dst.write(MAGIC + bytes(ALIGN - len(MAGIC)))
            for name, shape in shapes.items():
                matrix = len(shape) == 2
                offset = -(-dst.tell() // ALIGN) * ALIGN
                dst.write(bytes(offset - dst.tell()))
                begin, end = regions[name]
                src.seek(data_start + begin)
                seen, written = hashlib.sha256(), hashlib.sha256()
                left = end - begin
                while left:
                    raw = src.read(min(left, BLOCK))
                    if not raw:
                        raise ValueError('Truncated tensor during export')
                    seen.update(raw)
                    out = convert_block(raw, matrix, name)
                    written.update(out)
                    dst.write(out)
                    left -= len(raw)
                rows, cols = shape if matrix else (shape[0], 1)
                length = dst.tell() - offset
                if length != rows * cols * (2 if matrix else 4):
                    raise ValueError('Internal converted tensor length mismatch')
                records.append(dict(name=name, dtype='F16' if matrix else 'F32', rows=rows, columns=cols,
                                    offset_bytes=offset, length_bytes=length,
                                    checkpoint_sha256=seen.hexdigest(), sha256=written.hexdigest()))
            dst.flush()
            os.fsync(dst.fileno())
        staged[1].write_text(f'QWCPU01 {len(records)}\n' + ''.join(
            f"{r['name']} {r['dtype']} {r['rows']} {r['columns']} {r['offset_bytes']} {r['length_bytes']}\n"
            for r in records))
        if _sha256(source) != source_hash:
            raise RuntimeError('Checkpoint changed while exporting')
        manifest = dict(format='QWCPU01', completed=True, gpu=False, pytorch=False,
                        checkpoint=dict(path=str(source.resolve()), sha256=source_hash),
                        exporter_sha256=_sha256(Path(__file__)), numpy_version=np.__version__,
                        binary=dict(path=output.name, bytes=staged[0].stat().st_size, sha256=_sha256(staged[0])),
                        index=dict(path=targets[1].name, sha256=_sha256(staged[1])),
                        tensor_count=len(records), tied_lm_head_verified=True, rounding=ROUNDING,
                        tensors=records)
        staged[2].write_text(json.dumps(manifest, indent=2) + '\n')
        published = []
        try:
            for path, target in zip(staged, targets):  # manifest last: it marks completion
                with path.open('rb') as f:
                    os.fsync(f.fileno())
                path.chmod(0o444)
                os.link(path, target)
                published.append(target)
            fd = os.open(output.parent, os.O_RDONLY)
            try:
                os.fsync(fd)
            finally:
                os.close(fd)
        except BaseException:
            for target in reversed(published):
                target.unlink()
            raise
    return targets[2]


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument('--checkpoint', type=Path, required=True,
                        help='model.safetensors or the directory holding it')
    parser.add_argument('--output', type=Path, required=True, help='weights.bin to create')
    args = parser.parse_args()
    print(export(args.checkpoint, args.output.resolve()))


if __name__ == '__main__':
    main()
