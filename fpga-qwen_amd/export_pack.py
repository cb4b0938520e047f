#!/usr/bin/env python3
"""Writes the engine's weight pack from a Qwen3-0.6B BF16 checkpoint.

Input: ``model.safetensors`` (or the directory holding it). Output: the
QWCPU01 pack of engine/INTERFACE.md:6-21, three files ``weights.bin``,
``weights.bin.index`` and ``weights.bin.manifest.json``; the binary is the
same bytes the reference's exporter writes for the same checkpoint.

How it works:

1. The checkpoint is memory-mapped. Its JSON header (keys must be unique) is
   checked against the tensor table below: exactly those 310 tensors plus
   ``lm_head.weight``, all BF16 with the expected shapes, byte ranges that
   lie inside the file and together cover its data area exactly once.
2. ``lm_head.weight`` must equal the embedding byte for byte; the engine ties
   its output head to the embedding, so the pack stores the embedding once.
3. The pack layout is computed up front: a 64-byte ``QWCPU01`` header, then
   the tensors in table order at 64-byte aligned offsets. The binary is
   allocated at its final size and filled through a memory map, one block of
   rows at a time: BF16 widened exactly to FP32, 2-D matrices rounded to FP16
   (round to nearest even), 1-D norms kept FP32. A non-finite input value or
   a matrix value beyond FP16's range stops the export.
4. Packs are immutable. Each file is written under a temporary name in the
   output directory, synced, made read-only and then hard-linked to its final
   name, which fails rather than replace an existing file; the manifest goes
   last and marks the pack complete. On any failure the files already linked
   are removed again.

Needs NumPy only (no GPU, no Torch).

Usage: python export_pack.py --checkpoint DIR_OR_FILE --output weights.bin
"""
import argparse
import hashlib
import json
import mmap
import os
import struct
import tempfile
from dataclasses import dataclass
from pathlib import Path

import numpy as np

FORMAT = 'QWCPU01'
HEADER_BYTES = 64
ALIGN = 64
ROWS_PER_BLOCK = 2048
ROUNDING = ('BF16 widened exactly to FP32; 2-D matrices rounded to FP16 (round to nearest even); '
            '1-D norm weights kept FP32; little endian')


class PackError(ValueError):
    """The checkpoint cannot become a pack (the message says why)."""


def qwen3_tensor_table():
    """The pack's tensors in file order, name -> shape (fpga-qwen_amd/csrc/pack.cpp
    validates the same table; engine/core.cpp:235-276)."""
    table = {'model.embed_tokens.weight': (151936, 1024), 'model.norm.weight': (1024,)}
    layer = (('input_layernorm', (1024,)), ('post_attention_layernorm', (1024,)),
             ('self_attn.q_norm', (128,)), ('self_attn.k_norm', (128,)),
             ('self_attn.q_proj', (2048, 1024)), ('self_attn.k_proj', (1024, 1024)),
             ('self_attn.v_proj', (1024, 1024)), ('self_attn.o_proj', (1024, 2048)),
             ('mlp.gate_proj', (3072, 1024)), ('mlp.up_proj', (3072, 1024)), ('mlp.down_proj', (1024, 3072)))
    for index in range(28):
        table.update((f'model.layers.{index}.{part}.weight', shape) for part, shape in layer)
    return table


@dataclass(frozen=True)
class Slot:
    """Where one tensor goes in the pack."""
    name: str
    shape: tuple
    offset: int

    @property
    def matrix(self):
        return len(self.shape) == 2

    @property
    def rows(self):
        return self.shape[0]

    @property
    def columns(self):
        return self.shape[1] if self.matrix else 1

    @property
    def dtype(self):
        return 'F16' if self.matrix else 'F32'

    @property
    def length(self):
        return self.rows * self.columns * (2 if self.matrix else 4)


def plan(table):
    """Pack slots in table order and the binary's total size."""
    slots, cursor = [], HEADER_BYTES
    for name, shape in table.items():
        cursor = -(-cursor // ALIGN) * ALIGN
        slots.append(Slot(name, tuple(shape), cursor))
        cursor += slots[-1].length
    return slots, cursor


def _unique_keys(pairs):
    seen = {}
    for key, value in pairs:
        if key in seen:
            raise PackError(f'safetensors header repeats the key {key!r}')
        seen[key] = value
    return seen


class Checkpoint:
    """A memory-mapped safetensors file and its parsed header."""

    def __init__(self, path):
        self.path = Path(path)
        self._file = self.path.open('rb')
        self.size = os.fstat(self._file.fileno()).st_size
        if self.size < 8:
            raise PackError('safetensors file is shorter than its 8-byte header length')
        self.map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
        (header_bytes,) = struct.unpack_from('<Q', self.map, 0)
        if not 2 <= header_bytes <= min(self.size - 8, 64 << 20):
            raise PackError(f'safetensors header length {header_bytes} does not fit the file')
        try:
            header = json.loads(self.map[8:8 + header_bytes], object_pairs_hook=_unique_keys)
        except PackError:
            raise
        except ValueError as error:
            raise PackError(f'safetensors header is not JSON: {error}') from None
        if not isinstance(header, dict):
            raise PackError('safetensors header is not a JSON object')
        header.pop('__metadata__', None)
        self.header, self.data = header, 8 + header_bytes

    def bf16(self, name):
        """The tensor's BF16 bit patterns as a read-only uint16 array view."""
        begin, end = self.header[name]['data_offsets']
        shape = self.header[name]['shape']
        return np.frombuffer(self.map, dtype='<u2', count=(end - begin) // 2, offset=self.data + begin).reshape(shape)

    def sha256(self):
        digest = hashlib.sha256()
        view = memoryview(self.map)
        for start in range(0, self.size, 64 << 20):
            digest.update(view[start:start + (64 << 20)])
        view.release()
        return digest.hexdigest()

    def close(self):
        try:
            self.map.close()
        except BufferError:  # an array view is still alive; the map closes when it goes
            pass
        self._file.close()


def audit(checkpoint, table):
    """Checks the checkpoint against the table (step 1 and 2 of the module
    docstring); raises PackError with the first problem found."""
    expected = dict(table, **{'lm_head.weight': table['model.embed_tokens.weight']})
    missing = sorted(set(expected) - set(checkpoint.header))
    unexpected = sorted(set(checkpoint.header) - set(expected))
    if missing or unexpected:
        raise PackError(f'checkpoint tensors are not the {len(expected)} of Qwen3-0.6B: '
                        f'missing {missing[:4]}, unexpected {unexpected[:4]}')
    spans = []
    for name, shape in expected.items():
        entry = checkpoint.header[name]
        found = (entry.get('dtype'), entry.get('shape')) if isinstance(entry, dict) else (None, None)
        if found != ('BF16', list(shape)):
            raise PackError(f'{name}: expected BF16 {list(shape)}, found {found[0]} {found[1]}')
        offsets = entry.get('data_offsets')
        if not (isinstance(offsets, list) and len(offsets) == 2 and all(type(v) is int for v in offsets)):
            raise PackError(f'{name}: data_offsets must be two integers')
        begin, end = offsets
        if not (0 <= begin and end - begin == 2 * int(np.prod(shape)) and checkpoint.data + end <= checkpoint.size):
            raise PackError(f'{name}: byte range [{begin}, {end}) does not hold its {int(np.prod(shape))} '
                            'BF16 values inside the file')
        spans.append((begin, end))
    spans.sort()
    covered = 0
    for begin, end in spans:
        if begin != covered:
            raise PackError('the tensors do not cover the data area exactly once (a gap or an overlap)')
        covered = end
    if checkpoint.data + covered != checkpoint.size:
        raise PackError('the tensors do not cover the data area exactly once (trailing bytes)')
    head, embedding = checkpoint.bf16('lm_head.weight'), checkpoint.bf16('model.embed_tokens.weight')
    for start in range(0, head.shape[0], 8 * ROWS_PER_BLOCK):
        if not np.array_equal(head[start:start + 8 * ROWS_PER_BLOCK], embedding[start:start + 8 * ROWS_PER_BLOCK]):
            raise PackError('lm_head.weight differs from model.embed_tokens.weight; the engine needs a tied head')


def convert(block, matrix, name):
    """BF16 bits -> FP16 values (matrix) or FP32 values (norm), checked."""
    wide = (block.astype(np.uint32) << 16).view(np.float32)
    if not np.isfinite(wide).all():
        raise PackError(f'{name}: the checkpoint holds a non-finite value')
    if not matrix:
        return wide
    with np.errstate(over='ignore'):
        narrow = wide.astype(np.float16)
    if not np.isfinite(narrow).all():
        raise PackError(f'{name}: a value lies beyond the FP16 range')
    return narrow


def _file_sha256(path):
    digest = hashlib.sha256()
    with open(path, 'rb') as f:
        for block in iter(lambda: f.read(16 << 20), b''):
            digest.update(block)
    return digest.hexdigest()


def write_pack(checkpoint_path, output, table=None):
    """Writes OUTPUT, OUTPUT.index and OUTPUT.manifest.json and returns the
    manifest's path. `table` replaces the Qwen3-0.6B tensor table (tests)."""
    table = qwen3_tensor_table() if table is None else table
    checkpoint_path, output = Path(checkpoint_path), Path(output)
    source = checkpoint_path / 'model.safetensors' if checkpoint_path.is_dir() else checkpoint_path
    finals = [output, Path(f'{output}.index'), Path(f'{output}.manifest.json')]
    output.parent.mkdir(parents=True, exist_ok=True)
    taken = [p for p in finals if p.exists() or p.is_symlink()]
    if taken:
        raise FileExistsError(f'{taken[0]} already exists; packs are never overwritten, choose a new path')
    before = os.stat(source)
    checkpoint = Checkpoint(source)
    temporaries, descriptors = [], []
    try:
        audit(checkpoint, table)
        source_sha = checkpoint.sha256()
        slots, total = plan(table)

        def close(fd):
            descriptors.remove(fd)
            os.close(fd)

        def temporary(suffix):
            fd, name = tempfile.mkstemp(prefix=f'.{output.name}.', suffix=suffix, dir=output.parent)
            temporaries.append(Path(name))
            descriptors.append(fd)
            return fd, Path(name)

        fd, binary = temporary('.bin')
        os.ftruncate(fd, total)
        out = np.memmap(binary, dtype=np.uint8, mode='r+', shape=(total,))
        out[:len(FORMAT)] = np.frombuffer(FORMAT.encode(), np.uint8)
        records = []
        for slot in slots:
            bits = checkpoint.bf16(slot.name).reshape(slot.rows, -1)
            target = out[slot.offset:slot.offset + slot.length].view(np.float16 if slot.matrix else np.float32)
            target = target.reshape(slot.rows, slot.columns)
            source_digest, pack_digest = hashlib.sha256(), hashlib.sha256()
            for start in range(0, slot.rows, ROWS_PER_BLOCK):
                block = bits[start:start + ROWS_PER_BLOCK]
                values = convert(block, slot.matrix, slot.name).reshape(block.shape[0], slot.columns)
                target[start:start + block.shape[0]] = values
                source_digest.update(block.tobytes())
                pack_digest.update(values.tobytes())
            records.append(dict(name=slot.name, dtype=slot.dtype, rows=slot.rows, columns=slot.columns,
                                offset_bytes=slot.offset, length_bytes=slot.length,
                                source_sha256=source_digest.hexdigest(), sha256=pack_digest.hexdigest()))
        out.flush()
        del out, target, bits
        os.fsync(fd)
        close(fd)

        fd, index = temporary('.index')
        lines = [f'{FORMAT} {len(records)}'] + [
            f"{r['name']} {r['dtype']} {r['rows']} {r['columns']} {r['offset_bytes']} {r['length_bytes']}"
            for r in records]
        os.write(fd, ('\n'.join(lines) + '\n').encode())
        os.fsync(fd)
        close(fd)

        after = os.stat(source)
        if (after.st_size, after.st_mtime_ns, after.st_ino) != (before.st_size, before.st_mtime_ns, before.st_ino):
            raise PackError('the checkpoint changed while the pack was being written')
        manifest = dict(
            format=FORMAT, completed=True,
            producer=dict(tool='fpga-qwen_amd/export_pack.py', sha256=_file_sha256(Path(__file__)),
                          numpy=np.__version__),
            source=dict(path=str(source.resolve()), bytes=checkpoint.size, sha256=source_sha),
            binary=dict(path=output.name, bytes=total, sha256=_file_sha256(binary)),
            index=dict(path=finals[1].name, sha256=_file_sha256(index)),
            tensor_count=len(records), tied_lm_head_verified=True, rounding=ROUNDING, tensors=records)
        fd, manifest_path = temporary('.json')
        os.write(fd, (json.dumps(manifest, indent=2) + '\n').encode())
        os.fsync(fd)
        close(fd)

        linked = []
        try:
            for staged, final in zip((binary, index, manifest_path), finals):  # the manifest last
                staged.chmod(0o444)
                os.link(staged, final)
                linked.append(final)
            directory = os.open(output.parent, os.O_RDONLY)
            try:
                os.fsync(directory)
            finally:
                os.close(directory)
        except BaseException:
            for final in reversed(linked):
                final.unlink()
            raise
    finally:
        for fd in descriptors:
            os.close(fd)
        checkpoint.close()
        for path in temporaries:
            path.unlink(missing_ok=True)
    return finals[2]


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument('--checkpoint', type=Path, required=True,
                        help='model.safetensors or the directory that holds it')
    parser.add_argument('--output', type=Path, required=True, help='the weights.bin to create')
    args = parser.parse_args()
    print(write_pack(args.checkpoint, args.output.resolve()))


if __name__ == '__main__':
    main()
