"""QWCPU01 pack: writer output, golden digest, statistics, and the loader's
rejection of malformed packs (tools/check_native_cpu_robustness.py:108-155),
exercised through the CLI, whose validation runs before any GPU work."""
import hashlib
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

from conftest import GOLDEN



def index_rows(pack):
    lines = Path(str(pack) + '.index').read_text().splitlines()
    return lines[0], [line.split() for line in lines[1:]]


def test_layout(pack0):
    header, rows = index_rows(pack0)
    assert header == 'QWCPU01 310' and len(rows) == 310
    assert pack0.read_bytes()[:64] == b'QWCPU01' + bytes(57)
    names = [r[0] for r in rows]
    assert names[0] == 'model.embed_tokens.weight' and names[1] == 'model.norm.weight'
    assert 'lm_head.weight' not in names and len(set(names)) == 310
    end = 64
    for name, dtype, r, c, offset, length in rows:
        r, c, offset, length = int(r), int(c), int(offset), int(length)
        assert offset % 64 == 0 and offset >= end
        assert dtype == ('F32' if c == 1 else 'F16') and length == r * c * (4 if c == 1 else 2)
        end = offset + length
    assert end == pack0.stat().st_size
    manifest = json.loads(Path(str(pack0) + '.manifest.json').read_text())
    assert manifest['format'] == 'QWCPU01' and manifest['completed'] is True
    assert manifest['synthetic']['seed'] == 0


def test_golden_digest(pack0):
    """The seeded generator is deterministic (counter-based splitmix64)."""
    golden = json.loads((GOLDEN / 'pack_seed0.json').read_text())
    digest = hashlib.sha256()
    with pack0.open('rb') as f:
        for block in iter(lambda: f.read(1 << 24), b''):
            digest.update(block)
    assert pack0.stat().st_size == golden['bytes']
    assert digest.hexdigest() == golden['sha256']


def test_statistics(pack0):
    """Box-Muller output is N(0, 0.02): mean, spread and the 2-sigma mass."""
    _, rows = index_rows(pack0)
    blob = np.memmap(pack0, dtype=np.uint8, mode='r')
    name, _, r, c, offset, length = rows[0]
    w = blob[int(offset):int(offset) + int(length)].view(np.float16)[:20_000_000].astype(np.float64)
    assert abs(w.mean()) < 2e-5
    assert abs(w.std() / 0.02 - 1) < 2e-3
    assert abs(np.mean(np.abs(w) < 0.04) - 0.954499736) < 1e-3
    for name, dtype, r, c, offset, length in rows:
        if dtype == 'F32':
            assert np.all(blob[int(offset):int(offset) + int(length)].view(np.float32) == 1.0)


def test_writer_refuses_existing_outputs(qpkg, pack0):
    with pytest.raises(RuntimeError, match='immutable'):
        qpkg.write_random_pack(pack0, seed=0)


def run_cli(qpkg, *args, stdin='quit\n'):
    return subprocess.run([str(qpkg.CLI_PATH), *args], input=stdin, text=True, capture_output=True, timeout=120)


@pytest.mark.parametrize('case,expected', [
    ('bad_header', 'Invalid weight pack header'),
    ('bad_count', 'Invalid weight index header/count'),
    ('wrong_shape', 'Wrong tensor shape'),
    ('out_of_bounds', 'Invalid tensor range'),
    ('unaligned', 'Invalid tensor range'),
    ('duplicate', 'Unexpected or duplicate tensor'),
    ('overlap', 'Overlapping tensors'),
    ('nonfinite_norm', 'Nonfinite norm'),
])
def test_malformed_packs_rejected(qpkg, pack0, tmp_path, case, expected):
    original = Path(str(pack0) + '.index').read_text().splitlines()
    lines = list(original)
    binary = tmp_path / 'weights.bin'
    if case == 'bad_header':
        binary.write_bytes(b'BADCPU1' + bytes(57))
    elif case == 'nonfinite_norm':
        # Rows are validated in index order, so a first row holding a NaN
        # norm is rejected before any later row is looked at.
        binary.write_bytes(b'QWCPU01' + bytes(57) + np.full(1024, np.nan, np.float32).tobytes())
        row = next(i for i, l in enumerate(lines) if l.startswith('model.norm.weight '))
        f = lines[row].split(); f[4] = '64'; lines[row] = ' '.join(f)
        lines.insert(1, lines.pop(row))
    else:
        binary.symlink_to(pack0)
        if case == 'bad_count':
            lines[0] = 'QWCPU01 309'
        elif case == 'wrong_shape':
            f = lines[1].split(); f[2] = '1'; lines[1] = ' '.join(f)
        elif case == 'out_of_bounds':
            f = lines[1].split(); f[4] = str((pack0.stat().st_size + 63) // 64 * 64); lines[1] = ' '.join(f)
        elif case == 'unaligned':
            f = lines[1].split(); f[4] = '65'; lines[1] = ' '.join(f)
        elif case == 'duplicate':
            lines[2] = lines[1]
        elif case == 'overlap':
            src = next(l.split() for l in original[1:] if l.split()[0] == 'model.layers.0.input_layernorm.weight')
            row = next(i for i, l in enumerate(lines) if l.split()[0] == 'model.norm.weight')
            f = lines[row].split(); f[4] = src[4]; lines[row] = ' '.join(f)
    Path(str(binary) + '.index').write_text('\n'.join(lines) + '\n')
    result = run_cli(qpkg, '--weights', str(binary), '--threads', '1', '--prefill-threads', '1', '--context', '8')
    assert result.returncode != 0 and result.stdout.strip() == ''
    assert expected in result.stderr, result.stderr


@pytest.mark.parametrize('args,expected', [
    (['--weights'], 'Missing option value'),
    (['--bogus', '1'], 'Unknown option: --bogus'),
    (['--threads', '2'], '--weights is required'),
    (['--weights', '/nonexistent/weights.bin'], 'Cannot open weights'),
    (['--threads', 'x'], 'Invalid integer: x'),
])
def test_cli_argument_errors(qpkg, args, expected):
    result = run_cli(qpkg, *args)
    assert result.returncode == 1 and expected in result.stderr and result.stdout == ''


@pytest.mark.parametrize('args,expected', [
    (['--threads', '0'], 'Threads must be in 1..64'),
    (['--prefill-threads', '65'], 'Threads must be in 1..64'),
    (['--context', '4097'], 'Context must be in 1..4096'),
    (['--context', '0'], 'Context must be in 1..4096'),
])
def test_cli_option_ranges(qpkg, pack0, args, expected):
    result = run_cli(qpkg, '--weights', str(pack0), *args)
    assert result.returncode == 1 and expected in result.stderr and result.stdout == ''
