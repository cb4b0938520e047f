"""ORACLE (test infrastructure only): NumPy restatement of the reference's
independent per-token oracle, ``NumpyQwen.token`` (tests/test_full_model.py:40-80),
with FP16 matrix weights and FP16 K/V rounding (test_full_model.py:32-33, 59-63).

It reads a QWCPU01 pack (engine/INTERFACE.md:8-21) instead of a BF16
safetensors checkpoint. Its arithmetic is NumPy/BLAS FP32, deliberately
different from the C++ restatement's lane order, so agreement between the two
within the reference's gate (atol 1e-2, RMS 2e-3, greedy identity;
tools/check_native_saved_oracle.py:36) pins the C++ oracle end to end.
Only tests/ use this module.
"""
from pathlib import Path

import numpy as np

H, D, Q, K, F, L, V = 1024, 128, 16, 8, 3072, 28, 151936


def read_pack(path):
    """Map a QWCPU01 pack: name -> float32 array (matrices widened from FP16)."""
    path = Path(path)
    blob = np.memmap(path, dtype=np.uint8, mode='r')
    if bytes(blob[:7]) != b'QWCPU01':
        raise ValueError('Invalid weight pack header')
    lines = Path(str(path) + '.index').read_text().split('\n')
    signature, count = lines[0].split()
    if signature != 'QWCPU01' or int(count) != 310:
        raise ValueError('Invalid weight index header/count')
    weights = {}
    for line in lines[1:1 + int(count)]:
        name, dtype, rows, cols, offset, length = line.split()
        rows, cols, offset, length = int(rows), int(cols), int(offset), int(length)
        raw = blob[offset:offset + length]
        if dtype == 'F16':
            weights[name] = raw.view('<f2').reshape(rows, cols)
        else:
            weights[name] = raw.view('<f4').reshape(rows).astype(np.float32)
    return weights


class NumpyQwen:
    """Per-token FP32 forward pass with FP16-rounded K/V (test_full_model.py:40-80)."""

    def __init__(self, pack_path):
        raw = read_pack(pack_path)
        self.w = {}
        for name, value in raw.items():
            self.w[name] = value.astype(np.float32) if value.dtype == np.float16 else value
        self.cache = []

    def reset(self):
        self.cache = []

    def truncate(self, position):
        self.cache = self.cache[:position]

    def token(self, token, logits=True):
        w = self.w
        position = len(self.cache)
        payload = []

        def norm(x, weight):
            return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + np.float32(1e-6)) * weight

        angle = position / (1000000.0 ** (np.arange(64, dtype=np.float64) * 2 / 128))
        cos, sin = np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)

        def rope(x):
            left, right = np.split(x, 2, axis=-1)
            return np.concatenate((left * cos - right * sin, right * cos + left * sin), axis=-1)

        x = w['model.embed_tokens.weight'][token].copy()
        for layer in range(L):
            def weight(suffix):
                return w[f'model.layers.{layer}.{suffix}.weight']
            h = norm(x, weight('input_layernorm'))
            q = rope(norm((weight('self_attn.q_proj') @ h).reshape(Q, D), weight('self_attn.q_norm')))
            k = rope(norm((weight('self_attn.k_proj') @ h).reshape(K, D), weight('self_attn.k_norm')))
            v = (weight('self_attn.v_proj') @ h).reshape(K, D)
            k = k.astype(np.float16).astype(np.float32)
            v = v.astype(np.float16).astype(np.float32)
            payload.append((k, v))
            keys = np.stack([entry[layer][0] for entry in self.cache] + [k])
            vals = np.stack([entry[layer][1] for entry in self.cache] + [v])
            keys, vals = np.repeat(keys, 2, axis=1), np.repeat(vals, 2, axis=1)
            scores = np.einsum('hd,thd->ht', q, keys) / np.float32(np.sqrt(128))
            probs = np.exp(scores - scores.max(axis=-1, keepdims=True))
            probs /= probs.sum(axis=-1, keepdims=True)
            attended = np.einsum('ht,thd->hd', probs, vals).reshape(-1)
            x += weight('self_attn.o_proj') @ attended
            h = norm(x, weight('post_attention_layernorm'))
            gate, up = weight('mlp.gate_proj') @ h, weight('mlp.up_proj') @ h
            activated = gate * (.5 + .5 * np.tanh(gate * .5)) * up
            x += weight('mlp.down_proj') @ activated
        self.cache.append(payload)
        if logits:
            return w['model.embed_tokens.weight'] @ norm(x, w['model.norm.weight'])
        return None
