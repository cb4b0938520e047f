"""ctypes binding of the oracle library (oracle/cpu_ref.h). Test-side only."""
import ctypes
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_LIB = ROOT / 'oracle' / 'build' / 'libcpuref.so'
VOCABULARY = 151936
_f = ctypes.POINTER(ctypes.c_float)
_u16 = ctypes.POINTER(ctypes.c_uint16)
_i = ctypes.POINTER(ctypes.c_int)


def fptr(a):
    return a.ctypes.data_as(_f)


def hptr(a):
    return a.view(np.uint16).ctypes.data_as(_u16)


class OracleLib:
    def __init__(self, path=ORACLE_LIB):
        if not Path(path).is_file():
            raise RuntimeError(f'oracle not built: {path} (run make -C oracle)')
        lib = self.lib = ctypes.CDLL(str(path))
        sig = {
            'cpuref_create': (ctypes.c_void_p, [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                ctypes.c_char_p, ctypes.c_size_t]),
            'cpuref_destroy': (None, [ctypes.c_void_p]),
            'cpuref_error': (ctypes.c_char_p, [ctypes.c_void_p]),
            'cpuref_reset': (ctypes.c_int, [ctypes.c_void_p]),
            'cpuref_truncate': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
            'cpuref_prefill': (ctypes.c_int, [ctypes.c_void_p, _i, ctypes.c_size_t]),
            'cpuref_step': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
            'cpuref_position': (ctypes.c_int, [ctypes.c_void_p]),
            'cpuref_logits': (_f, [ctypes.c_void_p]),
            'cpuref_hidden': (_f, [ctypes.c_void_p]),
            'cpuref_dot': (ctypes.c_float, [_f, _u16, ctypes.c_int]),
            'cpuref_gemv': (None, [_f, _u16, _f, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            'cpuref_norm': (None, [_f, _f, _f, ctypes.c_int]),
            'cpuref_rope_tables': (None, [ctypes.c_int, _f, _f]),
            'cpuref_rope': (None, [_f, _f, _f]),
            'cpuref_attention': (None, [_f, _u16, _u16, ctypes.c_int, _f]),
            'cpuref_swiglu': (None, [_f, _f, _f, ctypes.c_int]),
            'cpuref_argmax': (ctypes.c_int, [_f, ctypes.c_int]),
            'cpuref_f32_to_f16': (ctypes.c_uint16, [ctypes.c_float]),
            'cpuref_f16_to_f32': (ctypes.c_float, [ctypes.c_uint16]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args

    # ---- single operations ----
    def dot(self, x, w):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float16)
        return np.float32(self.lib.cpuref_dot(fptr(x), hptr(w), x.size))

    def gemv(self, w, x, threads=8):
        w = np.ascontiguousarray(w, np.float16)
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(w.shape[0], np.float32)
        self.lib.cpuref_gemv(fptr(x), hptr(w), fptr(y), w.shape[0], w.shape[1], threads)
        return y

    def norm(self, x, w):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        out = np.empty_like(x)
        self.lib.cpuref_norm(fptr(x), fptr(w), fptr(out), x.size)
        return out

    def rope_tables(self, context):
        c = np.empty(context * 64, np.float32)
        s = np.empty_like(c)
        self.lib.cpuref_rope_tables(context, fptr(c), fptr(s))
        return c.reshape(context, 64), s.reshape(context, 64)

    def rope(self, x, cs, sn):
        x = np.array(x, np.float32)
        cs = np.ascontiguousarray(cs, np.float32)
        sn = np.ascontiguousarray(sn, np.float32)
        self.lib.cpuref_rope(fptr(x), fptr(cs), fptr(sn))
        return x

    def attention(self, q, keys, values):
        q = np.ascontiguousarray(q, np.float32)
        keys = np.ascontiguousarray(keys, np.float16)
        values = np.ascontiguousarray(values, np.float16)
        out = np.empty(128, np.float32)
        self.lib.cpuref_attention(fptr(q), hptr(keys), hptr(values), keys.shape[0], fptr(out))
        return out

    def swiglu(self, gate, up):
        gate = np.ascontiguousarray(gate, np.float32)
        up = np.ascontiguousarray(up, np.float32)
        out = np.empty_like(gate)
        self.lib.cpuref_swiglu(fptr(gate), fptr(up), fptr(out), gate.size)
        return out

    def argmax(self, logits):
        logits = np.ascontiguousarray(logits, np.float32)
        return self.lib.cpuref_argmax(fptr(logits), logits.size)

    def model(self, pack, decode_threads=8, prefill_threads=8, context=4096):
        return OracleModel(self, pack, decode_threads, prefill_threads, context)


class OracleModel:
    """The oracle's qwen_cpu::Model restatement."""

    def __init__(self, olib, pack, decode_threads, prefill_threads, context):
        self.o = olib
        err = ctypes.create_string_buffer(512)
        self.h = olib.lib.cpuref_create(str(pack).encode(), decode_threads, prefill_threads, context, err, 512)
        if not self.h:
            raise RuntimeError(err.value.decode())

    def close(self):
        if self.h:
            self.o.lib.cpuref_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _check(self, status):
        if status:
            raise RuntimeError(self.o.lib.cpuref_error(self.h).decode())

    def reset(self):
        self._check(self.o.lib.cpuref_reset(self.h))

    def truncate(self, position):
        self._check(self.o.lib.cpuref_truncate(self.h, position))

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, np.int32)
        self._check(self.o.lib.cpuref_prefill(self.h, ids.ctypes.data_as(_i), ids.size))

    def step(self, token):
        self._check(self.o.lib.cpuref_step(self.h, int(token)))

    def position(self):
        return self.o.lib.cpuref_position(self.h)

    def logits(self):
        p = self.o.lib.cpuref_logits(self.h)
        return np.ctypeslib.as_array(p, (VOCABULARY,)).copy() if p else np.zeros(0, np.float32)

    def hidden(self):
        p = self.o.lib.cpuref_hidden(self.h)
        return np.ctypeslib.as_array(p, (1024,)).copy() if p else None


def compare_logits(actual, expected, atol=0.01, rms_atol=0.002):
    """The reference's full-vocabulary gate (tools/check_native_logits.py:124-152,
    limits from tools/check_native_saved_oracle.py:36): max-abs, RMS and greedy
    identity, with greedy taken as the lowest id among maxima."""
    actual = np.asarray(actual, np.float32)
    expected = np.asarray(expected, np.float32)
    assert actual.shape == (VOCABULARY,) and expected.shape == (VOCABULARY,)
    assert np.isfinite(actual).all() and np.isfinite(expected).all()
    delta = actual.astype(np.float64) - expected.astype(np.float64)
    order = np.argsort(-expected, kind='stable')
    return dict(max_abs=float(np.abs(delta).max()), rms=float(np.sqrt(np.mean(delta * delta))),
                actual_argmax=int(np.argmax(actual)), expected_argmax=int(np.argmax(expected)),
                expected_margin=float(expected[order[0]] - expected[order[1]]),
                passed=bool(np.abs(delta).max() <= atol and np.sqrt(np.mean(delta * delta)) <= rms_atol
                            and int(np.argmax(actual)) == int(np.argmax(expected))))
