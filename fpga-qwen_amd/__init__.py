"""Python host side of the MI355X Qwen3-0.6B engine (ctypes over the C ABI).

``Model`` mirrors the reference engine API ``qwen_cpu::Model``
(engine/core.hpp:25-56): reset, truncate, prefill, step, verify_two,
commit_verified, logits, hidden, position. Errors raise ``RuntimeError`` with
the engine's message, as the C++ API throws ``std::runtime_error``.
All inference runs in ``build/libqwen_gpu.so``; there is no CPU fallback:
importing this module without the built library raises.
"""
import ctypes
import json
import os
from pathlib import Path

import numpy as np

PACKAGE_DIR = Path(__file__).resolve().parent
BUILD_DIR = PACKAGE_DIR / 'build'
LIBRARY_PATH = BUILD_DIR / 'libqwen_gpu.so'
CLI_PATH = BUILD_DIR / 'qwen_gpu'
VOCABULARY = 151936
HIDDEN = 1024
PREFIX_REUSE_CHUNK = 512
EOS = (151643, 151645)

# Every exported symbol of include/qwen_gpu.h with its ctypes signature.
_c_float_p = ctypes.POINTER(ctypes.c_float)
_c_int_p = ctypes.POINTER(ctypes.c_int)
_c_size_p = ctypes.POINTER(ctypes.c_size_t)


class Options(ctypes.Structure):
    """qwen_cpu::Options (engine/core.hpp:11-15)."""
    _fields_ = [('decode_threads', ctypes.c_int), ('prefill_threads', ctypes.c_int), ('context', ctypes.c_int)]


SIGNATURES = {
    'qwen_gpu_last_error': (ctypes.c_char_p, []),
    'qwen_gpu_create': (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(Options), ctypes.POINTER(ctypes.c_void_p)]),
    'qwen_gpu_destroy': (None, [ctypes.c_void_p]),
    'qwen_gpu_reset': (ctypes.c_int, [ctypes.c_void_p]),
    'qwen_gpu_truncate': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    'qwen_gpu_prefill': (ctypes.c_int, [ctypes.c_void_p, _c_int_p, ctypes.c_size_t]),
    'qwen_gpu_step': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    'qwen_gpu_verify_two': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                           ctypes.POINTER(_c_float_p), ctypes.POINTER(_c_float_p), _c_int_p]),
    'qwen_gpu_commit_verified': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    'qwen_gpu_logits': (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(_c_float_p), _c_size_p]),
    'qwen_gpu_hidden': (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(_c_float_p), _c_size_p]),
    'qwen_gpu_position': (ctypes.c_int, [ctypes.c_void_p]),
    'qwen_gpu_decode_kernels': (ctypes.c_int, [ctypes.c_void_p]),
    'qwen_gpu_lossless_bf16_cache_bytes': (ctypes.c_size_t, [ctypes.c_void_p]),
    'qwen_gpu_get_options': (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Options)]),
    'qwen_gpu_greedy': (ctypes.c_int, [ctypes.c_void_p, _c_int_p]),
    'qwen_gpu_verify_greedy': (ctypes.c_int, [ctypes.c_void_p, _c_int_p, _c_int_p]),
    'qwen_gpu_top_scores': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_float, ctypes.c_float, ctypes.c_int,
                                           _c_float_p, _c_int_p]),
    'qwen_gpu_update_penalized': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _c_int_p, ctypes.c_size_t]),
    'qwen_gpu_verify_two_greedy': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _c_int_p, _c_int_p]),
    'qwen_gpu_write_random_pack': (ctypes.c_int, [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_double, ctypes.c_int]),
    'qwen_gpu_validate_pack': (ctypes.c_int, [ctypes.c_char_p]),
    'qwen_gpu_device_malloc': (ctypes.c_int, [ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)]),
    'qwen_gpu_device_free': (ctypes.c_int, [ctypes.c_void_p]),
    'qwen_gpu_memcpy_to_device': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    'qwen_gpu_memcpy_to_host': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    'qwen_gpu_device_synchronize': (ctypes.c_int, []),
    'qwen_gpu_op_tile_matrix': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    'qwen_gpu_op_gemv': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    'qwen_gpu_op_gemm': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    'qwen_gpu_create_sharing': (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(Options),
                                               ctypes.POINTER(ctypes.c_void_p)]),
    'qwen_gpu_copy_prefix': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]),
    'qwen_gpu_step_batch': (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), _c_int_p, ctypes.c_int]),
    'qwen_gpu_step_batch_greedy': (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), _c_int_p, ctypes.c_int, _c_int_p]),
    'qwen_gpu_op_attention_prefill': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                                     ctypes.c_int, ctypes.c_void_p]),
    'qwen_gpu_op_gemm_static': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    'qwen_gpu_op_gemm_swiglu': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_void_p]),
    'qwen_gpu_op_norm_qkv': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_void_p]),
    'qwen_gpu_op_norm_gate_up': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    'qwen_gpu_op_down_residual': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                 ctypes.c_void_p]),
    'qwen_gpu_op_fused_ffn': (ctypes.c_int, [ctypes.c_void_p] * 9 + [ctypes.c_uint32, ctypes.c_void_p]),
    'qwen_gpu_op_norm_qkv_folded': (ctypes.c_int, [ctypes.c_void_p] * 7),
    'qwen_gpu_op_bgemv': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    'qwen_gpu_op_gemv_time': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p,
                                             ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _c_float_p]),
    'qwen_gpu_op_copy': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    'qwen_gpu_time_kernel': (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _c_float_p]),
}


def load_library(path=LIBRARY_PATH):
    """Load the engine library; raises if it has not been built."""
    path = Path(path)
    if not path.is_file():
        raise RuntimeError(f'qwen_gpu library not built: {path} (run __graft_entry__.build())')
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


_LIB = load_library()


def _check(status):
    if status != 0:
        raise RuntimeError(_LIB.qwen_gpu_last_error().decode())


class VerificationRows:
    """qwen_cpu::VerificationRows (engine/core.hpp:16-22), copied to NumPy."""

    def __init__(self, logits, hidden, base_position):
        self.logits, self.hidden, self.base_position = logits, hidden, base_position


class Model:
    """qwen_cpu::Model on the GPU (engine/core.hpp:25-56)."""

    def __init__(self, weights_file, decode_threads=12, prefill_threads=6, context=4096):
        handle = ctypes.c_void_p()
        options = Options(decode_threads, prefill_threads, context)
        _check(_LIB.qwen_gpu_create(str(weights_file).encode(), ctypes.byref(options), ctypes.byref(handle)))
        self._handle = handle

    @classmethod
    def _from_handle(cls, handle):
        model = cls.__new__(cls)
        model._handle = handle
        return model

    def share(self, decode_threads=None, prefill_threads=None, context=None):
        """A further model on this model's uploaded weights, with its own K/V
        cache and state (options default to this model's)."""
        own = self.options()
        options = Options(decode_threads or own['decode_threads'], prefill_threads or own['prefill_threads'],
                          context or own['context'])
        handle = ctypes.c_void_p()
        _check(_LIB.qwen_gpu_create_sharing(self._handle, ctypes.byref(options), ctypes.byref(handle)))
        return Model._from_handle(handle)

    def copy_prefix(self, src, positions):
        """Become `src` truncated to `positions` (K/V rows copied on the device)."""
        _check(_LIB.qwen_gpu_copy_prefix(self._handle, src._handle, int(positions)))

    def close(self):
        if self._handle:
            _LIB.qwen_gpu_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def reset(self):
        _check(_LIB.qwen_gpu_reset(self._handle))

    def truncate(self, position):
        _check(_LIB.qwen_gpu_truncate(self._handle, int(position)))

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        _check(_LIB.qwen_gpu_prefill(self._handle, ids.ctypes.data_as(_c_int_p), ids.size))

    def step(self, token):
        _check(_LIB.qwen_gpu_step(self._handle, int(token)))

    def verify_two(self, first, second):
        logits, hidden, base = _c_float_p(), _c_float_p(), ctypes.c_int()
        _check(_LIB.qwen_gpu_verify_two(self._handle, int(first), int(second), ctypes.byref(logits),
                                        ctypes.byref(hidden), ctypes.byref(base)))
        return VerificationRows(np.ctypeslib.as_array(logits, (2, VOCABULARY)).copy(),
                                np.ctypeslib.as_array(hidden, (2, HIDDEN)).copy(), base.value)

    def commit_verified(self, count):
        _check(_LIB.qwen_gpu_commit_verified(self._handle, int(count)))

    def logits(self):
        """Copy of the current FP32 logits; an empty array when there are none."""
        data, count = _c_float_p(), ctypes.c_size_t()
        _check(_LIB.qwen_gpu_logits(self._handle, ctypes.byref(data), ctypes.byref(count)))
        if not count.value:
            return np.zeros(0, dtype=np.float32)
        return np.ctypeslib.as_array(data, (count.value,)).copy()

    def hidden(self):
        data, count = _c_float_p(), ctypes.c_size_t()
        _check(_LIB.qwen_gpu_hidden(self._handle, ctypes.byref(data), ctypes.byref(count)))
        return np.ctypeslib.as_array(data, (count.value,)).copy()

    def decode_kernels(self):
        """2: one launch per token, 1: two fused launches per layer, 0: separate kernels."""
        return _LIB.qwen_gpu_decode_kernels(self._handle)

    def position(self):
        return _LIB.qwen_gpu_position(self._handle)

    def lossless_bf16_cache_bytes(self):
        return _LIB.qwen_gpu_lossless_bf16_cache_bytes(self._handle)

    def options(self):
        o = Options()
        _check(_LIB.qwen_gpu_get_options(self._handle, ctypes.byref(o)))
        return dict(decode_threads=o.decode_threads, prefill_threads=o.prefill_threads, context=o.context)

    def greedy(self):
        token = ctypes.c_int()
        _check(_LIB.qwen_gpu_greedy(self._handle, ctypes.byref(token)))
        return token.value

    def verify_greedy(self):
        a, b = ctypes.c_int(), ctypes.c_int()
        _check(_LIB.qwen_gpu_verify_greedy(self._handle, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def verify_two_greedy(self, first, second):
        """verify_two + verify_greedy without copying the rows to the host."""
        a, b = ctypes.c_int(), ctypes.c_int()
        _check(_LIB.qwen_gpu_verify_two_greedy(self._handle, int(first), int(second), ctypes.byref(a),
                                               ctypes.byref(b)))
        return a.value, b.value

    def top_scores(self, penalty=1.5, temperature=0.7, k=20):
        """Chat-mode candidates of the current logits: (values, ids) of the k
        best (logit - (penalized ? penalty : 0)) / temperature, value
        descending then id ascending."""
        values = np.zeros(k, dtype=np.float32)
        ids = np.zeros(k, dtype=np.int32)
        _check(_LIB.qwen_gpu_top_scores(self._handle, float(penalty), float(temperature), int(k),
                                        values.ctypes.data_as(_c_float_p), ids.ctypes.data_as(_c_int_p)))
        return values, ids

    def update_penalized(self, ids=(), clear=False):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        _check(_LIB.qwen_gpu_update_penalized(self._handle, 1 if clear else 0, ids.ctypes.data_as(_c_int_p),
                                              ids.size))

    def time_kernel(self, which, iterations):
        ms = ctypes.c_float()
        _check(_LIB.qwen_gpu_time_kernel(self._handle, int(which), int(iterations), ctypes.byref(ms)))
        return ms.value


def step_batch(models, tokens):
    """One decode step for each model (1..8, sharing weights): models[i]
    consumes tokens[i], all projections batched on the matrix cores."""
    handles = (ctypes.c_void_p * len(models))(*[m._handle for m in models])
    toks = np.ascontiguousarray(tokens, dtype=np.int32)
    if toks.size != len(models):
        raise ValueError('one token per model')
    _check(_LIB.qwen_gpu_step_batch(handles, toks.ctypes.data_as(_c_int_p), len(models)))


_BATCH_ARRAYS = {}  # handles of a model list -> its ctypes argument arrays, reused across steps


def step_batch_greedy(models, tokens):
    """step_batch, then each model's greedy selection, in one call; returns
    the selections (the next tokens of a greedy decode loop)."""
    n = len(models)
    if len(tokens) != n:
        raise ValueError('one token per model')
    key = tuple(m._handle.value if m._handle else 0 for m in models)  # a closed model passes null
    arrays = _BATCH_ARRAYS.get(key)
    if arrays is None:
        if len(_BATCH_ARRAYS) > 64:
            _BATCH_ARRAYS.clear()
        arrays = _BATCH_ARRAYS[key] = ((ctypes.c_void_p * n)(*key), ctypes.c_int * n, (ctypes.c_int * n)())
    handles, token_type, out = arrays
    _check(_LIB.qwen_gpu_step_batch_greedy(handles, token_type(*tokens), n, out))
    return out[:]


def validate_pack(path):
    """The engine's pack checks (no device needed); raises RuntimeError with
    the reference's message on a malformed pack."""
    _check(_LIB.qwen_gpu_validate_pack(str(path).encode()))


def write_random_pack(path, seed=0, stddev=0.02, threads=None):
    """Seeded QWCPU01 pack: matrices N(0, stddev) in FP16, norm gains 1.0."""
    threads = threads or min(16, os.cpu_count() or 1)
    _check(_LIB.qwen_gpu_write_random_pack(str(path).encode(), int(seed), float(stddev), int(threads)))
    return Path(path)


def ensure_random_pack(directory, seed=0, stddev=0.02):
    """Reuse ``directory/weights.bin`` when its manifest records the same seed."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    path = directory / 'weights.bin'
    manifest = Path(str(path) + '.manifest.json')
    if manifest.is_file():
        info = json.loads(manifest.read_text())
        synthetic = info.get('synthetic', {})
        if info.get('completed') and synthetic.get('seed') == seed and synthetic.get('stddev') == stddev:
            return path
        raise RuntimeError(f'{manifest} holds a different pack; choose another directory')
    return write_random_pack(path, seed, stddev)


# ---- kernel-level entry points on device memory of this library's runtime ----

class DeviceBuffer:
    """Device allocation made through the engine's own HIP runtime."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        ptr = ctypes.c_void_p()
        _check(_LIB.qwen_gpu_device_malloc(self.nbytes, ctypes.byref(ptr)))
        self.ptr = ptr

    @classmethod
    def from_array(cls, array):
        array = np.ascontiguousarray(array)
        buf = cls(array.nbytes)
        _check(_LIB.qwen_gpu_memcpy_to_device(buf.ptr, array.ctypes.data_as(ctypes.c_void_p), array.nbytes))
        return buf

    def to_array(self, dtype, count):
        out = np.empty(count, dtype=dtype)
        _check(_LIB.qwen_gpu_memcpy_to_host(out.ctypes.data_as(ctypes.c_void_p), self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            _check(_LIB.qwen_gpu_device_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceView:
    """A byte range inside a DeviceBuffer (keeps the buffer alive; never frees)."""

    def __init__(self, base, offset, nbytes=None):
        offset = int(offset)
        nbytes = base.nbytes - offset if nbytes is None else int(nbytes)
        if offset < 0 or nbytes < 0 or offset + nbytes > base.nbytes:
            raise ValueError('DeviceView outside its buffer')
        self.base, self.nbytes = base, nbytes
        self.ptr = ctypes.c_void_p(base.ptr.value + offset)


def synchronize():
    _check(_LIB.qwen_gpu_device_synchronize())


def tile_matrix(first, second=None):
    """Natural FP16 [rows, cols] array(s) -> chain-tiled GEMV layout on the device."""
    first = np.ascontiguousarray(first, np.float16)
    rows, cols = first.shape
    a = DeviceBuffer.from_array(first)
    b = DeviceBuffer.from_array(np.ascontiguousarray(second, np.float16)) if second is not None else None
    out = DeviceBuffer(first.nbytes * (2 if second is not None else 1))
    _check(_LIB.qwen_gpu_op_tile_matrix(a.ptr, b.ptr if b else None, out.ptr, rows, cols, None))
    synchronize()
    return out


def gemv(tiled, x, rows):
    """y = W x with the reference dot's chain order (W chain-tiled DeviceBuffer)."""
    x = np.ascontiguousarray(x, np.float32)
    xd = DeviceBuffer.from_array(x)
    yd = DeviceBuffer(rows * 4)
    _check(_LIB.qwen_gpu_op_gemv(tiled.ptr, xd.ptr, yd.ptr, rows, x.size, None))
    synchronize()
    return yd.to_array(np.float32, rows)


def gemv_time(tiled, copy_stride, copies, x, y, rows, cols, iterations):
    """Average ms of one GEMV launch cycling through `copies` tiled weight
    copies `copy_stride` bytes apart in DeviceBuffer `tiled` (x, y DeviceBuffers)."""
    ms = ctypes.c_float()
    _check(_LIB.qwen_gpu_op_gemv_time(tiled.ptr, int(copy_stride), int(copies), x.ptr, y.ptr, int(rows), int(cols),
                                      int(iterations), ctypes.byref(ms)))
    return ms.value


def copy_device(src, dst, nbytes):
    """Plain device copy between DeviceBuffers (counter calibration)."""
    _check(_LIB.qwen_gpu_op_copy(src.ptr, dst.ptr, int(nbytes), None))


def bgemv(w, x):
    """Y = X W^T for 1..8 rows on the matrix cores (batched decode projection):
    W FP16 natural [rows, cols], X FP32 [batch, cols]. Returns Y [batch, rows]."""
    w = np.ascontiguousarray(w, np.float16)
    x = np.ascontiguousarray(x, np.float32)
    batch, cols = x.shape
    rows = w.shape[0]
    wd, xd, yd = DeviceBuffer.from_array(w), DeviceBuffer.from_array(x), DeviceBuffer(batch * rows * 4)
    _check(_LIB.qwen_gpu_op_bgemv(wd.ptr, xd.ptr, yd.ptr, batch, rows, cols, None))
    synchronize()
    return yd.to_array(np.float32, batch * rows).reshape(batch, rows)


def attention_prefill(qkv, keys, values, pos0):
    """Causal GQA attention of a prefill chunk on the matrix cores: qkv FP32
    [rows, 4096] (queries in columns 0..2047), keys / values FP16 [8, context,
    128] holding positions 0 .. pos0 + rows - 1. Returns FP32 [rows, 2048]
    (the kernel's FP16 hi + lo planes summed)."""
    qkv = np.ascontiguousarray(qkv, np.float32)
    keys = np.ascontiguousarray(keys, np.float16)
    values = np.ascontiguousarray(values, np.float16)
    # The kernel reads qkv rows of 4096 and [8][context][128] caches: shapes
    # are checked here, before any device copy.
    if qkv.ndim != 2 or qkv.shape[1] != 4096:
        raise ValueError(f'qkv must be [rows, 4096], got {qkv.shape}')
    if keys.ndim != 3 or keys.shape[0] != 8 or keys.shape[2] != 128 or values.shape != keys.shape:
        raise ValueError(f'keys and values must both be [8, context, 128], got {keys.shape} and {values.shape}')
    rows, context = qkv.shape[0], keys.shape[1]
    if not (rows >= 1 and 0 <= pos0 and pos0 + rows <= context):
        raise ValueError(f'need 1 <= rows and 0 <= pos0 with pos0 + rows <= context ({rows}, {pos0}, {context})')
    qd, kd, vd = DeviceBuffer.from_array(qkv), DeviceBuffer.from_array(keys), DeviceBuffer.from_array(values)
    hi, lo = DeviceBuffer(rows * 2048 * 2), DeviceBuffer(rows * 2048 * 2)
    _check(_LIB.qwen_gpu_op_attention_prefill(qd.ptr, kd.ptr, vd.ptr, hi.ptr, lo.ptr, rows, pos0, context, None))
    synchronize()
    h = hi.to_array(np.float16, rows * 2048).astype(np.float32)
    l = lo.to_array(np.float16, rows * 2048).astype(np.float32)
    return (h + l).reshape(rows, 2048)


def _gemm_operands(a, w, c):
    """A FP32 [M, K], W FP16 [N, K] with N % 128 == 0 and K % 64 == 0, C (if
    given) [M, N]: checked before anything reaches the device, since the
    kernel reads and writes whole tiles of these shapes."""
    a = np.ascontiguousarray(a, np.float32)
    w = np.ascontiguousarray(w, np.float16)
    if a.ndim != 2 or w.ndim != 2:
        raise ValueError(f'gemm: a and w must be matrices, got {a.shape} and {w.shape}')
    m, k = a.shape
    n = w.shape[0]
    if m < 1 or w.shape[1] != k or n % 128 or k % 64 or n < 128 or k < 64:
        raise ValueError(f'gemm: w must be [N, {k}] with N % 128 == 0 and K % 64 == 0, got a {a.shape}, w {w.shape}')
    if c is not None and np.shape(c) != (m, n):
        raise ValueError(f'gemm: c must be [{m}, {n}], got {np.shape(c)}')
    return a, w, m, n, k


def gemm(a, w, c=None):
    """C = A W^T (or C += A W^T when C is given) on the matrix cores: A FP32
    [M, K], W FP16 [N, K] natural layout. Returns C as a NumPy array."""
    a, w, m, n, k = _gemm_operands(a, w, c)
    ad, wd = DeviceBuffer.from_array(a), DeviceBuffer.from_array(w)
    cd = DeviceBuffer.from_array(np.ascontiguousarray(c, np.float32)) if c is not None else DeviceBuffer(m * n * 4)
    _check(_LIB.qwen_gpu_op_gemm(ad.ptr, wd.ptr, cd.ptr, m, n, k, int(c is not None), None))
    synchronize()
    return cd.to_array(np.float32, m * n).reshape(m, n)


def gemm_swiglu(a, w, exponents=False):
    """Prefill gate/up GEMM with its SwiGLU epilogue: A FP32 [M, K], W FP16
    [N, K] holding N / 2 gate rows then N / 2 up rows. Returns the FP32
    activation [M, N / 2] (the kernel's FP16 hi + lo planes summed and scaled
    by 2^exponent of each group of 8), and with exponents=True also those
    exponents [M, N / 16]."""
    a = np.ascontiguousarray(a, np.float32)
    w = np.ascontiguousarray(w, np.float16)
    m, k = a.shape
    n = w.shape[0]
    if w.shape[1] != k or n % 256 or k % 64:
        raise ValueError(f'need W [N, K] with N % 256 == 0 and K % 64 == 0, got A {a.shape} W {w.shape}')
    ad, wd = DeviceBuffer.from_array(a), DeviceBuffer.from_array(w)
    hi, lo = DeviceBuffer(m * n // 2 * 2), DeviceBuffer(m * n // 2 * 2)
    ex = DeviceBuffer(m * n // 16)
    _check(_LIB.qwen_gpu_op_gemm_swiglu(ad.ptr, wd.ptr, hi.ptr, lo.ptr, ex.ptr, m, n, k, None))
    synchronize()
    h = hi.to_array(np.float16, m * n // 2).astype(np.float32)
    l = lo.to_array(np.float16, m * n // 2).astype(np.float32)
    e = ex.to_array(np.uint8, m * n // 16).reshape(m, n // 16)
    act = ((h + l).reshape(m, n // 16, 8) * np.exp2(e.astype(np.float32))[:, :, None]).reshape(m, n // 2)
    return (act, e) if exponents else act


def _vector(values, size, name):
    values = np.ascontiguousarray(values, np.float32)
    if values.shape != (size,):
        raise ValueError(f'{name} must have shape ({size},), got {values.shape}')
    return DeviceBuffer.from_array(values)


def _parts(parts):
    if parts is None:
        return None
    parts = np.ascontiguousarray(parts, np.float32)
    if parts.shape != (16, HIDDEN):
        raise ValueError(f'parts must be [16, 1024], got {parts.shape}')
    return DeviceBuffer.from_array(parts)


def norm_qkv(tiled, norm_weight, x):
    """Decode QKV projection as a step runs it: W_qkv (chain-tiled [4096 x
    1024] DeviceBuffer) . RMSNorm(x). Returns qkv [4096]."""
    nd, xd, out = _vector(norm_weight, HIDDEN, 'norm_weight'), _vector(x, HIDDEN, 'x'), DeviceBuffer(4096 * 4)
    _check(_LIB.qwen_gpu_op_norm_qkv(tiled.ptr, nd.ptr, xd.ptr, out.ptr, None))
    synchronize()
    return out.to_array(np.float32, 4096)


def norm_gate_up(tiled, norm_weight, x, parts=None):
    """Decode gate/up projection + SwiGLU as a step runs it (tiled: gate and
    up interleaved, tile_matrix(gate, up)); parts: pending [16, 1024] O
    partials folded into x first, or None. Returns (act [3072], gate [3072],
    up [3072]), the last two being the kernel's dot products."""
    nd, xd = _vector(norm_weight, HIDDEN, 'norm_weight'), _vector(x, HIDDEN, 'x')
    pd, out, raw = _parts(parts), DeviceBuffer(3072 * 4), DeviceBuffer(6144 * 4)
    _check(_LIB.qwen_gpu_op_norm_gate_up(tiled.ptr, nd.ptr, xd.ptr, pd.ptr if pd else None, out.ptr, raw.ptr, None))
    synchronize()
    rows = raw.to_array(np.float32, 6144).reshape(768, 2, 4)  # tile, (gate, up), row in tile
    return out.to_array(np.float32, 3072), rows[:, 0, :].reshape(3072), rows[:, 1, :].reshape(3072)


def down_residual(tiled, act, x, parts=None):
    """Decode down projection + residual as a step runs it: returns
    (x + folded parts) + W_down . act, W_down chain-tiled [1024 x 3072]."""
    ad, xd, pd = _vector(act, 3072, 'act'), _vector(x, HIDDEN, 'x'), _parts(parts)
    _check(_LIB.qwen_gpu_op_down_residual(tiled.ptr, ad.ptr, pd.ptr if pd else None, xd.ptr, None))
    synchronize()
    return xd.to_array(np.float32, HIDDEN)


class FusedFfn:
    """The fused decode FFN kernel on caller data (parity-test entry): holds
    the exchange buffer and the launch tag, as an engine does."""

    def __init__(self):
        self.exchange = DeviceBuffer.from_array(np.zeros(3072, np.uint64))
        self.stall = DeviceBuffer.from_array(np.zeros(1, np.int32))
        self.tag = 0

    def __call__(self, gateup_tiled, down_tiled, norm_weight, x, parts=None):
        """Returns (xm [1024], dparts [8, 1024], act [3072] as exchanged,
        stalled)."""
        nd, xd = _vector(norm_weight, HIDDEN, 'norm_weight'), _vector(x, HIDDEN, 'x')
        pd = _parts(parts if parts is not None else np.zeros((16, HIDDEN), np.float32))
        xm, dparts = DeviceBuffer(HIDDEN * 4), DeviceBuffer(8 * HIDDEN * 4)
        self.tag = self.tag % 0xFFFFFFFF + 1
        _check(_LIB.qwen_gpu_op_fused_ffn(gateup_tiled.ptr, down_tiled.ptr, nd.ptr, xd.ptr, pd.ptr, xm.ptr, dparts.ptr,
                                          self.exchange.ptr, self.stall.ptr, self.tag, None))
        synchronize()
        words = self.exchange.to_array(np.uint64, 3072)
        if not np.all((words >> np.uint64(32)) == np.uint64(self.tag)):
            raise RuntimeError('fused FFN: exchange words do not carry this launch tag')
        act = (words & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
        stalled = int(self.stall.to_array(np.int32, 1)[0])
        return (xm.to_array(np.float32, HIDDEN), dparts.to_array(np.float32, 8 * HIDDEN).reshape(8, HIDDEN), act,
                stalled)


def norm_qkv_folded(tiled, norm_weight, xm, dparts):
    """QKV of a layer after a fused FFN layer: x = xm + the 8 down slices
    (fixed tree order), qkv = W_qkv . RMSNorm(x). Returns (x, qkv)."""
    dparts = np.ascontiguousarray(dparts, np.float32)
    if dparts.shape != (8, HIDDEN):
        raise ValueError(f'dparts must be [8, 1024], got {dparts.shape}')
    nd, xmd, dd = _vector(norm_weight, HIDDEN, 'norm_weight'), _vector(xm, HIDDEN, 'xm'), DeviceBuffer.from_array(dparts)
    xd, out = DeviceBuffer(HIDDEN * 4), DeviceBuffer(4096 * 4)
    _check(_LIB.qwen_gpu_op_norm_qkv_folded(tiled.ptr, nd.ptr, xmd.ptr, dd.ptr, xd.ptr, out.ptr, None))
    synchronize()
    return xd.to_array(np.float32, HIDDEN), out.to_array(np.float32, 4096)


def gemm_static(a, w, c=None):
    """gemm() through the entry point that allocates nothing (operand planes
    in the library's static device array; M x K at most 1048576)."""
    a, w, m, n, k = _gemm_operands(a, w, c)
    ad, wd = DeviceBuffer.from_array(a), DeviceBuffer.from_array(w)
    cd = DeviceBuffer.from_array(np.ascontiguousarray(c, np.float32)) if c is not None else DeviceBuffer(m * n * 4)
    _check(_LIB.qwen_gpu_op_gemm_static(ad.ptr, wd.ptr, cd.ptr, m, n, k, int(c is not None), None))
    synchronize()
    return cd.to_array(np.float32, m * n).reshape(m, n)
