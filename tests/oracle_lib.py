"""numpy-facing ctypes wrapper of the CPU oracle (oracle/libkvref.so). Test infrastructure."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
# KVREF_LIBRARY selects another build of the same source (the sanitizer build of `make sanitize`)
ORACLE_LIB = os.environ.get("KVREF_LIBRARY", os.path.join(ORACLE_DIR, "libkvref.so"))

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")


def _build():
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


class Oracle:
    def __init__(self):
        if not os.path.exists(ORACLE_LIB):
            _build()
        lib = ctypes.CDLL(ORACLE_LIB)
        lib.kvref_value_index.restype = ctypes.c_uint64
        lib.kvref_value_index.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        lib.kvref_value_bytes.restype = ctypes.c_uint64
        lib.kvref_value_bytes.argtypes = [ctypes.c_uint32]
        lib.kvref_quantize.argtypes = [_f32p, _i8p, ctypes.POINTER(ctypes.c_float)]
        lib.kvref_store.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, _i8p, _i8p, _f32p, _f32p]
        lib.kvref_store_mt.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, _i8p, _i8p, _f32p, _f32p, ctypes.c_int]
        lib.kvref_rotate_f64.restype = ctypes.c_double
        lib.kvref_rotate_f64.argtypes = [_f32p, ctypes.c_int, ctypes.c_int]
        lib.kvref_half_bits.restype = ctypes.c_uint16
        lib.kvref_half_bits.argtypes = [ctypes.c_float]
        lib.kvref_half_to_float.restype = ctypes.c_float
        lib.kvref_half_to_float.argtypes = [ctypes.c_uint16]
        lib.kvref_bf16_round.restype = ctypes.c_float
        lib.kvref_bf16_round.argtypes = [ctypes.c_float]
        lib.kvref_query_grouped_half.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _u16p]
        lib.kvref_attention_f64.argtypes = [_f32p, ctypes.c_int, _i8p, _i8p, _f32p, _f32p, _f32p,
                                            ctypes.c_int, ctypes.c_int, _f64p, ctypes.c_void_p, ctypes.c_int]
        lib.kvref_attention_fp16kv_f64.argtypes = [_f32p, ctypes.c_int, _u16p, _u16p, _f32p,
                                                   ctypes.c_int, ctypes.c_int, _f64p, ctypes.c_int]
        lib.kvref_attention_online_emulate.argtypes = [_f32p, _i8p, _i8p, _f32p, _f32p, _f32p, ctypes.c_int,
                                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int]
        lib.kvref_fill_hash.argtypes = [_f32p, ctypes.c_int64, ctypes.c_uint32, ctypes.c_float]
        lib.kvref_normal.argtypes = [_f32p, ctypes.c_int64, ctypes.c_uint64]
        lib.kvref_splitmix64.argtypes = [ctypes.c_uint64, np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS"),
                                         ctypes.c_int64]
        lib.kvref_student_t4.argtypes = [_f32p, ctypes.c_int64, ctypes.c_uint64]
        self.lib = lib
        self.threads = min(16, os.cpu_count() or 1)

    # ---- layout
    def value_index(self, vector: int, d: int) -> int:
        return int(self.lib.kvref_value_index(vector, d))

    def value_bytes(self, length: int) -> int:
        return int(self.lib.kvref_value_bytes(length))

    # ---- quantization
    def quantize(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        codes = np.zeros(256, np.int8)
        scale = ctypes.c_float()
        self.lib.kvref_quantize(x, codes, ctypes.byref(scale))
        return codes, np.float32(scale.value)

    def store(self, k, v, pos, kc, vc, ks, vs):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        rows = k.size // 512
        self.lib.kvref_store(k.ravel(), v.ravel(), rows, pos, kc, vc, ks, vs)

    def store_mt(self, k, v, pos, kc, vc, ks, vs):
        """kvref_store split over ``self.threads`` threads (same bytes)."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.lib.kvref_store_mt(k.ravel(), v.ravel(), k.size // 512, pos, kc, vc, ks, vs, self.threads)

    def empty_cache(self, length: int, fill: int = 0):
        """Host INT8 cache with room for `length` tokens (whole V pages)."""
        kc = np.full(length * 512, fill, np.uint8).view(np.int8)
        vc = np.full(self.value_bytes(length), fill, np.uint8).view(np.int8)
        ks = np.full(length * 2 * 4, fill, np.uint8).view(np.float32)
        vs = np.full(length * 2 * 4, fill, np.uint8).view(np.float32)
        return kc, vc, ks, vs

    # ---- RoPE / rounding
    def rotate_f64(self, x: np.ndarray, d: int, position: int) -> float:
        return float(self.lib.kvref_rotate_f64(np.ascontiguousarray(x, np.float32), d, position))

    def rotate_vector_f64(self, x: np.ndarray, position: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        return np.array([self.lib.kvref_rotate_f64(x, d, position) for d in range(256)])

    def half_bits(self, f: float) -> int:
        return int(self.lib.kvref_half_bits(f))

    def half_round(self, x: np.ndarray) -> np.ndarray:
        flat = np.ascontiguousarray(x, np.float32).ravel()
        bits = np.array([self.lib.kvref_half_bits(float(v)) for v in flat], np.uint16)
        return np.array([self.lib.kvref_half_to_float(int(b)) for b in bits], np.float32).reshape(np.shape(x))

    def bf16_round(self, f: float) -> float:
        return float(self.lib.kvref_bf16_round(f))

    def query_grouped_half(self, x: np.ndarray, rows: int, group: int = 8) -> np.ndarray:
        y = np.zeros(rows * 4096, np.uint16)
        self.lib.kvref_query_grouped_half(np.ascontiguousarray(x, np.float32).ravel(), rows, group, y)
        return y

    # ---- attention
    def attention(self, q, kc, vc, ks, vs, gate, rows, pos, round_q_half, with_bound=False):
        out = np.zeros(rows * 4096, np.float64)
        bound = np.zeros(rows * 4096, np.float64) if with_bound else None
        self.lib.kvref_attention_f64(np.ascontiguousarray(q, np.float32).ravel(), int(round_q_half),
                                     kc, vc, ks, vs, np.ascontiguousarray(gate, np.float32).ravel(),
                                     rows, pos, out,
                                     bound.ctypes.data if bound is not None else None, self.threads)
        return (out, bound) if with_bound else out

    def attention_fp16kv(self, q, kh, vh, gate, rows, pos, round_q_half):
        out = np.zeros(rows * 4096, np.float64)
        self.lib.kvref_attention_fp16kv_f64(np.ascontiguousarray(q, np.float32).ravel(), int(round_q_half),
                                            kh, vh, np.ascontiguousarray(gate, np.float32).ravel(),
                                            rows, pos, out, self.threads)
        return out

    def online_emulate(self, q, kc, vc, ks, vs, gate, rows, pos, p_mode, tile_keys=256):
        """The reference's online INT8 prefill with its roundings; p_mode 0 BF16 operand
        (kernels.metal:1427), 1 this build's FP16(e*vs/vs_ref), 2 unrounded."""
        out = np.zeros(rows * 4096, np.float32)
        self.lib.kvref_attention_online_emulate(np.ascontiguousarray(q, np.float32).ravel(), kc, vc, ks, vs,
                                                np.ascontiguousarray(gate, np.float32).ravel(), rows, pos,
                                                tile_keys, p_mode, out, self.threads)
        return out

    # ---- generators
    def fill_hash(self, count: int, seed: int, scale: float) -> np.ndarray:
        out = np.zeros(count, np.float32)
        self.lib.kvref_fill_hash(out, count, seed, scale)
        return out

    def splitmix64(self, seed: int, count: int) -> np.ndarray:
        out = np.empty(count, np.uint64)
        self.lib.kvref_splitmix64(seed, out, count)
        return out

    def normal(self, count: int, seed: int) -> np.ndarray:
        out = np.zeros(count, np.float32)
        self.lib.kvref_normal(out, count, seed)
        return out

    def student_t4(self, count: int, seed: int) -> np.ndarray:
        out = np.zeros(count, np.float32)
        self.lib.kvref_student_t4(out, count, seed)
        return out
