"""Shared GPU-test fixtures: seeded INT8 caches built on the host by the oracle, uploaded
to device buffers, with the reference's poisoned tails (Int8KvTests.cs:107-122)."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def reference_kv(length: int, seed: int = 2941):
    """Int8KvTests.cs:107-113 structure: K ~ U(-3,3), V ~ U(-1,1), V zero every 41st vector,
    K zero every 37th, K[13] = -17 when vector % 43 == 1 (own seeded RNG)."""
    rng = np.random.default_rng(seed)
    keys = rng.uniform(-3, 3, (length * 2, 256)).astype(np.float32)
    values = rng.uniform(-1, 1, (length * 2, 256)).astype(np.float32)
    vec = np.arange(length * 2)
    values[vec % 41 == 0] = 0
    keys[vec % 37 == 0] = 0
    keys[vec % 43 == 1, 13] = -17
    return keys.reshape(length, 2, 256), values.reshape(length, 2, 256)


def outlier_kv(oracle, length: int, seed: int, heavy: bool = False):
    """Config distributions: N(0,1) (or Student-t nu=4) with K channels {30,31,62,63} x 20."""
    gen = oracle.student_t4 if heavy else oracle.normal
    k = gen(length * 512, seed).reshape(length, 2, 256)
    v = gen(length * 512, seed + 1).reshape(length, 2, 256)
    k[:, :, [30, 31, 62, 63]] *= 20
    return np.ascontiguousarray(k), np.ascontiguousarray(v)


def poison_tail(oracle, kc, vc, ks, vs, length: int):
    """Codes -128 and NaN scales for every token >= length (Int8KvTests.cs:121-122)."""
    kc[length * 512:] = -128
    pages = vc.reshape(-1, 2, 256, 256)
    tokens = np.arange(pages.shape[0] * 256)
    for t in tokens[tokens >= length]:
        pages[t // 256, :, :, t % 256] = -128
    ks[length * 2:] = np.nan
    vs[length * 2:] = np.nan


@dataclass
class DeviceCache:
    kc: object
    vc: object
    ks: object
    vs: object

    def dispose(self):
        for b in (self.kc, self.vc, self.ks, self.vs):
            b.dispose()


def upload_cache(device, kc, vc, ks, vs) -> DeviceCache:
    bufs = []
    for host in (kc, vc, ks, vs):
        b = device.allocate(host.nbytes)
        b.write(host)
        bufs.append(b)
    return DeviceCache(*bufs)


def upload(device, array: np.ndarray, extra_bytes: int = 0):
    b = device.allocate(array.nbytes + extra_bytes)
    b.write(array)
    return b


def rel_l2(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(got, np.float64) - ref) / max(np.linalg.norm(ref), 1e-300))


def fp32_reader(q, kc, vc, ks, vs, gate, rows: int, history: int) -> np.ndarray:
    """The reference's scalar reader in float32 arithmetic on the CPU, with its order of
    accumulation (kernels.metal:147-166): each score's dot product summed over the dimensions in
    order, times ks / 16; the softmax's sum as 256 strided per-thread sums (one threadgroup of 256
    per row and head) then combined; each output summed over the keys in order, p * vs * code,
    times sigmoid(gate). A float32 baseline for the GPU paths' rounding (NumPy reduces along a
    leading axis element by element in order)."""
    length = history + rows
    codes_k = kc.reshape(-1, 2, 256)[:length].astype(np.float32)
    pages = (length + 255) // 256
    codes_v = vc[:pages * 2 * 65536].reshape(pages, 2, 256, 256).transpose(0, 3, 1, 2).reshape(pages * 256, 2, 256)
    codes_v = codes_v[:length].astype(np.float32)
    ks2, vs2 = ks.reshape(-1, 2)[:length], vs.reshape(-1, 2)[:length]
    q3, g3 = q.reshape(rows, 16, 256).astype(np.float32), gate.reshape(rows, 16, 256).astype(np.float32)
    kt = [np.ascontiguousarray(codes_k[:, kv].T) for kv in range(2)]   # [256 dims][keys]
    y = np.empty((rows, 16, 256), np.float32)
    for r in range(rows):
        end = history + r + 1
        for h in range(16):
            kv = h // 8
            dots = (kt[kv][:, :end] * q3[r, h][:, None]).sum(axis=0, dtype=np.float32)
            s = dots * ks2[:end, kv] * np.float32(1.0 / 16.0)
            e = np.exp(s - s.max(), dtype=np.float32)
            padded = np.zeros(((end + 255) // 256) * 256, np.float32)
            padded[:end] = e
            total = padded.reshape(-1, 256).sum(axis=0, dtype=np.float32).sum(dtype=np.float32)
            w = (e / total) * vs2[:end, kv]
            o = (codes_v[:end, kv] * w[:, None]).sum(axis=0, dtype=np.float32)
            y[r, h] = o * (np.float32(1.0) / (np.float32(1.0) + np.exp(-g3[r, h], dtype=np.float32)))
    return y.ravel()
