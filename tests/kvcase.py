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
