"""INT8 append parity on the GPU: codes and scales bit-exact against the oracle
(kernels.metal:129-141), guards around the written range (Int8KvTests.cs:43,64-70),
partial RoPE to tolerance (KvStorageTests.cs:44-57, Int8KvTests.cs:46-62)."""
import hashlib
import json
import os

import numpy as np
import pytest

from bootstrap_hip import KernelArgs, engine
from kvcase import outlier_kv, reference_kv, upload

pytestmark = pytest.mark.gpu


def run_store(device, oracle, k, v, pos, guard=0x55):
    rows = k.shape[0]
    length = pos + rows
    kc, vc, ks, vs = oracle.empty_cache(length + 1, fill=guard)
    ref = [a.copy() for a in (kc, vc, ks, vs)]
    oracle.store(k, v, pos, *ref)
    bufs = [upload(device, a) for a in (kc, vc, ks, vs)]
    kb, vb = upload(device, k), upload(device, v)
    device.begin()
    device.dispatch("kv_store_int8", KernelArgs(M=rows, Position=pos), rows * 512, 256, kb, vb, *bufs)
    device.end()
    got = [b.read(a.dtype, a.size) for b, a in zip(bufs, (kc, vc, ks, vs))]
    for b in bufs + [kb, vb]:
        b.dispose()
    return got, ref


def assert_same_bytes(got, ref):
    names = ("K codes", "V codes", "K scales", "V scales")
    for name, a, b in zip(names, got, ref):
        assert a.view(np.uint8).tobytes() == b.view(np.uint8).tobytes(), name


def test_config1_append_512_bitexact(device, oracle):
    """Config 1: 512 tokens of N(0,1) K/V, seed 0, at position 0; the device cache also
    hashes to the committed digests of tests/golden/kv_golden.json."""
    k = oracle.normal(512 * 512, 0).reshape(512, 2, 256)
    v = oracle.normal(512 * 512, 1).reshape(512, 2, 256)
    got, ref = run_store(device, oracle, k, v, 0, guard=0)
    assert_same_bytes(got, ref)
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kv_golden.json")) as f:
        digests = json.load(f)["config1"]["sha256"]
    for name, a in zip(("key_codes", "value_pages", "key_scales", "value_scales"), got):
        assert hashlib.sha256(a.tobytes()).hexdigest() == digests[name], name


@pytest.mark.parametrize("pos,rows", [(0, 1), (17, 7), (63, 2), (255, 2), (4093, 33), (1000, 600), (4096, 512),
                                      (200000 - 37, 80), (37, 5000), (8192, 8192), (65536 - 100, 4300)])
def test_append_positions_and_guards(device, oracle, pos, rows):
    """Unaligned starts, page crossings and single tokens; bytes outside the written range keep 0x55.
    Appends of 4096 rows or more take the 64-token tiles (whole and partial ones)."""
    k, v = reference_kv(rows, seed=pos + rows)
    assert_same_bytes(*run_store(device, oracle, k, v, pos))


# A seeded sweep of (position, rows): starts anywhere in a page, 1 to 9000 rows (both tile sizes,
# partial tiles at either end), Student-t K/V
APPEND_SWEEP = [(int(p), int(r)) for p, r in zip(np.random.default_rng(2029).integers(0, 250000, 10),
                                                 [1, 3, 16, 17, 255, 257, 1023, 4095, 4097, 9000])]


@pytest.mark.parametrize("pos,rows", APPEND_SWEEP)
def test_append_shape_sweep(device, oracle, pos, rows):
    rng = np.random.default_rng(pos + rows)
    k = rng.standard_t(4, (rows, 2, 256)).astype(np.float32)
    v = rng.standard_t(4, (rows, 2, 256)).astype(np.float32)
    assert_same_bytes(*run_store(device, oracle, k, v, pos))


def test_append_special_values(device, oracle):
    rows = 8
    k = np.zeros((rows, 2, 256), np.float32)
    v = np.zeros((rows, 2, 256), np.float32)
    k[1, 0, :6] = [127.0, 2.5, 3.5, -2.5, -3.5, -0.0]        # exact ties -> even
    v[1, 1, :3] = [-0.0, 1e-30, -1e-30]                       # tiny magnitudes
    k[2] = np.float32(-97.0)                                  # constant vector
    v[3, 0, 255] = 41.0                                       # single outlier
    rng = np.random.default_rng(4)
    k[4:] = (rng.standard_t(4, (4, 2, 256)) * 30).astype(np.float32)
    v[4:] = (rng.standard_normal((4, 2, 256)) * 1e-4).astype(np.float32)
    (got, ref) = run_store(device, oracle, k, v, 300)
    assert_same_bytes(got, ref)
    ks = got[2]
    assert ks[300 * 2] == 0 and ks[300 * 2 + 1] == 0         # zero vectors: scale 0 (Int8KvTests.cs:60)


def test_heavy_tailed_outliers_bitexact(device, oracle):
    k, v = outlier_kv(oracle, 1024, seed=12, heavy=True)
    assert_same_bytes(*run_store(device, oracle, k, v, 131072 - 512, guard=0))


def rotate_fp32_angle(x, position, theta=1e7):
    """kernels.metal:122-125 with the reference's FP32 angle: angle = float(position) *
    float(theta^(-2j/64)) rounded to FP32 at each step, then an exact rotation of that angle
    (FP64 cos/sin); dims >= 64 pass through."""
    x = np.asarray(x, np.float64)
    j = np.arange(32)
    ifreq = np.power(np.float64(theta), -2.0 * j / 64.0).astype(np.float32)
    angle = (np.float32(position) * ifreq).astype(np.float32).astype(np.float64)
    out = x.copy()
    a, b = x[:32], x[32:64]
    out[:32] = a * np.cos(angle) - b * np.sin(angle)
    out[32:64] = b * np.cos(angle) + a * np.sin(angle)
    return out


def test_batch_rope_int8_fp32_angles_deep_window(device, oracle):
    """The last 8 positions of the 262144-token window, where an FP32 angle is off from the exact
    one by up to ~0.016 rad: the rotation must follow the reference's FP32 angle arithmetic
    (kernels.metal:122-125), so against that restatement the error is the FP32 rounding of
    cos/sin and of the rotation alone."""
    rows, position = 8, 262136
    length = position + rows
    q = oracle.fill_hash(rows * 4096, 41, 3)
    k = oracle.fill_hash(rows * 512, 43, 3)
    v = oracle.fill_hash(rows * 512, 47, 1)
    kc, vc, ks, vs = oracle.empty_cache(length)
    bufs = [upload(device, a) for a in (kc, vc, ks, vs)]
    qb, kb, vb = upload(device, q), upload(device, k), upload(device, v)
    qr = device.allocate(q.nbytes)
    layer = engine.Int8KvLayer.__new__(engine.Int8KvLayer)
    layer.key, layer.value, layer.key_scale, layer.value_scale = bufs
    device.begin()
    engine.append_rows(device, layer, qb, kb, vb, qr, rows, position)
    device.end()
    rotated_q = qr.read(np.float32, rows * 4096)
    exact_gap = 0.0
    for row in range(rows):
        for head in range(16):
            src = q[(row * 16 + head) * 256:][:256]
            ref = rotate_fp32_angle(src, position + row)
            got = rotated_q[(row * 16 + head) * 256:][:256]
            assert np.max(np.abs(got - ref)) < 2e-5, (row, head, np.max(np.abs(got - ref)))
            exact_gap = max(exact_gap, np.max(np.abs(ref - oracle.rotate_vector_f64(src, position + row))))
    assert exact_gap > 1e-3          # the FP32 angle is far from the exact one this deep
    for b in bufs + [qb, kb, vb, qr]:
        b.dispose()


def test_batch_rope_int8(device, oracle):
    """Int8KvTests.Store (Int8KvTests.cs:33-70) with its inputs and bounds: position 4093,
    33 rows, zero vectors, outliers; Q rotation against FP64 (KvStorageTests.cs:55)."""
    rows, position = 33, 4093
    length = position + rows
    q = oracle.fill_hash(rows * 4096, 17, 3)
    k = oracle.fill_hash(rows * 512, 31, 3)
    v = oracle.fill_hash(rows * 512, 23, 1)
    k[:256] = 0
    v[:256] = 0
    k[777] = -97
    v[999] = 41
    kc, vc, ks, vs = oracle.empty_cache(length + 1, fill=0x55)
    bufs = [upload(device, a) for a in (kc, vc, ks, vs)]
    qb, kb, vb = upload(device, q), upload(device, k), upload(device, v)
    qr = device.allocate(q.nbytes)
    layer = engine.Int8KvLayer.__new__(engine.Int8KvLayer)
    layer.key, layer.value, layer.key_scale, layer.value_scale = bufs
    device.begin()
    engine.append_rows(device, layer, qb, kb, vb, qr, rows, position)
    device.end()
    gkc, gvc, gks, gvs = [b.read(a.dtype, a.size) for b, a in zip(bufs, (kc, vc, ks, vs))]
    rotated_q = qr.read(np.float32, rows * 4096)
    worst = 0.0
    for row in range(rows):
        for head in range(16):
            ref = oracle.rotate_vector_f64(q[(row * 16 + head) * 256:][:256], position + row)
            got = rotated_q[(row * 16 + head) * 256:][:256]
            # fp32 angle rounding at position ~4125 (ulp 4.9e-4 rad) times |x| <= 2
            assert np.max(np.abs(got - ref)) < 2e-3
        for h in range(2):
            vector, dest = row * 2 + h, (position + row) * 2 + h
            key = oracle.rotate_vector_f64(k[vector * 256:][:256], position + row)
            val = v[vector * 256:][:256].astype(np.float64)
            for codes, scale, original in (
                    (gkc[dest * 256:(dest + 1) * 256], gks[dest], key),
                    (np.array([gvc[oracle.value_index(dest, d)] for d in range(256)], np.int8), gvs[dest], val)):
                maximum = np.abs(original).max()
                assert abs(scale - maximum / 127) < 2e-5                              # Int8KvTests.cs:54
                err = np.abs(codes.astype(np.float64) * scale - original)
                worst = max(worst, err.max())
                assert codes.min() >= -127 and np.all(err <= maximum / 254 + 3e-3)   # Int8KvTests.cs:59
                if maximum == 0:
                    assert not codes.any() and scale == 0
            # V is not rotated: its codes are exactly the oracle's quantization
            cv, sv = oracle.quantize(v[vector * 256:][:256])
            assert np.array_equal(np.array([gvc[oracle.value_index(dest, d)] for d in range(256)], np.int8), cv)
            assert gvs[dest] == sv
    # prefix and tail guards (Int8KvTests.cs:64-70)
    assert np.all(gkc[:position * 512].view(np.uint8) == 0x55)
    assert np.all(gkc[length * 512:].view(np.uint8) == 0x55)
    assert np.all(gks[:position * 2].view(np.uint32) == 0x55555555)
    pages = gvc.reshape(-1, 2, 256, 256).view(np.uint8)
    for t in list(range(position - 3, position)) + list(range(length, length + 1)):
        assert np.all(pages[t // 256, :, :, t % 256] == 0x55)
    for b in bufs + [qb, kb, vb, qr]:
        b.dispose()


def test_query_grouped_half_bitexact(device, oracle):
    rows = 37
    x = oracle.fill_hash(rows * 4096, 5, 40)
    xb = upload(device, x)
    yb = device.allocate(rows * 4096 * 2)
    device.begin()
    device.dispatch("attention_query_grouped_half", KernelArgs(M=rows, A=8), rows * 1024, 128, xb, yb)
    device.end()
    assert np.array_equal(yb.read(np.uint16, rows * 4096), oracle.query_grouped_half(x, rows, 8))
    xb.dispose()
    yb.dispose()


def test_dispatch_validation_errors(device):
    """Undersized bindings are rejected on the host before any launch (no GPU fault)."""
    from bootstrap_hip import HipError
    small = device.allocate(1024)
    device.begin()
    with pytest.raises(HipError, match="too small|smaller"):
        device.dispatch("kv_store_int8", KernelArgs(M=4, Position=0), 2048, 256, small, small, small, small, small,
                        small)
    with pytest.raises(HipError, match="Unknown kernel"):
        device.dispatch("no_such_kernel", KernelArgs(), 1, 1, small)
    device.end()
    with pytest.raises(HipError, match="requires an active command"):
        device.dispatch("kv_store_int8", KernelArgs(M=1), 1, 1, small)
    small.dispose()


def test_attention_dispatch_validation_errors(device):
    """The attention launchers reject, on the host and before any launch, what the
    reference's call sites never pass: a group size other than 8, K != Position + M,
    a history beyond the 262144-token window, missing or undersized or misaligned
    bindings, more than 64 decode rows, and more reader rows than the values merge's grid holds."""
    from bootstrap_hip import HipError
    rows, pos = 4, 100
    keys = pos + rows
    q = device.allocate(rows * 8192 + 64)
    cache_k, cache_v = device.allocate(keys * 512), device.allocate((keys + 255) // 256 * 256 * 512)
    gate, y = device.allocate(rows * 16384), device.allocate(rows * 16384)
    ks, vs = device.allocate(keys * 8), device.allocate(keys * 8)
    name = "attention_online_int8_q32_k256_r2"
    bind = (q, cache_k, cache_v, gate, y, ks, vs)
    cases = [
        (name, KernelArgs(M=rows, K=keys, Position=pos, A=4), bind, "A = 8"),
        (name, KernelArgs(M=rows, K=keys + 1, Position=pos, A=8), bind, "K must equal"),
        (name, KernelArgs(M=1, K=262145, Position=262144, A=8), bind, "262144-token window"),
        (name, KernelArgs(M=rows, K=keys, Position=pos, A=8), bind[:6], "needs 7 bindings"),
        (name, KernelArgs(M=rows, K=keys, Position=pos, A=8), (ks,) + bind[1:], "query smaller"),
        (name, KernelArgs(M=rows, K=keys, Position=pos, A=8), (q.at(4),) + bind[1:], "misaligned"),
        ("attention_decode_int8", KernelArgs(M=65, K=keys, Position=pos), bind, "at most 64 rows"),
        ("attention_decode_int8", KernelArgs(M=rows, K=keys, Position=pos), bind[:6], "needs 7 bindings"),
        ("batch_attention_values_int8", KernelArgs(M=65536, K=65636, Position=pos), bind[:5], "at most 65535 rows"),
    ]
    for kernel, args, bindings, message in cases:
        device.begin()
        with pytest.raises(HipError, match=message):
            device.dispatch(kernel, args, rows * 4096, 256, *bindings)
        device.end()
    for b in bind:
        b.dispose()
