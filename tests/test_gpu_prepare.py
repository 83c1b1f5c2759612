"""Fused INT8 preparation (attention_prepare_fused_int8, kernels.metal:1902-1914) on the GPU.

Pinned the way the reference pins it (Int8KvTests.cs:71-90): bitwise equal to the unfused
chain batch_split_q -> rmsnorm (q_norm, k_norm) -> batch_rope_int8 ->
attention_query_grouped_half, on the reference's inputs (position 4093, 33 rows, hash-filled
qkv/K/V, q_norm weight 0x3e00, k_norm weight 0xbe00). Also checked against an FP64
RMSNorm + RoPE + quantization reference with the bounds of Int8KvTests.cs:54-59."""
import numpy as np
import pytest

from bootstrap_hip import KernelArgs
from kvcase import upload

pytestmark = pytest.mark.gpu

ROWS, POSITION = 33, 4093
LENGTH = POSITION + ROWS


def inputs(oracle):
    raw = oracle.fill_hash(ROWS * 8192, 31, 2)
    k = oracle.fill_hash(ROWS * 512, 31, 3)
    v = oracle.fill_hash(ROWS * 512, 23, 1)
    k[:256] = 0
    v[:256] = 0
    k[777] = -97
    v[999] = 41
    qw = np.full(256, 0x3E00, np.uint16)    # bf16 0.125
    kw = np.full(256, 0xBE00, np.uint16)    # bf16 -0.125
    return raw, k, v, qw, kw


def cache_buffers(device, oracle):
    kc, vc, ks, vs = oracle.empty_cache(LENGTH + 1, fill=0x55)
    return [upload(device, a) for a in (kc, vc, ks, vs)], (kc, vc, ks, vs)


def test_fused_equals_unfused_bitwise(device, oracle):
    raw, k, v, qw, kw = inputs(oracle)
    p = KernelArgs(M=ROWS, Position=POSITION, K=LENGTH, Theta=10_000_000.0, Epsilon=1e-6, A=8)
    rawb, kb, vb, qwb, kwb = (upload(device, a) for a in (raw, k, v, qw, kw))
    fused_cache, hosts = cache_buffers(device, oracle)
    ref_cache, _ = cache_buffers(device, oracle)
    packed, packed_ref = device.allocate(ROWS * 8192), device.allocate(ROWS * 8192)
    gate, gate_ref = device.allocate(ROWS * 16384), device.allocate(ROWS * 16384)
    split, norm_k, rotated = device.allocate(ROWS * 16384), device.allocate(ROWS * 2048), device.allocate(ROWS * 16384)
    dummy = device.allocate(4)
    device.begin()
    device.dispatch("batch_split_q", p, ROWS * 4096, 128, rawb, split, gate_ref)
    device.dispatch("rmsnorm", KernelArgs(N=256, M=ROWS * 16, Flags=1, Epsilon=1e-6), ROWS * 16 * 256, 256,
                    split, qwb, split, dummy)
    device.dispatch("rmsnorm", KernelArgs(N=256, M=ROWS * 2, Flags=1, Epsilon=1e-6), ROWS * 2 * 256, 256,
                    kb, kwb, norm_k, dummy)
    device.dispatch("batch_rope_int8", p, ROWS * 4096, 256, split, norm_k, vb, rotated, *ref_cache)
    device.dispatch("attention_query_grouped_half", p, ROWS * 1024, 128, rotated, packed_ref)
    device.dispatch("attention_prepare_fused_int8", p, ROWS * 18 * 256, 256, rawb, kb, vb, qwb, kwb, packed, gate,
                    *fused_cache)
    device.end()
    assert packed.read(np.uint8, ROWS * 8192).tobytes() == packed_ref.read(np.uint8, ROWS * 8192).tobytes()
    assert gate.read(np.uint8, ROWS * 16384).tobytes() == gate_ref.read(np.uint8, ROWS * 16384).tobytes()
    for a, b, host in zip(fused_cache, ref_cache, hosts):
        assert a.read(np.uint8, host.nbytes).tobytes() == b.read(np.uint8, host.nbytes).tobytes()
    for buf in [rawb, kb, vb, qwb, kwb, packed, packed_ref, gate, gate_ref, split, norm_k, rotated, dummy,
                *fused_cache, *ref_cache]:
        buf.dispose()


def test_fused_matches_fp64(device, oracle):
    raw, k, v, qw, kw = inputs(oracle)
    p = KernelArgs(M=ROWS, Position=POSITION, K=LENGTH, Theta=10_000_000.0, Epsilon=1e-6, A=8)
    rawb, kb, vb, qwb, kwb = (upload(device, a) for a in (raw, k, v, qw, kw))
    cache, hosts = cache_buffers(device, oracle)
    packed, gate = device.allocate(ROWS * 8192), device.allocate(ROWS * 16384)
    device.begin()
    device.dispatch("attention_prepare_fused_int8", p, ROWS * 18 * 256, 256, rawb, kb, vb, qwb, kwb, packed, gate,
                    *cache)
    device.end()
    got_q = packed.read(np.float16, ROWS * 4096).astype(np.float64).reshape(2, ROWS, 8, 256)
    got_gate = gate.read(np.float32, ROWS * 4096).reshape(ROWS, 16, 256)
    kc, vc, ks, vs = (buf.read(h.dtype, h.size) for buf, h in zip(cache, hosts))
    qkv = raw.reshape(ROWS, 16, 2, 256)
    assert np.array_equal(got_gate, qkv[:, :, 1, :])                       # gate split is a copy

    def norm(x, w_bits):
        w = (w_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        x = x.astype(np.float64)
        return x / np.sqrt(np.mean(x * x) + 1e-6) * (w + 1)

    for row in range(ROWS):
        for h in range(16):
            expected = oracle.rotate_vector_f64(norm(qkv[row, h, 0], qw).astype(np.float32), POSITION + row)
            # FP16 rounding (<= 2^-11 relative) + fp32 angle rounding at position ~4125
            assert np.max(np.abs(got_q[h // 8, row, h % 8] - expected)) <= 2e-3 + np.abs(expected).max() * 2 ** -10
        for g in range(2):
            dest = (POSITION + row) * 2 + g
            key = oracle.rotate_vector_f64(norm(k.reshape(ROWS, 2, 256)[row, g], kw).astype(np.float32), POSITION + row)
            maximum = np.abs(key).max()
            codes = kc[dest * 256:(dest + 1) * 256]
            assert abs(ks[dest] - maximum / 127) < 2e-5                                   # Int8KvTests.cs:54
            assert codes.min() >= -127 and np.all(np.abs(codes * ks[dest] - key) <= maximum / 254 + 3e-3)
            cv, sv = oracle.quantize(v.reshape(ROWS, 2, 256)[row, g])
            assert np.array_equal(np.array([vc[oracle.value_index(dest, d)] for d in range(256)], np.int8), cv)
            assert vs[dest] == sv
    for buf in [rawb, kb, vb, qwb, kwb, packed, gate, *cache]:
        buf.dispose()


def test_fused_fp16_equals_unfused_bitwise(device, oracle):
    """FP16-KV fused preparation (attention_prepare_fused, kernels.metal:1889-1901) against the
    unfused FP16 chain batch_split_q -> rmsnorm -> batch_rope (flags 256) ->
    attention_query_grouped_half: packed query, gate and the FP16 K/V cache bitwise equal, and the
    cache outside the appended rows untouched."""
    raw, k, v, qw, kw = inputs(oracle)
    p = KernelArgs(M=ROWS, Position=POSITION, K=LENGTH, Theta=10_000_000.0, Epsilon=1e-6, A=8, Flags=256)
    rawb, kb, vb, qwb, kwb = (upload(device, a) for a in (raw, k, v, qw, kw))
    guard = np.full((LENGTH + 1) * 512, 0x5555, np.uint16)
    fused_k, fused_v, ref_k, ref_v = (upload(device, guard) for _ in range(4))
    packed, packed_ref = device.allocate(ROWS * 8192), device.allocate(ROWS * 8192)
    gate, gate_ref = device.allocate(ROWS * 16384), device.allocate(ROWS * 16384)
    split, norm_k, rotated = device.allocate(ROWS * 16384), device.allocate(ROWS * 2048), device.allocate(ROWS * 16384)
    dummy = device.allocate(4)
    device.begin()
    device.dispatch("batch_split_q", p, ROWS * 4096, 128, rawb, split, gate_ref)
    device.dispatch("rmsnorm", KernelArgs(N=256, M=ROWS * 16, Flags=1, Epsilon=1e-6), ROWS * 16 * 256, 256,
                    split, qwb, split, dummy)
    device.dispatch("rmsnorm", KernelArgs(N=256, M=ROWS * 2, Flags=1, Epsilon=1e-6), ROWS * 2 * 256, 256,
                    kb, kwb, norm_k, dummy)
    device.dispatch("batch_rope", p, ROWS * 4096, 128, split, norm_k, vb, rotated, ref_k, ref_v)
    device.dispatch("attention_query_grouped_half", p, ROWS * 1024, 128, rotated, packed_ref)
    device.dispatch("attention_prepare_fused", p, ROWS * 18 * 256, 256, rawb, kb, vb, qwb, kwb, packed, gate,
                    fused_k, fused_v)
    device.end()
    assert packed.read(np.uint8, ROWS * 8192).tobytes() == packed_ref.read(np.uint8, ROWS * 8192).tobytes()
    assert gate.read(np.uint8, ROWS * 16384).tobytes() == gate_ref.read(np.uint8, ROWS * 16384).tobytes()
    for a, b in ((fused_k, ref_k), (fused_v, ref_v)):
        got = a.read(np.uint16, guard.size)
        assert got.tobytes() == b.read(np.uint16, guard.size).tobytes()
        assert np.all(got[:POSITION * 512] == 0x5555) and np.all(got[LENGTH * 512:] == 0x5555)
    for buf in [rawb, kb, vb, qwb, kwb, fused_k, fused_v, ref_k, ref_v, packed, packed_ref, gate, gate_ref, split,
                norm_k, rotated, dummy]:
        buf.dispose()
