"""boot_dispatch_noalloc (the entry point that allocates nothing) against boot_dispatch on the
same inputs: split-K decode, prefill and the scalar reader on a fresh context, the no-allocation
calls first (before the context has any workspace) with boot_allocated unchanged across each of
them, two calls in a
row with the second smaller, results bitwise equal and within the FP64 bar; sizes beyond the
static scratch are refused, and so is a second context's split-K call while the first context's
command holds the scratch."""
import numpy as np
import pytest

from bootstrap_hip import Device, HipError, KernelArgs
from kvcase import outlier_kv, poison_tail, reference_kv, rel_l2, upload, upload_cache

pytestmark = pytest.mark.gpu


def host_cache(oracle, length, kv):
    kc, vc, ks, vs = oracle.empty_cache(length + 1)
    oracle.store_mt(*kv, 0, kc, vc, ks, vs)
    poison_tail(oracle, kc, vc, ks, vs, length)
    return kc, vc, ks, vs


def decode(device, q, gate, cache, rows, history, noalloc):
    qb, gb = upload(device, q), upload(device, gate)
    out = device.allocate(q.nbytes + 4)
    out.write(np.full(rows * 4096 + 1, np.nan, np.float32))
    before = device.allocated_bytes
    device.begin()
    device.dispatch("attention_decode_int8", KernelArgs(M=rows, K=history + rows, Position=history), rows * 4096, 256,
                    qb, cache.kc, cache.vc, gb, out, cache.ks, cache.vs, noalloc=noalloc)
    device.end()
    if noalloc:
        assert device.allocated_bytes == before, "boot_dispatch_noalloc allocated device memory"
    y = out.read(np.float32, rows * 4096 + 1)
    for b in (qb, gb, out):
        b.dispose()
    assert np.isnan(y[-1])
    return y[:-1]


def prefill(device, q, gate, cache, rows, history, noalloc):
    qb, gb = upload(device, q), upload(device, gate)
    packed, out = device.allocate(rows * 8192), device.allocate(q.nbytes + 4)
    out.write(np.full(rows * 4096 + 1, np.nan, np.float32))
    p = KernelArgs(M=rows, K=history + rows, Position=history, A=8)
    before = device.allocated_bytes
    device.begin()
    device.dispatch("attention_query_grouped_half", p, rows * 1024, 128, qb, packed, noalloc=noalloc)
    device.dispatch2d("attention_online_int8_q32_k256_r2", p, (rows * 8 + 31) // 32 * 256, 2, 256, packed, cache.kc,
                      cache.vc, gb, out, cache.ks, cache.vs, noalloc=noalloc)
    device.end()
    if noalloc:
        assert device.allocated_bytes == before, "boot_dispatch_noalloc allocated device memory"
    y = out.read(np.float32, rows * 4096 + 1)
    for b in (qb, gb, packed, out):
        b.dispose()
    assert np.isnan(y[-1])
    return y[:-1]


def reader(device, q, gate, cache, rows, history, noalloc):
    """The scalar reader of a verify block (batch_attention_scores_int8, attention_softmax,
    batch_attention_values_int8), whose softmax statistics and values partials are scratch."""
    qb, gb = upload(device, q), upload(device, gate)
    length = history + rows
    scores = device.allocate(rows * 16 * length * 4)
    out = device.allocate(q.nbytes + 4)
    out.write(np.full(rows * 4096 + 1, np.nan, np.float32))
    p = KernelArgs(M=rows, K=length, Position=history)
    before = device.allocated_bytes
    device.begin()
    device.dispatch2d("batch_attention_scores_int8", p, length * 32, rows * 16, 128, qb, cache.kc, scores, cache.ks,
                      noalloc=noalloc)
    device.dispatch("attention_softmax", KernelArgs(M=rows, K=length, Position=length - 1), rows * 16 * 256, 256,
                    scores, noalloc=noalloc)
    device.dispatch("batch_attention_values_int8", p, rows * 4096, 128, scores, cache.vc, gb, out, cache.vs,
                    noalloc=noalloc)
    device.end()
    if noalloc:
        assert device.allocated_bytes == before, "boot_dispatch_noalloc allocated device memory"
    y = out.read(np.float32, rows * 4096 + 1)
    for b in (qb, gb, scores, out):
        b.dispose()
    assert np.isnan(y[-1])
    return y[:-1]


@pytest.mark.parametrize("kind,cases", [
    ("decode", [(131071, 1), (4093, 7)]),        # 114 splits per group, then 6
    ("prefill", [(30208, 512), (257, 33)]),      # 68 MB of partial slots, then a 33-row chunk (decode kernel, 3 splits)
    ("reader", [(65528, 8), (4093, 3)]),         # 16 MB of values partials and 8-row softmax statistics, then 3 rows
])
def test_noalloc_matches_dispatch(oracle, kind, cases):
    """A fresh context: every no-allocation call runs before the context has a workspace, so a
    path that fell back to (or grew) the workspace would show in boot_allocated."""
    run = {"decode": decode, "prefill": prefill, "reader": reader}[kind]
    with Device() as device:
        prepared = []
        for history, rows in cases:
            length = history + rows
            kv = outlier_kv(oracle, length, seed=70) if length > 100000 else reference_kv(length)
            host = host_cache(oracle, length, kv)
            q = oracle.fill_hash(rows * 4096, 17, 3)
            gate = oracle.fill_hash(rows * 4096, 11, 1)
            prepared.append((history, rows, host, upload_cache(device, *host), q, gate))
        got = [run(device, q, gate, cache, rows, history, noalloc=True) for history, rows, _, cache, q, gate in prepared]
        for (history, rows, host, cache, q, gate), y in zip(prepared, got):
            expected = run(device, q, gate, cache, rows, history, noalloc=False)
            assert np.array_equal(y.view(np.uint32), expected.view(np.uint32)), (kind, history, rows)
            ref = oracle.attention(q, *host, gate, rows, history, round_q_half=1 if kind == "prefill" else 0)
            assert rel_l2(y, ref) <= 1e-3 and np.abs(y - ref).max() <= 2e-3
            cache.dispose()


def test_noalloc_scratch_held_by_one_context_command(device, oracle):
    """While one context's command holds the device's scratch (after its first split-K
    no-allocation call, until its boot_end), a split-K no-allocation call of another context is
    refused on the host before any launch; after boot_end it runs and matches."""
    history, rows = 4093, 7
    host = host_cache(oracle, history + rows, reference_kv(history + rows))
    q = oracle.fill_hash(rows * 4096, 17, 3)
    gate = oracle.fill_hash(rows * 4096, 11, 1)
    cache = upload_cache(device, *host)
    qb, gb, out = upload(device, q), upload(device, gate), device.allocate(q.nbytes)
    p = KernelArgs(M=rows, K=history + rows, Position=history)
    with Device() as other:
        ocache = upload_cache(other, *host)
        oq, og, oout = upload(other, q), upload(other, gate), other.allocate(q.nbytes)
        device.begin()
        device.dispatch("attention_decode_int8", p, rows * 4096, 256, qb, cache.kc, cache.vc, gb, out, cache.ks,
                        cache.vs, noalloc=True)
        other.begin()
        with pytest.raises(HipError, match="held by another context"):
            other.dispatch("attention_decode_int8", p, rows * 4096, 256, oq, ocache.kc, ocache.vc, og, oout, ocache.ks,
                           ocache.vs, noalloc=True)
        other.end()
        device.end()
        other.begin()
        other.dispatch("attention_decode_int8", p, rows * 4096, 256, oq, ocache.kc, ocache.vc, og, oout, ocache.ks,
                       ocache.vs, noalloc=True)
        other.end()
        a, b = out.read(np.float32, rows * 4096), oout.read(np.float32, rows * 4096)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for buf in (qb, gb, out):
        buf.dispose()
    cache.dispose()


def test_noalloc_refuses_beyond_the_static_scratch(device, oracle):
    """64 decode rows at the full window need 2 x 64 x 128 split partials of 8256 bytes
    (135 MB): refused on the host with the size, before any launch; the context stays usable."""
    rows, history = 64, 262144 - 64
    k = device.allocate(262144 * 512)
    v = device.allocate(262144 * 512)
    scales = [device.allocate(262144 * 8) for _ in range(2)]
    q, gate, out = device.allocate(rows * 16384), device.allocate(rows * 16384), device.allocate(rows * 16384)
    device.begin()
    with pytest.raises(HipError, match="static scratch"):
        device.dispatch("attention_decode_int8", KernelArgs(M=rows, K=history + rows, Position=history), rows * 4096,
                        256, q, k, v, gate, out, *scales, noalloc=True)
    device.end()
    for b in (k, v, q, gate, out, *scales):
        b.dispose()
