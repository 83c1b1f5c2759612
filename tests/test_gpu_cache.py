"""KV store policy on the GPU: growth by doubling with device copies (QwenEngine.cs:76-99),
reset (QwenEngine.cs:122-132), prefix restore = truncate by position (PrefixCache.cs:45-77)
with the state hash of PrefixCacheSelfTest.cs:133-148, and the config-5 full-window stress."""
import numpy as np
import pytest

from bootstrap_hip import Int8KvCache, engine
from kvcase import rel_l2, upload

pytestmark = pytest.mark.gpu

WINDOW = 262144


def append(device, cache, layer_index, k, v, pos):
    kb, vb = upload(device, np.ascontiguousarray(k)), upload(device, np.ascontiguousarray(v))
    device.begin()
    engine.store_rows(device, cache.layers[layer_index], kb, vb, k.shape[0], pos)
    device.end()
    kb.dispose()
    vb.dispose()


def test_growth_preserves_prefix_and_reset_clears(device, oracle):
    cache = Int8KvCache(device, context_window=WINDOW, layers=2)
    assert cache.capacity == 4096
    k = oracle.normal(4096 * 512, 5).reshape(4096, 2, 256)
    v = oracle.normal(4096 * 512, 6).reshape(4096, 2, 256)
    for layer in range(2):
        append(device, cache, layer, k, v, 0)
    cache.position = 4096
    before = cache.state_hash()
    cache.ensure_capacity(4097)                                  # doubles, copying every byte
    assert cache.capacity == 8192 and cache.growth_log == [8192]
    assert cache.layers[0].key.length == 8192 * 512
    assert cache.layers[0].value.length == 8192 * 512
    assert cache.state_hash() == before
    # the copied cache keeps the exact codes/scales of the oracle
    kc, vc, ks, vs = oracle.empty_cache(4096)
    oracle.store(k, v, 0, kc, vc, ks, vs)
    assert cache.layers[1].key.read(np.int8, 4096 * 512).tobytes() == kc.tobytes()
    assert cache.layers[1].value_scale.read(np.float32, 8192).tobytes() == vs.tobytes()
    cache.reset()
    for layer in cache.layers:
        for buffer in layer.buffers():
            assert not buffer.read(np.uint8, buffer.length).any()
    with pytest.raises(ValueError):
        cache.ensure_capacity(WINDOW + 1)


def test_full_window_truncate_reappend_equals_fresh_build(device):
    """Config 5: 10 layers x 262144 tokens of Student-t (nu=4) K/V, grown from 4096 by doubling;
    decode at the full window; restore the prefix at 200000 (page 781 holds 64 valid slots)
    and re-append 8192 tokens in 16 chunks of 512; codes, scales and decode outputs must equal
    a fresh 208192-token build."""
    layers, cut, extra, chunk = 10, 200000, 8192, 32768
    rng = np.random.default_rng(55)
    pool_k = rng.standard_t(4, (WINDOW + extra, 2, 256)).astype(np.float32)
    pool_v = rng.standard_t(4, (WINDOW + extra, 2, 256)).astype(np.float32)

    def data(layer, start, count, new=False):
        # each layer sees its own rotation of the pool; the new tokens follow the window
        base = WINDOW if new else 0
        idx = (np.arange(start, start + count) + 977 * layer) % (WINDOW if not new else extra) + base
        return pool_k[idx], pool_v[idx]

    cache = Int8KvCache(device, context_window=WINDOW, layers=layers)
    for pos in range(0, WINDOW, chunk):
        cache.ensure_capacity(pos + chunk)
        for layer in range(layers):
            append(device, cache, layer, *data(layer, pos, chunk), pos)
    cache.position = WINDOW
    # EnsureCacheCapacity doubles until the request fits and grows the buffers once per call
    # (QwenEngine.cs:88-95): 32768-token chunks grow 4096 -> 32768 -> ... -> 262144
    assert cache.capacity == WINDOW and cache.growth_log == [32768, 65536, 131072, 262144]
    assert cache.target_kv_bytes == 2_726_297_600
    # decode at the full window on the last layer against FP64
    import sys
    sys.path.insert(0, __import__("os").path.dirname(__file__))
    from oracle_lib import Oracle
    oracle = Oracle()
    q = rng.standard_normal(4096).astype(np.float32)
    gate = rng.standard_normal(4096).astype(np.float32)
    qb, gb, out = upload(device, q), upload(device, gate), device.allocate(4096 * 4)
    layer9 = cache.layers[9]
    device.begin()
    engine.decode(device, layer9, qb, gb, out, WINDOW - 1)
    device.end()
    y = out.read(np.float32, 4096)
    kc = layer9.key.read(np.int8, WINDOW * 512)
    vc = layer9.value.read(np.int8, WINDOW * 512)
    ks = layer9.key_scale.read(np.float32, WINDOW * 2)
    vs = layer9.value_scale.read(np.float32, WINDOW * 2)
    ref = oracle.attention(q, kc, vc, ks, vs, gate, 1, WINDOW - 1, round_q_half=0)
    assert rel_l2(y, ref) <= 1e-3 and np.abs(y - ref).max() <= 2e-3
    # prefix restore: truncate by position, then re-append in 512-token chunks
    assert cache.restore_prefix(cut) == cut
    for c in range(extra // 512):
        pos = cut + 512 * c
        for layer in range(layers):
            append(device, cache, layer, *data(layer, 512 * c, 512, new=True), pos)
    cache.position = cut + extra
    fresh = Int8KvCache(device, context_window=WINDOW, layers=layers)
    fresh.ensure_capacity(cut + extra)
    for layer in range(layers):
        for pos in range(0, cut, chunk):
            n = min(chunk, cut - pos)
            append(device, fresh, layer, *data(layer, pos, n), pos)
        append(device, fresh, layer, *data(layer, 0, extra, new=True), cut)
    fresh.position = cut + extra
    assert cache.state_hash() == fresh.state_hash()
    outs = []
    for c_ in (cache, fresh):
        device.begin()
        engine.decode(device, c_.layers[9], qb, gb, out, cut + extra - 1)
        device.end()
        outs.append(out.read(np.float32, 4096))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    for b in (qb, gb, out):
        b.dispose()
    for c_ in (cache, fresh):
        for layer in c_.layers:
            for buffer in layer.buffers():
                buffer.dispose()
        c_.scores.dispose()
