"""Many dispatches in one command (boot_begin .. boot_end) give results bit-identical to
running every dispatch in a command of its own (bridge.mm:214-217: a command's dispatches
run in order): chunked prefill and multi-layer decode, whose split-K combines reuse the
context's workspace, and a dispatch that reads the attention output or overwrites the gate
right after the attention in the same command."""
import numpy as np
import pytest

from bootstrap_hip import KernelArgs, engine
from kvcase import outlier_kv, upload

pytestmark = pytest.mark.gpu


def dispose_cache(cache):
    for layer in cache.layers:
        for b in layer.buffers():
            b.dispose()
    cache.scores.dispose()


def prefill_run(device, q, k, v, gate, tokens, chunk, one_command):
    cache = engine.Int8KvCache(device, context_window=engine.NATIVE_WINDOW, layers=1)
    cache.ensure_capacity(tokens)
    layer = cache.layers[0]
    ws = engine.DeviceAttentionWorkspace(device)
    ws.prepare(chunk)
    rotated = device.allocate(tokens * 16384)
    if one_command:
        device.begin()
    for pos in range(0, tokens, chunk):
        if not one_command:
            device.begin()
        engine.append_rows(device, layer, q.at(pos * 16384), k.at(pos * 2048), v.at(pos * 2048),
                           rotated.at(pos * 16384), chunk, pos)
        ws.encode_int8(rotated.at(pos * 16384), layer.key, layer.value, layer.key_scale, layer.value_scale,
                       gate.at(pos * 16384), rotated.at(pos * 16384), chunk, pos)
        if not one_command:
            device.end()
    if one_command:
        device.end()
    out = rotated.read(np.float32, tokens * 4096)
    rotated.dispose()
    ws.dispose()
    dispose_cache(cache)
    return out


def test_prefill_chunks_in_one_command_match_serial(device, oracle):
    """Config-3-shaped: append + attention per 512-row chunk (output aliasing the rotated
    query, as Prefill.cs does); every chunk after the first splits its keys."""
    tokens, chunk = 3072, 512
    k, v = outlier_kv(oracle, tokens, seed=40)
    q = upload(device, oracle.normal(tokens * 4096, 41))
    gate = upload(device, oracle.normal(tokens * 4096, 42))
    kb, vb = upload(device, k), upload(device, v)
    together = prefill_run(device, q, kb, vb, gate, tokens, chunk, True)
    apart = prefill_run(device, q, kb, vb, gate, tokens, chunk, False)
    assert np.all(np.isfinite(together))
    assert np.array_equal(together.view(np.uint32), apart.view(np.uint32))
    for b in (q, gate, kb, vb):
        b.dispose()


def decode_setup(device, oracle, layers, context, steps):
    cache = engine.Int8KvCache(device, context_window=engine.NATIVE_WINDOW, layers=layers)
    cache.ensure_capacity(context + steps)
    k, v = outlier_kv(oracle, context + steps, seed=50)
    kb, vb = upload(device, k[:context]), upload(device, v[:context])
    device.begin()
    for layer in cache.layers:
        engine.store_rows(device, layer, kb, vb, context, 0)
    device.end()
    kb.dispose()
    vb.dispose()
    return cache, k, v


def test_decode_layers_in_one_command_match_serial(device, oracle):
    """Config-4-shaped: each token appends to and attends over every layer; every decode's
    combine reads the split workspace the next decode writes again."""
    layers, context, steps = 3, 5000, 4
    outs = []
    for one_command in (True, False):
        cache, k, v = decode_setup(device, oracle, layers, context, steps)
        q = upload(device, oracle.normal(steps * 4096, 51))
        gate = upload(device, oracle.normal(steps * 4096, 52))
        kn, vn = upload(device, np.ascontiguousarray(k[context:])), upload(device, np.ascontiguousarray(v[context:]))
        rotated = device.allocate(steps * 16384)
        out = device.allocate(steps * 16384 * layers)
        if one_command:
            device.begin()
        for i in range(steps):
            for li, layer in enumerate(cache.layers):
                if not one_command:
                    device.begin()
                engine.append_rows(device, layer, q.at(i * 16384), kn.at(i * 2048), vn.at(i * 2048),
                                   rotated.at(i * 16384), 1, context + i)
                engine.decode(device, layer, rotated.at(i * 16384), gate.at(i * 16384),
                              out.at((li * steps + i) * 16384), context + i)
                if not one_command:
                    device.end()
        if one_command:
            device.end()
        outs.append(out.read(np.float32, steps * 4096 * layers))
        for b in (q, gate, kn, vn, rotated, out):
            b.dispose()
        dispose_cache(cache)
    assert np.all(np.isfinite(outs[0]))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_tail_hazards_read_after_write_and_write_after_read(device, oracle):
    """Inside one command, right after a split decode: a dispatch reads its output y (the
    FP16 grouping of y sees the combine's result) and the gate the combine reads is
    cleared (after the combine read it)."""
    context = 5000
    cache, k, v = decode_setup(device, oracle, 1, context, 1)
    layer = cache.layers[0]
    q = upload(device, oracle.normal(4096, 61))
    g_host = oracle.normal(4096, 62)
    gate = upload(device, g_host)
    kn, vn = upload(device, np.ascontiguousarray(k[context:])), upload(device, np.ascontiguousarray(v[context:]))
    rotated, out = device.allocate(16384), device.allocate(16384)
    packed = device.allocate(8192)

    # reference: decode alone in its command, then the grouping in another
    device.begin()
    engine.append_rows(device, layer, q, kn, vn, rotated, 1, context)
    engine.decode(device, layer, rotated, gate, out, context)
    device.end()
    ref = out.read(np.float32, 4096)

    # same decode (the appended token is rewritten with the same bytes) followed in the same
    # command by a read of y and a clear of the gate
    out.write(np.zeros(4096, np.float32))
    device.begin()
    engine.append_rows(device, layer, q, kn, vn, rotated, 1, context)
    engine.decode(device, layer, rotated, gate, out, context)
    device.dispatch("attention_query_grouped_half", KernelArgs(M=1, A=8), 1024, 128, out, packed)
    device.clear(gate)
    device.end()
    got = out.read(np.float32, 4096)
    grouped = packed.read(np.float16, 4096)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(grouped.view(np.uint16), ref.astype(np.float16).view(np.uint16))
    assert not np.any(gate.read(np.float32, 4096))
    for b in (q, gate, kn, vn, rotated, out, packed):
        b.dispose()
    dispose_cache(cache)
