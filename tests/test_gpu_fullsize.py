"""Parity at the configs' own sizes and distributions, through the C ABI.

* config 3: the 30720-token prompt in 60 chunks of 512 with outlier K channels, appended on the
  GPU chunk by chunk (kv_store_int8) with every chunk's attention run after its append; the
  device cache ends byte-identical to the oracle's, and chunks 30 and 59 meet the FP64 bar and
  the reference's per-element bound (Int8KvTests.cs:154-156).
* config 4: four sequential single-token steps at 131073.. (batch_rope_int8 append of one token,
  then attention_decode_int8 over the whole cache, QwenEngine.cs:161-165), each against FP64
  over the device's own cache bytes and rotated query, with the appended codes within the
  reference's quantization bounds (Int8KvTests.cs:54,59) and the prefix untouched."""
import hashlib

import numpy as np
import pytest

from bootstrap_hip import KernelArgs, engine
from kvcase import rel_l2, upload, upload_cache

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 2e-3
OUTLIERS = [30, 31, 62, 63]


def test_config3_chain_with_outliers(device, oracle):
    total, chunk = 30720, 512
    k = oracle.normal(total * 512, 300).reshape(total, 2, 256)
    k[:, :, OUTLIERS] *= 20
    v = oracle.normal(total * 512, 301).reshape(total, 2, 256)
    kc, vc, ks, vs = oracle.empty_cache(total)
    cache = upload_cache(device, kc, vc, ks, vs)
    oracle.store_mt(k, v, 0, kc, vc, ks, vs)                 # the expected cache bytes
    kb, vb = device.allocate(chunk * 2048), device.allocate(chunk * 2048)
    qb, gb = device.allocate(chunk * 16384 + 4), device.allocate(chunk * 16384)
    packed, out = device.allocate(chunk * 8192), device.allocate(chunk * 16384 + 4)
    checked = {}
    for c in range(total // chunk):
        pos = c * chunk
        q = oracle.normal(chunk * 4096, 1000 + c)
        gate = oracle.normal(chunk * 4096, 2000 + c)
        kb.write(k[pos:pos + chunk])
        vb.write(v[pos:pos + chunk])
        qb.write(q)
        gb.write(gate)
        out.write(np.full(chunk * 4096 + 1, np.nan, np.float32))
        p = KernelArgs(M=chunk, K=pos + chunk, Position=pos, A=8)
        device.begin()
        device.dispatch("kv_store_int8", KernelArgs(M=chunk, Position=pos), chunk * 512, 256, kb, vb, cache.kc,
                        cache.vc, cache.ks, cache.vs)
        device.dispatch("attention_query_grouped_half", p, chunk * 1024, 128, qb, packed)
        device.dispatch2d("attention_online_int8_q32_k256_r2", p, chunk * 8 * 256 // 32, 2, 256, packed, cache.kc,
                          cache.vc, gb, out, cache.ks, cache.vs)
        device.end()
        if c in (30, 59):
            y = out.read(np.float32, chunk * 4096 + 1)
            assert np.isnan(y[-1]), "output guard overwritten"
            checked[c] = (q, gate, y[:-1])
    for name, host, buf in (("K codes", kc, cache.kc), ("V pages", vc, cache.vc), ("K scales", ks, cache.ks),
                            ("V scales", vs, cache.vs)):
        assert buf.read(np.uint8, host.nbytes).tobytes() == host.view(np.uint8).tobytes(), name
    for c, (q, gate, y) in checked.items():
        pos = c * chunk
        assert np.all(np.isfinite(y))
        ref, bound = oracle.attention(q, kc, vc, ks, vs, gate, chunk, pos, round_q_half=1, with_bound=True)
        err = np.abs(y - ref)
        print(f"config 3 chunk {c}: rel-L2 {rel_l2(y, ref):.3e} max-abs {err.max():.3e}")
        assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (c, rel_l2(y, ref), err.max())
        assert np.all(err <= bound / 256 + 1e-4)
    for b in (kb, vb, qb, gb, packed, out):
        b.dispose()
    cache.dispose()


def test_config4_sequential_steps(device, oracle):
    context, steps = 131072, 4
    k = oracle.normal(context * 512, 400).reshape(context, 2, 256)
    k[:, :, OUTLIERS] *= 20
    v = oracle.normal(context * 512, 401).reshape(context, 2, 256)
    capacity = context + 8
    kc, vc, ks, vs = oracle.empty_cache(capacity)
    oracle.store_mt(k, v, 0, kc, vc, ks, vs)
    layer = engine.Int8KvLayer.__new__(engine.Int8KvLayer)
    layer.key, layer.value, layer.key_scale, layer.value_scale = [upload(device, a) for a in (kc, vc, ks, vs)]
    prefix = hashlib.sha256(kc[:context * 512].tobytes() + vc[:context * 512].tobytes()).hexdigest()
    q_all = oracle.normal(steps * 4096, 402)
    k_new = oracle.normal(steps * 512, 403).reshape(steps, 2, 256)
    k_new[:, :, OUTLIERS] *= 20
    v_new = oracle.normal(steps * 512, 404).reshape(steps, 2, 256)
    gate = oracle.normal(steps * 4096, 405)
    qb, kb, vb, gb = (upload(device, a) for a in (q_all, k_new, v_new, gate))
    rotated, out = device.allocate(steps * 16384), device.allocate(steps * 16384 + 4)
    for i in range(steps):
        pos = context + i
        device.begin()
        engine.append_rows(device, layer, qb.at(i * 16384), kb.at(i * 2048), vb.at(i * 2048), rotated.at(i * 16384), 1,
                           pos)
        engine.decode(device, layer, rotated.at(i * 16384), gb.at(i * 16384), out.at(i * 16384), pos)
        device.end()
        # the appended token: K within the reference's bounds of its FP64-rotated input, V exact
        for h in range(2):
            vector = pos * 2 + h
            codes = layer.key.read(np.int8, 256, vector * 256)
            scale = layer.key_scale.read(np.float32, 1, vector * 4)[0]
            key = oracle.rotate_vector_f64(k_new[i, h], pos)
            assert abs(scale - np.abs(key).max() / 127) < 2e-5 * max(1.0, np.abs(key).max())   # Int8KvTests.cs:54
            assert np.all(np.abs(codes * np.float64(scale) - key) <= np.abs(key).max() / 254 + 3e-3)   # :59
            kc[vector * 256:(vector + 1) * 256] = codes
            ks[vector] = scale
            cv, sv = oracle.quantize(v_new[i, h])
            got_v = np.array([layer.value.read(np.int8, 1, oracle.value_index(vector, d))[0] for d in (0, 1, 77, 255)])
            assert np.array_equal(got_v, cv[[0, 1, 77, 255]]) and layer.value_scale.read(np.float32, 1, vector * 4)[0] == sv
            for d in range(256):
                vc[oracle.value_index(vector, d)] = cv[d]
            vs[vector] = sv
        q = rotated.read(np.float32, 4096, i * 16384)
        y = out.read(np.float32, 4096, i * 16384)
        ref = oracle.attention(q, kc, vc, ks, vs, gate[i * 4096:(i + 1) * 4096], 1, pos, round_q_half=0)
        print(f"config 4 step {i} (L={pos + 1}): rel-L2 {rel_l2(y, ref):.3e} max-abs {np.abs(y - ref).max():.3e}")
        assert rel_l2(y, ref) <= REL_L2 and np.abs(y - ref).max() <= MAX_ABS, (i, rel_l2(y, ref))
    got = hashlib.sha256(layer.key.read(np.uint8, context * 512).tobytes() +
                         layer.value.read(np.uint8, context * 512).tobytes()).hexdigest()
    assert got == prefix, "the history changed under the appends"
    for b in (qb, kb, vb, gb, rotated, out, *layer.buffers()):
        b.dispose()
