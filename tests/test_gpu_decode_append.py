"""attention_decode_append_int8: one decode step (QwenEngine.cs:161-165: batch_rope_int8 with
M = 1, then attention over keys 0..pos) in one dispatch. Against the two-dispatch sequence
batch_rope_int8 -> attention_decode_int8 on identical inputs: the rotated query, every cache
byte and the output are bitwise equal, and the output meets the FP64 bar. The appended
position holds poisoned bytes beforehand (codes -128, NaN scales, Int8KvTests.cs:121-122), which
the fused step must not read."""
import numpy as np
import pytest

from bootstrap_hip import engine
from kvcase import outlier_kv, poison_tail, rel_l2, upload

pytestmark = pytest.mark.gpu


def layer_from(device, host):
    layer = engine.Int8KvLayer.__new__(engine.Int8KvLayer)
    layer.key, layer.value, layer.key_scale, layer.value_scale = [upload(device, a) for a in host]
    return layer


# chunk (128), page (256) and split edges: small contexts split every 128 tokens, the
# 131072-token one every 1152 (9 chunks); 262143 is the window's last position. 130181 and
# 130309 fall in 8-chunk splits at token 5 of the split's chunk 1 and chunk 2, whose registers
# are loaded before the key loop and patched there
# plus a seeded draw of eight positions up to 200000 (the new token anywhere in its split)
SWEEP = [int(x) for x in np.random.default_rng(2028).integers(1, 200000, 8)]


@pytest.mark.parametrize("pos", [0, 1, 127, 128, 255, 256, 1151, 1152, 4093, 130181, 130309, 131071, 131072, 262143]
                         + SWEEP)
def test_decode_append_equals_two_dispatches(device, oracle, pos):
    capacity = pos + 1
    k, v = outlier_kv(oracle, pos, seed=80) if pos else (np.zeros((0, 2, 256), np.float32),) * 2
    kc, vc, ks, vs = oracle.empty_cache(capacity)
    if pos:
        oracle.store_mt(k, v, 0, kc, vc, ks, vs)
    poison_tail(oracle, kc, vc, ks, vs, pos)
    host = (kc, vc, ks, vs)
    q = oracle.normal(4096, 81)
    knew = oracle.normal(512, 82).reshape(2, 256)
    knew[:, [30, 31, 62, 63]] *= 20
    vnew = oracle.normal(512, 83)
    gate = oracle.normal(4096, 84)
    qb, kb, vb, gb = (upload(device, a) for a in (q, knew, vnew, gate))
    a_layer, b_layer = layer_from(device, host), layer_from(device, host)
    a_rot, b_rot = device.allocate(16384), device.allocate(16384)
    a_out, b_out = device.allocate(16384), device.allocate(16384)
    device.begin()
    engine.append_rows(device, a_layer, qb, kb, vb, a_rot, 1, pos)
    engine.decode(device, a_layer, a_rot, gb, a_out, pos)
    engine.decode_append(device, b_layer, qb, kb, vb, b_rot, gb, b_out, pos)
    device.end()
    assert a_rot.read(np.uint32, 4096).tobytes() == b_rot.read(np.uint32, 4096).tobytes(), "rotated query"
    for name, a, b, h in zip(("K codes", "V pages", "K scales", "V scales"), a_layer.buffers(), b_layer.buffers(), host):
        assert a.read(np.uint8, h.nbytes).tobytes() == b.read(np.uint8, h.nbytes).tobytes(), name
    ya, yb = a_out.read(np.float32, 4096), b_out.read(np.float32, 4096)
    assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), "output"
    cache = [buf.read(h.dtype, h.size) for buf, h in zip(b_layer.buffers(), host)]
    ref = oracle.attention(b_rot.read(np.float32, 4096), *cache, gate, 1, pos, round_q_half=0)
    assert rel_l2(yb, ref) <= 1e-3 and np.abs(yb - ref).max() <= 2e-3
    for buf in (qb, kb, vb, gb, a_rot, b_rot, a_out, b_out, *a_layer.buffers(), *b_layer.buffers()):
        buf.dispose()
