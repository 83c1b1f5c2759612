"""FP16-KV control path (the comparator of config 3) on the GPU: batch_rope with FP16
storage (kernels.metal:322-324, flags bit 256) and the FP16 online attention
attention_online_q32_k256_s8_g8_r2 (kernels.metal:1356-1365), checked the way
OnlineAttentionTests.cs:78-97 checks it: FP64 over FP16-rounded Q/K/V, max-abs <= 5e-4,
output guard and in-place alias."""
import numpy as np
import pytest

from bootstrap_hip import DeviceAttentionWorkspace, Fp16KvLayer, append_rows_fp16, encode_online_fp16
from kvcase import rel_l2, upload

pytestmark = pytest.mark.gpu


def test_batch_rope_fp16_storage(device, oracle):
    rows, position = 7, 4093                         # KvStorageTests.cs:23-57 shape
    q = oracle.fill_hash(rows * 4096, 7, 1)
    k = oracle.fill_hash(rows * 512, 13, 1)
    v = oracle.fill_hash(rows * 512, 31, 1)
    layer = Fp16KvLayer(device, position + rows + 1)
    qb, kb, vb, qr = upload(device, q), upload(device, k), upload(device, v), device.allocate(q.nbytes)
    device.begin()
    append_rows_fp16(device, layer, qb, kb, vb, qr, rows, position)
    device.end()
    kc = layer.key.read(np.float16, (position + rows + 1) * 512)
    vc = layer.value.read(np.float16, (position + rows + 1) * 512)
    assert not kc[:position * 512].any() and not kc[(position + rows) * 512:].any()   # prefix/tail untouched
    for row in range(rows):
        for h in range(2):
            expected = oracle.rotate_vector_f64(k[(row * 2 + h) * 256:][:256], position + row)
            got = kc[((position + row) * 2 + h) * 256:][:256].astype(np.float64)
            assert np.max(np.abs(got - expected.astype(np.float32).astype(np.float16))) <= 6e-4   # KvStorageTests.cs:55
            assert np.array_equal(vc[((position + row) * 2 + h) * 256:][:256], v[(row * 2 + h) * 256:][:256].astype(np.float16))
    for b in (qb, kb, vb, qr, layer.key, layer.value):
        b.dispose()


CASES = [(0, 1), (17, 7), (127, 33), (257, 64), (4093, 7), (8192, 128), (3584, 512), (30208, 512)]
# the stress mode of OnlineAttentionTests.cs:28: Q and K x16 (logits x256, near one-hot rows)
STRESS = [(0, 1), (17, 7), (127, 33), (257, 64), (8192, 128), (3584, 512)]


@pytest.mark.parametrize("history,rows,stress", [c + (False,) for c in CASES] + [c + (True,) for c in STRESS])
def test_online_fp16_matches_fp64(device, oracle, history, rows, stress):
    length = history + rows
    k = oracle.fill_hash(length * 512, 31, 3)       # OnlineAttentionTests.cs:26-27 fills
    v = oracle.fill_hash(length * 512, 23, 1)
    q = oracle.fill_hash(rows * 4096, 17, 3)
    if stress:
        q, k = q * np.float32(16), k * np.float32(16)
    gate = oracle.fill_hash(rows * 4096, 11, 1)
    kh = np.full((length + 128) * 512, np.nan, np.float16)    # NaN padding (OnlineAttentionTests.cs:29)
    vh = np.full((length + 128) * 512, np.nan, np.float16)
    kh[:length * 512] = k.astype(np.float16)
    vh[:length * 512] = v.astype(np.float16)
    layer = Fp16KvLayer.__new__(Fp16KvLayer)
    layer.key, layer.value = upload(device, kh), upload(device, vh)
    ws = DeviceAttentionWorkspace(device)
    ws.prepare(rows)
    qb, gb = upload(device, q, extra_bytes=4), upload(device, gate)
    out = device.allocate(q.nbytes + 4)
    out.write(np.full(rows * 4096 + 1, np.nan, np.float32))
    device.begin()
    encode_online_fp16(ws, qb, layer, gb, out, rows, history)
    device.end()
    y = out.read(np.float32, rows * 4096 + 1)
    assert np.isnan(y[-1])
    y = y[:-1]
    assert np.all(np.isfinite(y))
    ref = oracle.attention_fp16kv(q, kh[:length * 512].view(np.uint16).copy(), vh[:length * 512].view(np.uint16).copy(),
                                  gate, rows, history, round_q_half=1)
    assert np.abs(y - ref).max() <= 5e-4 and rel_l2(y, ref) <= 1e-3
    device.begin()
    encode_online_fp16(ws, qb, layer, gb, qb, rows, history)      # in place over the FP32 query
    device.end()
    assert np.array_equal(qb.read(np.float32, rows * 4096).view(np.uint32), y.view(np.uint32))
    for b in (qb, gb, out, layer.key, layer.value):
        b.dispose()
    ws.dispose()
