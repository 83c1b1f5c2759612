"""Parity on the workloads the bench times and the configs name, through the C ABI.

* config 3's timed chain at full size: the bench's sequence per 512-token chunk,
  attention_prepare_fused_int8 (Q/K RMS norm with w + 1, RoPE, grouped FP16 query, gate split,
  INT8 append) -> attention_online_int8_q32_k256_r2 on the prepared query (Prefill.cs:249-261).
  For chunks 0, 30 and 59 the fused preparation's packed query, gate and the chunk's cache bytes
  are bitwise equal to the unfused chain batch_split_q -> rmsnorm x2 -> batch_rope_int8 ->
  attention_query_grouped_half (the reference's own pin, Int8KvTests.cs:71-90); the finished
  cache's V codes and scales are byte-equal to the oracle's, every K vector is within the
  quantizer's half step of an FP64 norm + RoPE (FP32 angles, as kernels.metal:122-125 computes
  them); chunks 0, 30 and 59 meet the FP64 attention bar and the per-element bound of
  Int8KvTests.cs:154-156.
* prefill over heavy-tailed K/V (config 5's Student-t nu = 4): the re-append chunks at history
  200000 + 512c (c = 0, 15) and a 64-row block ending at the 262144-token window.
* decode over the same heavy-tailed data, through the fused decode and through the three-dispatch
  scalar reader (scores, softmax, values), at history 200000 (1 row) and ending at the window
  (8 rows).
* INT8 against FP16 KV storage on the same raw K/V (Int8KvTests.cs:138-150,189): the GPU
  outputs of both paths and the FP64 quantization error the reference reports
  (max_abs_quantization_vs_fp16), at config 3's last chunk and at the reference's (8192, 128).
* config 4 through the path the bench times: a cache grown as the bench grows it (4096 ->
  131072 by 8192-token fills, each growth a doubling with device copies, then pre-grown to
  262144), byte-equal to the oracle's, then 16 consecutive attention_decode_append_int8 steps
  from 131072, each against FP64 over the device's own cache bytes."""
import numpy as np
import pytest

from bootstrap_hip import Int8KvCache, KernelArgs, engine
from bootstrap_hip import DeviceAttentionWorkspace, Fp16KvLayer, encode_online_fp16
from kvcase import fp32_reader, poison_tail, reference_kv, rel_l2, upload, upload_cache

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 2e-3
OUTLIERS = [30, 31, 62, 63]
THETA = 10_000_000.0


def rope_fp32_angles_f64(x, positions):
    """Partial RoPE (kernels.metal:122-125) of x [n][heads][256] at `positions` in FP64, with the
    angle position * theta^(-2j/64) formed in FP32 from the correctly rounded FP32 frequency, as
    the reference's FP32 arithmetic forms it; cos/sin and the rotation in FP64."""
    freq = np.array([np.float32(THETA ** (-(2.0 * j) / 64.0)) for j in range(32)], np.float32)
    angle = (np.asarray(positions, np.float32)[:, None] * freq[None, :]).astype(np.float64)
    c, s = np.cos(angle)[:, None, :], np.sin(angle)[:, None, :]
    y = np.asarray(x, np.float64).copy()
    a, b = y[:, :, :32].copy(), y[:, :, 32:64].copy()
    y[:, :, :32], y[:, :, 32:64] = a * c - b * s, b * c + a * s
    return y


def rms_norm_f64(x, weight_bits):
    """RMSNorm with (bf16 w + 1), eps 1e-6 (kernels.metal:51-57, flag 1), in FP64."""
    w = (np.asarray(weight_bits, np.uint32) << 16).view(np.float32).astype(np.float64)
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6) * (w + 1)


def test_config3_bench_chain(device, oracle):
    total, chunk = 30720, 512
    k = oracle.normal(total * 512, 500).reshape(total, 2, 256)
    k[:, :, OUTLIERS] *= 20
    v = oracle.normal(total * 512, 501).reshape(total, 2, 256)
    zero_w = np.zeros(256, np.uint16)                      # bench.py's norm weights (w + 1 = 1)
    kb, vb = upload(device, k), upload(device, v)
    qwb, kwb = upload(device, zero_w), upload(device, zero_w)
    layer, ref_layer = engine.Int8KvLayer(device, total), engine.Int8KvLayer(device, total)
    ws = engine.DeviceAttentionWorkspace(device)
    ws.prepare(chunk)
    raw = device.allocate(chunk * 32768)
    gate, out = device.allocate(chunk * 16384), device.allocate(chunk * 16384 + 4)
    packed_ref, gate_ref = device.allocate(chunk * 8192), device.allocate(chunk * 16384)
    split, norm_k, rotated = device.allocate(chunk * 16384), device.allocate(chunk * 2048), device.allocate(chunk * 16384)
    dummy = device.allocate(4)
    checked = {}
    for c in range(total // chunk):
        pos = c * chunk
        raw.write(oracle.normal(chunk * 8192, 3000 + c))
        out.write(np.full(chunk * 4096 + 1, np.nan, np.float32))
        device.begin()
        # the bench's step (bench.py PrefillWorkload.step)
        engine.prepare_fused(device, layer, raw, kb.at(pos * 2048), vb.at(pos * 2048), qwb, kwb, ws.packed_query,
                             gate, chunk, pos)
        ws.encode_int8(None, layer.key, layer.value, layer.key_scale, layer.value_scale, gate, out, chunk, pos,
                       prepared_query=True)
        device.end()
        if c not in (0, 30, 59):
            continue
        p = KernelArgs(M=chunk, Position=pos, K=pos + chunk, Theta=THETA, Epsilon=1e-6, A=8)
        device.begin()
        device.dispatch("batch_split_q", p, chunk * 4096, 128, raw, split, gate_ref)
        device.dispatch("rmsnorm", KernelArgs(N=256, M=chunk * 16, Flags=1, Epsilon=1e-6), chunk * 16 * 256, 256,
                        split, qwb, split, dummy)
        device.dispatch("rmsnorm", KernelArgs(N=256, M=chunk * 2, Flags=1, Epsilon=1e-6), chunk * 2 * 256, 256,
                        kb.at(pos * 2048), kwb, norm_k, dummy)
        device.dispatch("batch_rope_int8", p, chunk * 4096, 256, split, norm_k, vb.at(pos * 2048), rotated,
                        *ref_layer.buffers())
        device.dispatch("attention_query_grouped_half", p, chunk * 1024, 128, rotated, packed_ref)
        device.end()
        assert ws.packed_query.read(np.uint8, chunk * 8192).tobytes() == packed_ref.read(np.uint8, chunk * 8192).tobytes(), c
        assert gate.read(np.uint8, chunk * 16384).tobytes() == gate_ref.read(np.uint8, chunk * 16384).tobytes(), c
        pages = (pos // 256 * 131072, 2 * 131072)           # the chunk's two V pages (both heads)
        for name, a, b, span in (("K codes", layer.key, ref_layer.key, (pos * 512, chunk * 512)),
                                 ("V pages", layer.value, ref_layer.value, pages),
                                 ("K scales", layer.key_scale, ref_layer.key_scale, (pos * 8, chunk * 8)),
                                 ("V scales", layer.value_scale, ref_layer.value_scale, (pos * 8, chunk * 8))):
            assert a.read(np.uint8, span[1], span[0]).tobytes() == b.read(np.uint8, span[1], span[0]).tobytes(), (c, name)
        y = out.read(np.float32, chunk * 4096 + 1)
        assert np.isnan(y[-1]), "output guard overwritten"
        packed = ws.packed_query.read(np.float16, chunk * 4096).reshape(2, chunk, 8, 256)
        q = np.ascontiguousarray(packed.transpose(1, 0, 2, 3).astype(np.float32).ravel())
        checked[c] = (q, gate.read(np.float32, chunk * 4096), y[:-1])
    kc = layer.key.read(np.int8, total * 512)
    vc = layer.value.read(np.int8, total * 512)
    ks = layer.key_scale.read(np.float32, total * 2)
    vs = layer.value_scale.read(np.float32, total * 2)
    # V: byte-equal to the oracle's quantizer over the raw rows
    okc, ovc, oks, ovs = oracle.empty_cache(total)
    oracle.store_mt(k, v, 0, okc, ovc, oks, ovs)
    assert vc.tobytes() == ovc.tobytes() and vs.tobytes() == ovs.tobytes(), "V codes/scales differ from the oracle"
    # K: within half a quantization step of FP64 RMS norm + RoPE (FP32 angles)
    key = rope_fp32_angles_f64(rms_norm_f64(k, zero_w).astype(np.float32), np.arange(total))
    amax = np.abs(key).max(axis=-1)
    scale = ks.reshape(total, 2).astype(np.float64)
    assert np.all(np.abs(scale * 127 - amax) <= 2e-5 * amax + 1e-30), "K scales"
    codes = kc.reshape(total, 2, 256).astype(np.float64)
    assert codes.min() >= -127
    assert np.all(np.abs(codes * scale[:, :, None] - key) <= scale[:, :, None] * 0.5 + 2e-5 * amax[:, :, None]), "K codes"
    for c, (q, g, y) in checked.items():
        pos = c * chunk
        assert np.all(np.isfinite(y))
        ref, bound = oracle.attention(q, kc, vc, ks, vs, g, chunk, pos, round_q_half=1, with_bound=True)
        err = np.abs(y - ref)
        print(f"config 3 bench chain, chunk {c}: rel-L2 {rel_l2(y, ref):.3e} max-abs {err.max():.3e}")
        assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (c, rel_l2(y, ref), err.max())
        assert np.all(err <= bound / 256 + 1e-4)
    for b in (kb, vb, qwb, kwb, raw, gate, out, packed_ref, gate_ref, split, norm_k, rotated, dummy,
              *layer.buffers(), *ref_layer.buffers()):
        b.dispose()
    ws.dispose()


def heavy_case(oracle, history, rows, seed):
    """Student-t (nu = 4) K and V over history + rows tokens (config 5's distribution), poisoned
    tail, N(0,1) query and gate."""
    length = history + rows
    k = oracle.student_t4(length * 512, seed).reshape(length, 2, 256)
    v = oracle.student_t4(length * 512, seed + 1).reshape(length, 2, 256)
    kc, vc, ks, vs = oracle.empty_cache(length + 1)
    oracle.store_mt(k, v, 0, kc, vc, ks, vs)
    poison_tail(oracle, kc, vc, ks, vs, length)
    return oracle.normal(rows * 4096, seed + 2), oracle.normal(rows * 4096, seed + 3), (kc, vc, ks, vs)


def prefill(device, q, gate, cache, rows, history):
    qb, gb = upload(device, q), upload(device, gate)
    packed, out = device.allocate(rows * 8192), device.allocate(rows * 16384 + 4)
    out.write(np.full(rows * 4096 + 1, np.nan, np.float32))
    p = KernelArgs(M=rows, K=history + rows, Position=history, A=8)
    device.begin()
    device.dispatch("attention_query_grouped_half", p, rows * 1024, 128, qb, packed)
    device.dispatch2d("attention_online_int8_q32_k256_r2", p, (rows * 8 + 31) // 32 * 256, 2, 256, packed, cache.kc,
                      cache.vc, gb, out, cache.ks, cache.vs)
    device.end()
    y = out.read(np.float32, rows * 4096 + 1)
    for b in (qb, gb, packed, out):
        b.dispose()
    assert np.isnan(y[-1]), "output guard overwritten"
    return y[:-1]


@pytest.mark.parametrize("history,rows", [(200000, 512), (200000 + 512 * 15, 512), (262080, 64)])
def test_prefill_heavy_tailed(device, oracle, history, rows):
    """V scales vary widely within a split on Student-t data, which is where this kernel's
    FP16(e * vs / vs_ref) probability operand is most exposed (the reference rounds e * vs to BF16)."""
    q, gate, host = heavy_case(oracle, history, rows, seed=600 + history % 1000)
    vs = host[3][:(history + rows) * 2]
    print(f"heavy-tailed V scales: min {vs.min():.3g} max {vs.max():.3g}")
    cache = upload_cache(device, *host)
    y = prefill(device, q, gate, cache, rows, history)
    assert np.all(np.isfinite(y))
    ref, bound = oracle.attention(q, *host, gate, rows, history, round_q_half=1, with_bound=True)
    err = np.abs(y - ref)
    print(f"heavy-tailed prefill ({history},{rows}): rel-L2 {rel_l2(y, ref):.3e} max-abs {err.max():.3e}")
    assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (rel_l2(y, ref), err.max())
    assert np.all(err <= bound / 256 + 1e-4)           # Int8KvTests.cs:154-156
    cache.dispose()


def decode(device, q, gate, cache, rows, history, path):
    qb, gb = upload(device, q), upload(device, gate)
    out = device.allocate(rows * 16384 + 4)
    out.write(np.full(rows * 4096 + 1, np.nan, np.float32))
    length = history + rows
    p = KernelArgs(M=rows, K=length, Position=history)
    scores = None
    device.begin()
    if path == "fused":
        device.dispatch("attention_decode_int8", p, rows * 4096, 256, qb, cache.kc, cache.vc, gb, out, cache.ks,
                        cache.vs)
    else:
        scores = device.allocate(rows * 16 * length * 4)
        device.dispatch2d("batch_attention_scores_int8", p, length * 32, rows * 16, 128, qb, cache.kc, scores,
                          cache.ks)
        device.dispatch("attention_softmax", KernelArgs(M=rows, K=length, Position=length - 1), rows * 16 * 256, 256,
                        scores)
        device.dispatch("batch_attention_values_int8", p, rows * 4096, 128, scores, cache.vc, gb, out, cache.vs)
    device.end()
    y = out.read(np.float32, rows * 4096 + 1)
    for b in (qb, gb, out) + ((scores,) if scores is not None else ()):
        b.dispose()
    assert np.isnan(y[-1]), "output guard overwritten"
    return y[:-1]


@pytest.mark.parametrize("history,rows", [(200000, 1), (262136, 8)])
def test_decode_heavy_tailed(device, oracle, history, rows):
    """The fused decode (p * vs / vs_ref as FP16 hi + lo) and the scalar reader over Student-t
    K/V, whose V scales vary widely within a split, against FP64 (the reference's FP32 query,
    no FP16 rounding), with the per-element bound of Int8KvTests.cs:154-156."""
    q, gate, host = heavy_case(oracle, history, rows, seed=800 + history % 1000)
    cache = upload_cache(device, *host)
    ref, bound = oracle.attention(q, *host, gate, rows, history, round_q_half=0, with_bound=True)
    errors = {}
    for path in ("fused", "reader"):
        y = decode(device, q, gate, cache, rows, history, path)
        assert np.all(np.isfinite(y))
        err = np.abs(y - ref)
        errors[path] = rel_l2(y, ref)
        print(f"heavy-tailed decode {path} ({history},{rows}): rel-L2 {rel_l2(y, ref):.3e} max-abs {err.max():.3e}")
        assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (path, rel_l2(y, ref), err.max())
        assert np.all(err <= bound / 256 + 1e-4), path
    if rows == 1:
        # a long, flat row (p ~ 1 / 200000): both GPU paths as close to FP64 as the reference's
        # reader evaluated in float32 (its probabilities then sit far below FP16's normal range)
        e_fp32 = rel_l2(fp32_reader(q, *host, gate, rows, history), ref)
        print(f"float32 reader: rel-L2 {e_fp32:.3e}")
        for path, e in errors.items():
            assert e <= 1.5 * e_fp32 + 1e-6, (path, e, e_fp32)
    cache.dispose()


@pytest.mark.parametrize("case", ["config3_last_chunk", "reference_8192_128"])
def test_int8_vs_fp16_storage(device, oracle, case):
    """INT8 (codes + FP32 scales) against FP16 storage of the same raw K/V and the same query:
    the two GPU paths' outputs and the reference's max_abs_quantization_vs_fp16 (FP64 attention
    over each cache, Int8KvTests.cs:138-150). Both outputs are finite, and the GPU paths differ
    by no more than the FP64 quantization difference plus each kernel's own bar."""
    if case == "config3_last_chunk":
        history, rows = 30208, 512
        length = history + rows
        k = oracle.normal(length * 512, 700).reshape(length, 2, 256)
        k[:, :, OUTLIERS] *= 20
        v = oracle.normal(length * 512, 701).reshape(length, 2, 256)
        q, gate = oracle.normal(rows * 4096, 702), oracle.normal(rows * 4096, 703)
    else:
        history, rows = 8192, 128
        length = history + rows
        k, v = reference_kv(length)
        q, gate = oracle.fill_hash(rows * 4096, 17, 3), oracle.fill_hash(rows * 4096, 11, 1)
    kc, vc, ks, vs = oracle.empty_cache(length)
    oracle.store_mt(k, v, 0, kc, vc, ks, vs)
    cache = upload_cache(device, kc, vc, ks, vs)
    y8 = prefill(device, q, gate, cache, rows, history)
    kh, vh = k.astype(np.float16).ravel(), v.astype(np.float16).ravel()
    layer = Fp16KvLayer.__new__(Fp16KvLayer)
    layer.key, layer.value = upload(device, kh), upload(device, vh)
    ws = DeviceAttentionWorkspace(device)
    ws.prepare(rows)
    qb, gb, out = upload(device, q), upload(device, gate), device.allocate(rows * 16384)
    device.begin()
    encode_online_fp16(ws, qb, layer, gb, out, rows, history)
    device.end()
    y16 = out.read(np.float32, rows * 4096)
    assert np.all(np.isfinite(y8)) and np.all(np.isfinite(y16))
    gpu_abs, gpu_rel = float(np.abs(y8 - y16).max()), rel_l2(y8, y16)
    ref8 = oracle.attention(q, kc, vc, ks, vs, gate, rows, history, round_q_half=1)
    ref16 = oracle.attention_fp16kv(q, kh.view(np.uint16), vh.view(np.uint16), gate, rows, history, round_q_half=1)
    quant_abs, quant_rel = float(np.abs(ref8 - ref16).max()), rel_l2(ref8, ref16)
    print(f"INT8 vs FP16 KV ({history},{rows}): GPU max-abs {gpu_abs:.5g} rel-L2 {gpu_rel:.4g}; "
          f"FP64 quantization max-abs {quant_abs:.5g} rel-L2 {quant_rel:.4g}")
    assert np.isfinite(gpu_abs) and np.isfinite(quant_abs)
    assert gpu_abs <= quant_abs + MAX_ABS + 5e-4
    for b in (qb, gb, out, layer.key, layer.value):
        b.dispose()
    ws.dispose()
    cache.dispose()


def test_config4_grown_decode_append(device, oracle):
    context, steps, fill = 131072, 16, 8192
    k = oracle.normal((context + steps) * 512, 800).reshape(context + steps, 2, 256)
    k[:, :, OUTLIERS] *= 20
    v = oracle.normal((context + steps) * 512, 801).reshape(context + steps, 2, 256)
    cache = Int8KvCache(device, context_window=engine.NATIVE_WINDOW, layers=1)
    assert cache.capacity == 4096
    kb, vb = device.allocate(fill * 2048), device.allocate(fill * 2048)
    for pos in range(0, context, fill):                      # bench.py DecodeWorkload: fills of 8192
        cache.ensure_capacity(pos + fill)
        kb.write(k[pos:pos + fill])
        vb.write(v[pos:pos + fill])
        device.begin()
        engine.store_rows(device, cache.layers[0], kb, vb, fill, pos)
        device.end()
    cache.ensure_capacity(context + 256)                     # pre-grown before the timed steps
    assert cache.growth_log == [8192, 16384, 32768, 65536, 131072, 262144]
    layer = cache.layers[0]
    kc, vc, ks, vs = oracle.empty_cache(262144)
    oracle.store_mt(k[:context], v[:context], 0, kc, vc, ks, vs)
    for name, buf, host in (("K codes", layer.key, kc), ("V pages", layer.value, vc), ("K scales", layer.key_scale, ks),
                            ("V scales", layer.value_scale, vs)):
        assert buf.length == host.nbytes, name
        assert buf.read(np.uint8, host.nbytes).tobytes() == host.view(np.uint8).tobytes(), f"grown {name}"
    q = oracle.normal(steps * 4096, 802)
    gate = oracle.normal(steps * 4096, 803)
    qb, gb = upload(device, q), upload(device, gate)
    knew, vnew = upload(device, k[context:]), upload(device, v[context:])
    rotated, out = device.allocate(steps * 16384), device.allocate(steps * 16384)
    device.begin()
    for i in range(steps):                                   # one command, as the bench issues them
        engine.decode_append(device, layer, qb.at(i * 16384), knew.at(i * 2048), vnew.at(i * 2048),
                             rotated.at(i * 16384), gb.at(i * 16384), out.at(i * 16384), context + i)
    device.end()
    dev = (layer.key.read(np.int8, kc.size), layer.value.read(np.int8, vc.size),
           layer.key_scale.read(np.float32, ks.size), layer.value_scale.read(np.float32, vs.size))
    # history untouched, appended V bit-exact, appended K within the quantizer of FP64 RoPE
    assert dev[0][:context * 512].tobytes() == kc[:context * 512].tobytes()
    assert dev[2][:context * 2].tobytes() == ks[:context * 2].tobytes()
    oracle.store_mt(k[:context + steps], v[:context + steps], 0, kc, vc, ks, vs)
    assert dev[1].tobytes() == vc.tobytes() and dev[3].tobytes() == vs.tobytes(), "V pages/scales"
    key = rope_fp32_angles_f64(k[context:], context + np.arange(steps))
    amax = np.abs(key).max(axis=-1)
    scale = dev[2][context * 2:(context + steps) * 2].reshape(steps, 2).astype(np.float64)
    codes = dev[0][context * 512:(context + steps) * 512].reshape(steps, 2, 256).astype(np.float64)
    assert np.all(np.abs(scale * 127 - amax) <= 2e-5 * amax)
    assert np.all(np.abs(codes * scale[:, :, None] - key) <= scale[:, :, None] * 0.5 + 2e-5 * amax[:, :, None])
    assert not dev[0][(context + steps) * 512:].any(), "K beyond the appended tokens"
    rq = rotated.read(np.float32, steps * 4096)
    want_q = rope_fp32_angles_f64(q.reshape(steps, 16, 256), context + np.arange(steps)).ravel()
    assert np.all(np.abs(rq - want_q) <= 2e-5 * (1 + np.abs(want_q)))
    y = out.read(np.float32, steps * 4096)
    worst = 0.0
    for i in range(steps):
        ref = oracle.attention(rq[i * 4096:(i + 1) * 4096], *dev, gate[i * 4096:(i + 1) * 4096], 1, context + i,
                               round_q_half=0)
        yi = y[i * 4096:(i + 1) * 4096]
        worst = max(worst, rel_l2(yi, ref))
        assert rel_l2(yi, ref) <= REL_L2 and np.abs(yi - ref).max() <= MAX_ABS, (i, rel_l2(yi, ref))
    print(f"config 4 decode_append, 16 steps from 131072: worst rel-L2 {worst:.3e}")
    for b in (kb, vb, qb, gb, knew, vnew, rotated, out, *layer.buffers(), cache.scores):
        b.dispose()
