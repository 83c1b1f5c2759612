"""INT8 online attention parity on the GPU against the FP64 oracle.

Prefill (attention_online_int8_*): the case list, inputs, guards, alias and bounds of
Int8KvTests.Attention (Int8KvTests.cs:93-181) plus the north-star bar
rel-L2 <= 1e-3 and max-abs <= 2e-3 against FP64 over the dequantized cache with FP16 Q.
Decode (attention_decode_int8 and the reference three-kernel reader): FP32 Q, same bar."""
import numpy as np
import pytest

from bootstrap_hip import KernelArgs
from kvcase import fp32_reader, outlier_kv, poison_tail, reference_kv, rel_l2, upload, upload_cache

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 1e-3, 2e-3


def build_case(oracle, history, rows, kv=None):
    length = history + rows
    k, v = kv if kv is not None else reference_kv(length)
    kc, vc, ks, vs = oracle.empty_cache(length + 1)
    oracle.store(k, v, 0, kc, vc, ks, vs)
    poison_tail(oracle, kc, vc, ks, vs, length)
    q = oracle.fill_hash(rows * 4096, 17, 3)
    gate = oracle.fill_hash(rows * 4096, 11, 1)
    return q, gate, (kc, vc, ks, vs)


def run_prefill(device, q, gate, cache, rows, history, alias=False, kernel="attention_online_int8_q32_k256_r2"):
    qb = upload(device, q, extra_bytes=4)
    gb = upload(device, gate)
    packed = device.allocate(rows * 4096 * 2)
    out = qb if alias else device.allocate(q.nbytes + 4)
    if not alias:
        out.write(np.full(rows * 4096 + 1, np.nan, np.float32))
    p = KernelArgs(M=rows, K=history + rows, Position=history, A=8)
    device.begin()
    device.dispatch("attention_query_grouped_half", p, rows * 1024, 128, qb, packed)
    device.dispatch2d(kernel, p, (rows * 8 + 31) // 32 * 256, 2, 256, packed, cache.kc, cache.vc, gb, out, cache.ks,
                      cache.vs)
    device.end()
    y = out.read(np.float32, rows * 4096 + 1)
    for b in {id(x): x for x in (qb, gb, packed, out)}.values():
        b.dispose()
    return y


# (30208, 512): config 3's final chunk at full size; (262080, 64): a block ending exactly at the
# 262144-token window (ContextLimits.cs:5); (0, 33), (8192, 2048), (27900, 2048): the shapes the
# reference times its INT8 online kernel at (docs/INT8_30K_PREFILL_20261104.md:59-61), 2048 rows
# being the chunk its tuned preset dispatches (Program.cs:71, Prefill.cs:111-121)
# (9000, 500) and (5000, 100): split chunks whose last 256-row tile is partial, with a row tile's
# splits on one XCD (the combine's blocks skip the rows past the chunk); (4093, 7) and (262080, 64)
# take the other two block placements
PREFILL_CASES = [(0, 1), (17, 7), (127, 31), (127, 32), (257, 33), (4093, 7), (8192, 128), (0, 512), (3584, 512),
                 (30000, 33), (30208, 512), (262080, 64), (0, 33), (8192, 2048), (27900, 2048), (9000, 500), (5000, 100)]


# A seeded sweep of chunk shapes: rows across 256-row tile edges (1 to 511 rows: one to eight
# row tiles, full and partial) at histories up to 12000, so that split counts from 1 to 64 and
# each of the three block placements (a row tile's splits on one XCD, a key range's blocks on one
# XCD, plain order) meet partial tiles and ragged last splits.
SWEEP_ROWS = [1, 7, 31, 32, 33, 64, 97, 128, 129, 200, 255, 256, 300, 384, 511]
SWEEP_CASES = [(int(h), r) for h, r in zip(np.random.default_rng(2026).integers(0, 12000, len(SWEEP_ROWS)), SWEEP_ROWS)]


@pytest.mark.parametrize("history,rows", SWEEP_CASES)
def test_prefill_shape_sweep(device, oracle, history, rows):
    q, gate, host = build_case(oracle, history, rows)
    cache = upload_cache(device, *host)
    y = run_prefill(device, q, gate, cache, rows, history)
    assert np.isnan(y[-1]), "output guard overwritten"
    y = y[:-1]
    ref, bound = oracle.attention(q, *host, gate, rows, history, round_q_half=1, with_bound=True)
    err = np.abs(y - ref)
    assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (rel_l2(y, ref), err.max())
    assert np.all(err <= bound / 256 + 1e-4)
    cache.dispose()


@pytest.mark.parametrize("history,rows", PREFILL_CASES)
def test_prefill_matches_fp64(device, oracle, history, rows):
    q, gate, host = build_case(oracle, history, rows)
    cache = upload_cache(device, *host)
    y = run_prefill(device, q, gate, cache, rows, history)
    assert np.isnan(y[-1]), "output guard overwritten"                          # Int8KvTests.cs:127
    y = y[:-1]
    assert np.all(np.isfinite(y)), "nonfinite INT8 attention"                  # Int8KvTests.cs:126
    ref, bound = oracle.attention(q, *host, gate, rows, history, round_q_half=1, with_bound=True)
    err = np.abs(y - ref)
    assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (rel_l2(y, ref), err.max())
    # BF16 probability rounding bound of the reference (Int8KvTests.cs:154-156)
    assert np.all(err <= bound / 256 + 1e-4)
    # in-place: output aliases the FP32 query buffer (Int8KvTests.cs:128-129)
    y2 = run_prefill(device, q, gate, cache, rows, history, alias=True)[:-1]
    assert np.array_equal(y2.view(np.uint32), y.view(np.uint32))
    cache.dispose()


@pytest.mark.parametrize("history,rows", [(0, 1), (17, 7), (127, 33), (257, 64), (8192, 128), (3584, 512)])
def test_prefill_stress_x16(device, oracle, history, rows):
    """The stress mode of OnlineAttentionTests.cs:28 on the INT8 cache: Q and K x16 (K's codes
    are unchanged, its scales x16), logits x256 and near one-hot rows, which rebase often."""
    k, v = reference_kv(history + rows)
    q, gate, host = build_case(oracle, history, rows, kv=(k * np.float32(16), v))
    q = q * np.float32(16)
    cache = upload_cache(device, *host)
    y = run_prefill(device, q, gate, cache, rows, history)
    assert np.isnan(y[-1])
    y = y[:-1]
    assert np.all(np.isfinite(y))
    ref, bound = oracle.attention(q, *host, gate, rows, history, round_q_half=1, with_bound=True)
    err = np.abs(y - ref)
    assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (rel_l2(y, ref), err.max())
    assert np.all(err <= bound / 256 + 1e-4)
    cache.dispose()


@pytest.mark.parametrize("slope", [0.05, 0.6])
def test_prefill_rising_scores(device, oracle, slope):
    """Scores that rise along the keys by about `slope` (natural log) per token: the online
    softmax meets a new maximum tile after tile, so its running maximum is rebased and the
    accumulator rescaled many times within one split (every 15 / (slope log2 e) tokens)."""
    history, rows = 3584, 512
    length = history + rows
    q = (np.abs(oracle.fill_hash(rows * 4096, 17, 3)) + np.float32(0.25)).astype(np.float32)
    k, v = reference_kv(length)
    per_token = slope * 16.0 / float(q.reshape(-1, 256).sum(1).mean())
    k = np.ascontiguousarray(k / 3 + (per_token * np.arange(length, dtype=np.float32))[:, None, None])
    kc, vc, ks, vs = oracle.empty_cache(length + 1)
    oracle.store(k, v, 0, kc, vc, ks, vs)
    poison_tail(oracle, kc, vc, ks, vs, length)
    gate = oracle.fill_hash(rows * 4096, 11, 1)
    cache = upload_cache(device, kc, vc, ks, vs)
    y = run_prefill(device, q, gate, cache, rows, history)[:-1]
    assert np.all(np.isfinite(y))
    ref = oracle.attention(q, kc, vc, ks, vs, gate, rows, history, round_q_half=1)
    assert rel_l2(y, ref) <= REL_L2 and np.abs(y - ref).max() <= MAX_ABS, (rel_l2(y, ref), np.abs(y - ref).max())
    cache.dispose()


def test_prefill_score_spikes(device, oracle):
    """Single keys whose scores jump far (tens of log2 units) above all earlier keys, at
    tile offsets that fall on both halves of the key tile; each spike outgrows the last."""
    history, rows = 3584, 64
    length = history + rows
    q = (np.abs(oracle.fill_hash(rows * 4096, 17, 3)) + np.float32(0.25)).astype(np.float32)
    k, v = reference_kv(length)
    k = k / 3
    for j, token in enumerate((45, 77, 1000, 2059, 3000, 3600, 3620, 3631)):
        k[token] += np.float32(1.0 + 0.5 * j)
    kc, vc, ks, vs = oracle.empty_cache(length + 1)
    oracle.store(np.ascontiguousarray(k), v, 0, kc, vc, ks, vs)
    poison_tail(oracle, kc, vc, ks, vs, length)
    gate = oracle.fill_hash(rows * 4096, 11, 1)
    cache = upload_cache(device, kc, vc, ks, vs)
    y = run_prefill(device, q, gate, cache, rows, history)[:-1]
    assert np.all(np.isfinite(y))
    ref = oracle.attention(q, kc, vc, ks, vs, gate, rows, history, round_q_half=1)
    assert rel_l2(y, ref) <= REL_L2 and np.abs(y - ref).max() <= MAX_ABS, (rel_l2(y, ref), np.abs(y - ref).max())
    cache.dispose()


def test_prefill_kernel_aliases_agree(device, oracle):
    """The r2, r1 and K128 names of the reference are serviced by the same gfx950 kernel."""
    q, gate, host = build_case(oracle, 257, 33)
    cache = upload_cache(device, *host)
    outs = [run_prefill(device, q, gate, cache, 33, 257, kernel=name)
            for name in ("attention_online_int8_q32_k256_r2", "attention_online_int8", "attention_online_int8_q32_k128")]
    assert all(np.array_equal(outs[0][:-1].view(np.uint32), o[:-1].view(np.uint32)) for o in outs[1:])
    cache.dispose()


def test_prefill_small_value_scale(device, oracle):
    """V scales x 1e-6 scale the output by 1e-6 within 0.8% (Int8KvTests.cs:171-181)."""
    q, gate, host = build_case(oracle, 0, 1)
    cache = upload_cache(device, *host)
    y = run_prefill(device, q, gate, cache, 1, 0)[:-1]
    kc, vc, ks, vs = host
    small = vs.copy()
    small[:2] *= np.float32(1e-6)
    cache.vs.write(small)
    y_small = run_prefill(device, q, gate, cache, 1, 0)[:-1]
    magnitude = np.abs(y).max()
    assert np.all(np.abs(y_small / 1e-6 - y) < magnitude * 0.008 + 1e-6)
    cache.dispose()


def test_config2_chunked_prefill(device, oracle):
    """Config 2: 4096-token causal prompt in 8 chunks of 512 with outlier K channels; the cache
    is appended on the GPU chunk by chunk and every chunk is checked against FP64 (gate N(0,1))."""
    total, chunk = 4096, 512
    k, v = outlier_kv(oracle, total, seed=20)
    q_all = oracle.normal(total * 4096, 22)
    gate_all = oracle.normal(total * 4096, 23)
    kc, vc, ks, vs = oracle.empty_cache(total)
    cache = upload_cache(device, kc, vc, ks, vs)
    worst_rel, worst_abs = 0.0, 0.0
    for c in range(total // chunk):
        pos = c * chunk
        kb, vb = upload(device, k[pos:pos + chunk]), upload(device, v[pos:pos + chunk])
        device.begin()
        device.dispatch("kv_store_int8", KernelArgs(M=chunk, Position=pos), chunk * 512, 256, kb, vb, cache.kc,
                        cache.vc, cache.ks, cache.vs)
        device.end()
        kb.dispose()
        vb.dispose()
        q = q_all[pos * 4096:(pos + chunk) * 4096]
        gate = gate_all[pos * 4096:(pos + chunk) * 4096]
        y = run_prefill(device, q, gate, cache, chunk, pos)[:-1]
        oracle.store(k[pos:pos + chunk], v[pos:pos + chunk], pos, kc, vc, ks, vs)
        ref = oracle.attention(q, kc, vc, ks, vs, gate, chunk, pos, round_q_half=1)
        worst_rel = max(worst_rel, rel_l2(y, ref))
        worst_abs = max(worst_abs, float(np.abs(y - ref).max()))
        # the GPU-appended cache is byte-identical to the oracle's
        assert cache.kc.read(np.int8, (pos + chunk) * 512).tobytes() == kc[:(pos + chunk) * 512].tobytes()
        assert cache.vs.read(np.float32, (pos + chunk) * 2).tobytes() == vs[:(pos + chunk) * 2].tobytes()
    assert worst_rel <= REL_L2 and worst_abs <= MAX_ABS, (worst_rel, worst_abs)
    cache.dispose()


# ------------------------------------------------------------------------------- decode

def run_decode(device, q, gate, cache, rows, history, path="fused", length_cap=None):
    qb, gb = upload(device, q), upload(device, gate)
    out = device.allocate(q.nbytes + 4)
    out.write(np.full(rows * 4096 + 1, np.nan, np.float32))
    length = history + rows
    device.begin()
    if path == "fused":
        device.dispatch("attention_decode_int8", KernelArgs(M=rows, K=length, Position=history), rows * 4096, 256,
                        qb, cache.kc, cache.vc, gb, out, cache.ks, cache.vs)
    else:
        scores = device.allocate(rows * 16 * length * 4)
        p = KernelArgs(M=rows, K=length, Position=history)
        device.dispatch2d("batch_attention_scores_int8", p, length * 32, rows * 16, 128, qb, cache.kc, scores,
                          cache.ks)
        device.dispatch("attention_softmax", KernelArgs(M=rows, K=length, Position=length - 1), rows * 16 * 256, 256,
                        scores)
        device.dispatch("batch_attention_values_int8", p, rows * 4096, 128, scores, cache.vc, gb, out, cache.vs)
    device.end()
    y = out.read(np.float32, rows * 4096 + 1)
    for b in (qb, gb, out):
        b.dispose()
    if path != "fused":
        scores.dispose()
    return y


# (7423, 2): on 256 CUs, 59 one-chunk splits; row 0 (7424 tokens, 58 chunks) ends on a split
# boundary, so its last split is empty while row 1's holds one token
DECODE_CASES = [(0, 1), (1, 1), (17, 7), (127, 1), (255, 1), (256, 1), (1000, 64), (4093, 7), (7423, 2), (8191, 1),
                (30000, 1), (65535, 2)]


@pytest.mark.parametrize("path", ["fused", "reference"])
@pytest.mark.parametrize("history,rows", DECODE_CASES)
def test_decode_matches_fp64(device, oracle, history, rows, path):
    q, gate, host = build_case(oracle, history, rows)
    cache = upload_cache(device, *host)
    y = run_decode(device, q, gate, cache, rows, history, path=path)
    assert np.isnan(y[-1])
    y = y[:-1]
    assert np.all(np.isfinite(y))
    ref = oracle.attention(q, *host, gate, rows, history, round_q_half=0)
    err = np.abs(y - ref)
    assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (rel_l2(y, ref), err.max())
    cache.dispose()


# A seeded sweep of the fused decode: 1 to 64 rows (each causal at its own position) at
# histories up to 60000, so that split counts, chunk and page edges and the rows' ragged ends vary
DECODE_SWEEP_ROWS = [1, 1, 2, 3, 5, 8, 13, 16, 31, 47, 64, 64]
DECODE_SWEEP_CASES = [(int(h), r) for h, r in
                      zip(np.random.default_rng(2027).integers(0, 60000, len(DECODE_SWEEP_ROWS)), DECODE_SWEEP_ROWS)]


@pytest.mark.parametrize("history,rows", DECODE_SWEEP_CASES)
def test_decode_shape_sweep(device, oracle, history, rows):
    q, gate, host = build_case(oracle, history, rows)
    cache = upload_cache(device, *host)
    y = run_decode(device, q, gate, cache, rows, history, path="fused")
    assert np.isnan(y[-1])
    y = y[:-1]
    ref = oracle.attention(q, *host, gate, rows, history, round_q_half=0)
    err = np.abs(y - ref)
    assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (rel_l2(y, ref), err.max())
    cache.dispose()


@pytest.mark.parametrize("path", ["prefill", "fused", "reference"])
def test_zero_value_run(device, oracle, path):
    """A run of 2048 tokens whose V vectors are all zero (scale 0, codes 0: the quantizer's rule for
    a zero vector, Int8KvTests.cs:60) covers whole key splits of the prefill, the fused decode and
    the reader, so a split's largest V scale is 0: such a split adds its keys' weight to the
    denominator and nothing to the output."""
    history, rows = 8192, 33
    k, v = reference_kv(history + rows)
    v[1024:3072] = 0
    q, gate, host = build_case(oracle, history, rows, kv=(k, v))
    assert not host[3][1024 * 2:3072 * 2].any()
    cache = upload_cache(device, *host)
    if path == "prefill":
        y = run_prefill(device, q, gate, cache, rows, history)
        ref, bound = oracle.attention(q, *host, gate, rows, history, round_q_half=1, with_bound=True)
    else:
        y = run_decode(device, q, gate, cache, rows, history, path=path)
        ref, bound = oracle.attention(q, *host, gate, rows, history, round_q_half=0, with_bound=True)
    assert np.isnan(y[-1])
    y = y[:-1]
    assert np.all(np.isfinite(y))
    err = np.abs(y - ref)
    assert rel_l2(y, ref) <= REL_L2 and err.max() <= MAX_ABS, (rel_l2(y, ref), err.max())
    assert np.all(err <= bound / 256 + 1e-4)
    cache.dispose()


@pytest.mark.parametrize("history,rows,spikes", [
    # a 131072-token context: 1152-token splits of nine 128-token chunks, spikes in later
    # chunks of the first split, mid-context and at the end
    (131071, 1, (5, 200, 300, 700, 1000, 1151, 60000, 60130, 131000, 131071)),
    # several rows, spikes inside the block's own causal ends
    (4093, 7, (5, 200, 1000, 4094, 4096, 4099)),
])
def test_decode_score_spikes(device, oracle, history, rows, spikes):
    """Single keys whose scores jump far (tens of log2 units) above every earlier key, each
    outgrowing the last: a work-group's shared running maximum must rebase between chunks."""
    length = history + rows
    q = (np.abs(oracle.fill_hash(rows * 4096, 17, 3)) + np.float32(0.25)).astype(np.float32)
    k, v = reference_kv(length)
    k = k / 3
    for j, token in enumerate(spikes):
        k[token] += np.float32(1.0 + 0.5 * j)
    kc, vc, ks, vs = oracle.empty_cache(length + 1)
    oracle.store(np.ascontiguousarray(k), v, 0, kc, vc, ks, vs)
    poison_tail(oracle, kc, vc, ks, vs, length)
    gate = oracle.fill_hash(rows * 4096, 11, 1)
    cache = upload_cache(device, kc, vc, ks, vs)
    y = run_decode(device, q, gate, cache, rows, history)[:-1]
    assert np.all(np.isfinite(y))
    ref = oracle.attention(q, kc, vc, ks, vs, gate, rows, history, round_q_half=0)
    assert rel_l2(y, ref) <= REL_L2 and np.abs(y - ref).max() <= MAX_ABS, (rel_l2(y, ref), np.abs(y - ref).max())
    cache.dispose()


def test_decode_fused_vs_reference_reader(device, oracle):
    """The fused decode and the engine's scalar reader agree (Int8KvTests.cs:159-170 bound)."""
    history, rows = 4093, 7
    q, gate, host = build_case(oracle, history, rows)
    cache = upload_cache(device, *host)
    a = run_decode(device, q, gate, cache, rows, history, path="fused")[:-1]
    b = run_decode(device, q, gate, cache, rows, history, path="reference")[:-1]
    assert np.max(np.abs(a - b)) < 4.1e-3
    cache.dispose()


def test_decode_long_context_outliers(device, oracle):
    """Decode at 131072 context over N(0,1) + outlier K channels (config 4 distribution)."""
    length = 131072
    k, v = outlier_kv(oracle, length, seed=40)
    kc, vc, ks, vs = oracle.empty_cache(length)
    oracle.store(k, v, 0, kc, vc, ks, vs)
    cache = upload_cache(device, kc, vc, ks, vs)
    q = oracle.normal(4096, 41)
    gate = oracle.normal(4096, 42)
    y = run_decode(device, q, gate, cache, 1, length - 1)[:-1]
    ref = oracle.attention(q, kc, vc, ks, vs, gate, 1, length - 1, round_q_half=0)
    assert rel_l2(y, ref) <= REL_L2 and np.abs(y - ref).max() <= MAX_ABS
    cache.dispose()


@pytest.mark.parametrize("history,rows,q_outlier", [(4093, 7, 20.0), (131071, 1, 20.0), (131071, 1, 100.0)])
def test_decode_query_outliers_match_fp32_reader(device, oracle, history, rows, q_outlier):
    """Outlier channels in Q as well as K (dims {30,31,62,63} x20 in both, and x100 in Q): one
    large query dimension sets the split query's scale for its head. The fused decode, whose
    scores use the three-part INT8 query, stays as close to FP64 as the reference's scalar reader
    evaluated in float32 (kernels.metal:147-166, on the CPU: fp32_reader): its error is at most
    1.5x that reader's + 1e-6. The GPU reader (whose scores use the same exact integer split)
    meets the same bound, and both meet the bar."""
    length = history + rows
    k, v = outlier_kv(oracle, length, seed=40)
    kc, vc, ks, vs = oracle.empty_cache(length + 1)
    oracle.store(k, v, 0, kc, vc, ks, vs)
    poison_tail(oracle, kc, vc, ks, vs, length)
    q = oracle.normal(rows * 4096, 41).reshape(rows, 16, 256)
    q[:, :, [30, 31, 62, 63]] *= np.float32(q_outlier)
    q = np.ascontiguousarray(q.ravel())
    gate = oracle.normal(rows * 4096, 42)
    cache = upload_cache(device, kc, vc, ks, vs)
    fused = run_decode(device, q, gate, cache, rows, history, path="fused")
    reader = run_decode(device, q, gate, cache, rows, history, path="reference")
    assert np.isnan(fused[-1]) and np.isnan(reader[-1])
    fused, reader = fused[:-1], reader[:-1]
    ref = oracle.attention(q, kc, vc, ks, vs, gate, rows, history, round_q_half=0)
    e_fused, e_reader = rel_l2(fused, ref), rel_l2(reader, ref)
    e_fp32 = rel_l2(fp32_reader(q, kc, vc, ks, vs, gate, rows, history), ref)
    print(f"decode q-outliers x{q_outlier} ({history},{rows}): fused rel-L2 {e_fused:.3e}, GPU reader "
          f"{e_reader:.3e}, float32 reader {e_fp32:.3e}")
    assert e_fused <= 1.5 * e_fp32 + 1e-6, (e_fused, e_fp32)
    assert e_reader <= 1.5 * e_fp32 + 1e-6, (e_reader, e_fp32)
    assert e_reader <= REL_L2 and np.abs(reader - ref).max() <= MAX_ABS
    assert np.abs(fused - ref).max() <= MAX_ABS
    cache.dispose()
