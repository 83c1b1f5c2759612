"""Speculative verification over the INT8 cache, KV part of VerificationSelfTest
(Verification.cs:105-139): a verify block of `width` candidate rows appended at the prompt end
and read by the scalar reader (Prefill.cs:269-285), then committed at `retained` rows
(rollback = move the position back; the rejected KV stays in place, Verification.cs:5-8), must
leave the same KV state and row outputs as verifying only the `retained` rows, and an unrelated
continuation token must overwrite the rejected slot without reading anything stale."""
import numpy as np
import pytest

from bootstrap_hip import Int8KvCache, engine
from kvcase import upload

pytestmark = pytest.mark.gpu

LAYERS = 2


class Stream:
    """Per-layer FP32 rows of one synthetic request: prompt, 8 candidates, one continuation."""

    def __init__(self, device, prompt, seed):
        rng = np.random.default_rng(seed)

        def rows(n):
            q = rng.standard_normal((n, 4096), dtype=np.float32)
            k = rng.standard_normal((n, 512), dtype=np.float32)
            v = rng.standard_normal((n, 512), dtype=np.float32)
            k[:, [30, 31, 286, 287]] *= 20                       # outlier K channels
            g = rng.standard_normal((n, 4096), dtype=np.float32)
            return [upload(device, a) for a in (q, k, v, g)]

        self.prompt = [rows(prompt) for _ in range(LAYERS)]
        self.candidates = [rows(8) for _ in range(LAYERS)]
        self.continuation = [rows(1) for _ in range(LAYERS)]
        self.rotated = [device.allocate(prompt * 4096 * 4) for _ in range(LAYERS)]
        self.verify = [device.allocate(8 * 4096 * 4) for _ in range(LAYERS)]
        self.step = [device.allocate(4096 * 4) for _ in range(LAYERS)]
        self.out_reader = [device.allocate(4096 * 4) for _ in range(LAYERS)]
        self.out_fused = [device.allocate(4096 * 4) for _ in range(LAYERS)]

    def dispose(self):
        for group in (self.prompt, self.candidates, self.continuation):
            for bufs in group:
                for b in bufs:
                    b.dispose()
        for group in (self.rotated, self.verify, self.step, self.out_reader, self.out_fused):
            for b in group:
                b.dispose()


def run(device, cache, s, scores, prompt, verified, retained, workspace=engine.ATTENTION_WORKSPACE_FLOATS):
    """Reset, prefill the prompt, verify `verified` candidates, commit `retained`, continue once."""
    cache.reset()
    cache.ensure_capacity(prompt)
    device.begin()
    for l, layer in enumerate(cache.layers):
        q, k, v, _ = s.prompt[l]
        engine.append_rows(device, layer, q, k, v, s.rotated[l], prompt, 0)
    device.end()
    cache.position = prompt
    cache.ensure_capacity(prompt + verified)
    device.begin()
    for l, layer in enumerate(cache.layers):
        q, k, v, g = s.candidates[l]
        engine.append_rows(device, layer, q, k, v, s.verify[l], verified, prompt)
        engine.verify_attention_int8(device, layer, s.verify[l], g, scores, verified, prompt, workspace)
    device.end()
    cache.position = prompt + verified
    rows = [s.verify[l].read(np.float32, verified * 4096).reshape(verified, 4096) for l in range(LAYERS)]
    cache.restore_prefix(prompt + retained)
    committed = cache.state_hash()
    at = prompt + retained
    cache.ensure_capacity(at + 1)
    device.begin()
    for l, layer in enumerate(cache.layers):
        q, k, v, g = s.continuation[l]
        engine.append_rows(device, layer, q, k, v, s.step[l], 1, at)
        engine.decode(device, layer, s.step[l], g, s.out_fused[l], at)
        engine.decode_reference_path(device, layer, s.step[l], g, s.out_reader[l], scores, at)
    device.end()
    cache.position = at + 1
    continued = cache.state_hash()
    reader = [s.out_reader[l].read(np.float32, 4096) for l in range(LAYERS)]
    fused = [s.out_fused[l].read(np.float32, 4096) for l in range(LAYERS)]
    return rows, committed, continued, reader, fused


@pytest.mark.parametrize("prompt", [250, 4092])
def test_verify_rollback_matches_accepted_prefix(device, prompt):
    """Every (width, retained) of Verification.cs:113-114. prompt 250 puts the block across the
    256-token V page boundary; 4092 grows the cache from 4096 to 8192 inside the verify step."""
    s = Stream(device, prompt, seed=prompt)
    cache = Int8KvCache(device, context_window=16384, layers=LAYERS)
    scores = device.allocate(8 * 16 * (prompt + 9) * 4)
    checks = 0
    for width in (1, 2, 4, 8):
        for retained in range(1, width + 1):
            rows_a, committed_a, continued_a, reader_a, fused_a = run(device, cache, s, scores, prompt, width, retained)
            rows_b, committed_b, continued_b, reader_b, fused_b = run(device, cache, s, scores, prompt, retained,
                                                                      retained)
            case = f"prompt={prompt} width={width} retained={retained}"
            for l in range(LAYERS):
                assert np.array_equal(rows_a[l][:retained], rows_b[l]), f"verifier rows differ: {case} layer={l}"
                assert np.isfinite(rows_a[l]).all() and np.abs(rows_a[l]).max() > 1e-3, case
                assert np.array_equal(reader_a[l], reader_b[l]), f"rejected KV contaminated the reader: {case}"
                assert np.array_equal(fused_a[l], fused_b[l]), f"rejected KV contaminated the decode: {case}"
            assert committed_a == committed_b, f"accepted-prefix state mismatch: {case}"
            assert continued_a == continued_b, f"continuation state mismatch: {case}"
            checks += 3
    assert checks == 3 * 15                                      # 1 + 2 + 4 + 8 (width, retained) cases
    # the fused decode and the scalar reader agree on the continuation (Int8KvTests.cs:169 bound)
    for l in range(LAYERS):
        assert np.max(np.abs(fused_a[l] - reader_a[l])) < 4.1e-3
    scores.dispose()
    s.dispose()


def test_verify_slices_agree_with_one_slice(device):
    """A score workspace too small for the whole block splits it into query slices
    (Prefill.cs:273-276); each slice keeps its absolute position, so the rows are bitwise those
    of one slice."""
    prompt = 777
    s = Stream(device, prompt, seed=9)
    cache = Int8KvCache(device, context_window=4096, layers=LAYERS)
    scores = device.allocate(8 * 16 * (prompt + 9) * 4)
    whole = run(device, cache, s, scores, prompt, 8, 8)[0]
    small = 3 * 16 * (prompt + 8)                                # three rows per slice: 3 + 3 + 2
    assert engine.verify_slices(8, prompt, small) == [(0, 3), (3, 3), (6, 2)]
    sliced = run(device, cache, s, scores, prompt, 8, 8, workspace=small)[0]
    for l in range(LAYERS):
        assert np.array_equal(whole[l], sliced[l])
    scores.dispose()
    s.dispose()
