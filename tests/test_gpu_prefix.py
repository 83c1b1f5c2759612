"""Prefix-cache hits over the device store, KV part of PrefixCacheSelfTest.Run
(PrefixCacheSelfTest.cs:22-75): every warm request, resumed from a checkpoint of the single KV
lineage, must leave the same KV bytes (state hash) and the same attention outputs, bitwise, as a
cold build of the same prompt. The rows a token contributes (Q, K, V, gate) are drawn from a hash
of the whole token prefix up to it, as a model's would depend on it, so a branch changes every
row after the point where the prompts part."""
import numpy as np
import pytest

from bootstrap_hip import DeviceAttentionWorkspace, Int8KvCache, PrefixLineage, engine
from lineage_case import END, END_OF_TEXT, conversation, run_prompt, simple_chat, words

pytestmark = pytest.mark.gpu

MASK = (1 << 64) - 1
GENERATED = 3


def mix(h, token):
    """splitmix64 step over (h, token)."""
    z = (h + 0x9E3779B97F4A7C15 + token * 0xBF58476D1CE4E5B9) & MASK
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
    return z ^ (z >> 31)


class Request:
    """Drives one lineage: ``run(prompt)`` restores, prefills the rest chunk by chunk (INT8
    append + online attention) and decodes GENERATED tokens, keeping the last outputs."""

    def __init__(self, device, enabled=True):
        self.device = device
        self.cache = Int8KvCache(device, context_window=16384, layers=1)
        self.lineage = PrefixLineage(self.cache, END)
        self.lineage.enabled = enabled
        self.workspace = DeviceAttentionWorkspace(device)
        self.workspace.prepare(512)
        self.q = device.allocate(512 * 4096 * 4)
        self.k = device.allocate(512 * 512 * 4)
        self.v = device.allocate(512 * 512 * 4)
        self.gate = device.allocate(512 * 4096 * 4)
        self.rotated = device.allocate(512 * 4096 * 4)
        self.out = device.allocate(512 * 4096 * 4)

    def rows(self, hashes):
        q, k, v, g = [], [], [], []
        for h in hashes:
            rng = np.random.default_rng(h)
            q.append(rng.standard_normal(4096, dtype=np.float32))
            kk = rng.standard_normal(512, dtype=np.float32)
            kk[[30, 31, 286, 287]] *= 20
            k.append(kk)
            v.append(rng.standard_normal(512, dtype=np.float32))
            g.append(rng.standard_normal(4096, dtype=np.float32))
        for buf, data in ((self.q, q), (self.k, k), (self.v, v), (self.gate, g)):
            buf.write(np.ascontiguousarray(np.stack(data)))

    def run(self, prompt):
        chain = [0]
        for t in prompt:
            chain.append(mix(chain[-1], t))
        tokens = list(prompt) + [100 + (chain[-1] + i) % 50000 for i in range(GENERATED)]
        for t in tokens[len(prompt):]:
            chain.append(mix(chain[-1], t))
        self.last_chunk = None

        def step(pos, count):
            self.cache.ensure_capacity(pos + count)
            self.rows(chain[pos + 1:pos + count + 1])
            layer = self.cache.layers[0]
            self.device.begin()
            engine.append_rows(self.device, layer, self.q, self.k, self.v, self.rotated, count, pos)
            if pos < len(prompt):
                self.workspace.encode_int8(self.rotated, layer.key, layer.value, layer.key_scale, layer.value_scale,
                                           self.gate, self.out, count, pos)
            else:
                engine.decode(self.device, layer, self.rotated, self.gate, self.out, pos)
            self.device.end()
            out = self.out.read(np.float32, count * 4096)
            if pos < len(prompt):
                self.last_chunk = (pos, count, out)
            else:
                self.last_decode = out

        cached, plan = run_prompt(self.lineage, prompt, step, GENERATED)
        return cached, self.cache.state_hash()

    def dispose(self):
        for b in (self.q, self.k, self.v, self.gate, self.rotated, self.out, self.cache.scores):
            b.dispose()
        for layer in self.cache.layers:
            for b in layer.buffers():
                b.dispose()
        self.workspace.dispose()


def test_warm_requests_equal_cold_builds(device):
    warm, cold = Request(device), Request(device, enabled=False)
    passed = []

    def compare(name, prompt, expect_cached=None):
        cached, state = warm.run(prompt)
        cold_cached, cold_state = cold.run(prompt)
        assert cold_cached == 0, name
        if expect_cached is not None:
            assert cached == expect_cached, f"{name}: cached {cached}, expected {expect_cached}"
        assert state == cold_state, f"{name}: KV state differs from a cold build"
        assert np.array_equal(warm.last_decode, cold.last_decode), f"{name}: decode differs"
        if cached < len(prompt):
            assert warm.last_chunk[:2] == cold.last_chunk[:2], name
            assert np.array_equal(warm.last_chunk[2], cold.last_chunk[2]), f"{name}: prefill rows differ"
        passed.append(name)
        return cached

    question = words(14, 10)
    simple = simple_chat(question)
    compare("initial", simple, 0)
    compare("identical", simple, len(simple))
    talk = conversation(question, words(1, 11), words(9, 12))
    compare("conversation-append", talk, simple.index(END) + 1)
    padding = words(4300, 13)
    long_prompt = simple_chat(padding + words(12, 14))
    compare("growth-seed", long_prompt[:4090])
    compare("append-through-kv-growth", long_prompt, 4090)
    assert warm.cache.capacity > 4096
    compare("long-identical", long_prompt, len(long_prompt))
    compare("branch", simple_chat(padding + words(12, 15)), 4096)
    compare("long-again", long_prompt, 4096)
    compare("shortened", long_prompt[:4100], 4096)
    compare("long-third", long_prompt, 4100)                     # the shortened prompt's own end
    compare("exact-block-boundary", long_prompt[:4096], 4096)
    compare("simple-again", simple, 0)
    busted = list(simple)
    busted[0] = END_OF_TEXT
    compare("busted", busted, 0)
    assert len(warm.lineage.checkpoints) <= 4
    assert len(passed) == 13
    warm.dispose()
    cold.dispose()
