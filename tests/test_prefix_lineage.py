"""Checkpoint policy of the single KV lineage on the CPU (PrefixCache.cs:8-122,
QwenEngine.cs:195-233), driven through the sequence of PrefixCacheSelfTest.Run
(PrefixCacheSelfTest.cs:22-112) over a stand-in store that records truncations and resets."""
import pytest

from bootstrap_hip import PrefixLineage
from lineage_case import END, END_OF_TEXT, conversation, run_prompt, simple_chat, words


class Store:
    """Position bookkeeping of Int8KvCache without a device."""

    def __init__(self):
        self.position = 0
        self.resets = 0
        self.written = []

    def reset(self):
        self.position = 0
        self.resets += 1

    def restore_prefix(self, position):
        if position < 0 or position > self.position:
            raise ValueError("checkpoint beyond the live lineage")
        self.position = position
        return position


def make():
    store = Store()
    lineage = PrefixLineage(store, END)

    def step(pos, rows):
        assert pos == store.position, "prefill must resume exactly where the lineage ends"
        store.written.append((pos, rows))

    return lineage, lambda prompt, n=12: run_prompt(lineage, prompt, step, n)[0], store


def test_boundaries_and_plan():
    lineage, _, _ = make()
    simple = simple_chat(words(12, 1))
    end = simple.index(END) + 1
    assert lineage.boundaries(simple) == [end, len(simple)]
    long_prompt = simple_chat(words(4300, 2))
    assert lineage.boundaries(long_prompt) == [4096, long_prompt.index(END) + 1, len(long_prompt)]
    talk = conversation(words(9000, 3), words(5, 4), words(3000, 5))   # three message ends, two blocks
    ends = [i + 1 for i, t in enumerate(talk) if t == END]
    b = lineage.boundaries(talk)
    assert len(b) == 4 and ends[0] in b and ends[-1] in b and len(talk) in b
    assert b == sorted({len(talk), ends[0], ends[-1], (len(talk) - 1) // 4096 * 4096})
    # 512-row chunks up to each boundary; a tail under 8 rows runs token by token
    plan = PrefixLineage.plan(4200, 0, [4096, 4191, 4200])
    assert plan[:8] == [(i * 512, 512, i == 7) for i in range(8)]
    assert plan[8] == (4096, 95, True)
    assert plan[9] == (4191, 9, True)
    assert PrefixLineage.plan(10, 4, [6, 10]) == [(4, 1, False), (5, 1, True), (6, 1, False), (7, 1, False),
                                                 (8, 1, False), (9, 1, True)]
    # the attention workspace bounds rows per chunk deep in the window (ContextLimits.cs:5-19)
    deep = PrefixLineage.plan(200000 + 512, 200000, [200512])
    assert deep[0] == (200000, 10, False) and all(rows <= 10 for _, rows, _ in deep)


def test_self_test_sequence():
    lineage, run, store = make()
    question = words(14, 10)
    simple = simple_chat(question)
    assert run(simple) == 0                                              # initial miss
    assert run(simple) == len(simple)                                    # exact full hit
    assert store.written[-12:] == [(len(simple) + i, 1) for i in range(12)]
    assert run(simple, 16) == len(simple)                                # ignore_eos reuses the hit
    talk = conversation(question, words(1, 11), words(9, 12))
    run(simple)
    expected = lineage.cached_tokens(talk)
    assert 0 < expected < len(simple) and expected == simple.index(END) + 1
    assert run(talk) == expected                                         # append accounting
    # a checkpoint through KV growth, then the block checkpoint for branch / shorten / boundary
    padding = words(4300, 13)
    long_prompt = simple_chat(padding + words(12, 14))
    assert len(long_prompt) > 4096
    seed = long_prompt[:4090]
    run(seed)
    assert run(long_prompt) == 4090
    assert run(long_prompt) == len(long_prompt)                          # long exact hit
    branch = simple_chat(padding + words(12, 15))
    assert run(branch) == 4096                                           # branch falls back to the block
    run(long_prompt)
    assert run(long_prompt[:4100]) == 4096                               # shorten restores earlier state
    run(long_prompt)
    assert run(long_prompt[:4096]) == 4096                               # exact intermediate checkpoint
    assert store.written[-12][0] == 4096                                 # nothing re-prefilled
    run(simple)
    busted = list(simple)
    busted[0] = END_OF_TEXT
    assert lineage.cached_tokens(busted) == 0                            # first-token change misses
    resets = store.resets
    assert run(busted) == 0 and store.resets == resets + 1 and lineage.checkpoints == [busted.index(END) + 1,
                                                                                        len(busted)]
    run(simple)
    lineage.clear()                                                      # cancellation / writer failure
    assert lineage.cached_tokens(simple) == 0
    run(simple)
    lineage.reset()
    assert lineage.cached_tokens(simple) == 0                            # explicit reset
    run(simple)
    lineage.enabled = False
    assert lineage.cached_tokens(simple) == 0                            # mode change
    assert run(simple) == 0 and lineage.tokens == [] and lineage.checkpoints == []
    lineage.enabled = True
    mutable = list(simple)
    run(mutable)
    mutable[0] = END_OF_TEXT
    assert lineage.cached_tokens(simple) == len(simple) and lineage.cached_tokens(mutable) == 0
    assert len(lineage.checkpoints) <= 4


def test_restore_drops_later_checkpoints_and_eviction_keeps_boundaries():
    lineage, run, store = make()
    talk = conversation(words(9000, 20), words(5, 21), words(3000, 22))
    run(talk)
    saved = list(lineage.checkpoints)
    assert saved == lineage.boundaries(talk)                             # every boundary reached
    short = talk[:8192 + 5]
    assert run(short) == 8192
    assert saved[0] == 8192 and all(c > 8192 for c in saved[1:])
    assert lineage.checkpoints == [8192, 8192 + 5]                       # later ones dropped, own end saved
    # full index: the new checkpoint evicts the first one that is not this request's boundary
    lineage.checkpoints = [10, 20, 30, 40]
    lineage.save(50, [20, 30, 40, 50])
    assert lineage.checkpoints == [20, 30, 40, 50]
    lineage.save(60, [20, 30, 40, 50, 60])
    assert lineage.checkpoints == [30, 40, 50, 60]
    lineage.save(60, [60])                                               # already saved: no change
    assert lineage.checkpoints == [30, 40, 50, 60]
    with pytest.raises(ValueError):
        store.position = 5
        lineage.restore(talk[:35])                                       # checkpoint past the live end
