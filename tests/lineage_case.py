"""Synthetic token prompts in the shape of Tokenizer.SimpleChat (Tokenizer.cs:79-86) and a
driver that runs one request's prompt loop through ``PrefixLineage`` (QwenEngine.cs:195-233).
Token ids: IM_START 1, END 2 (<|im_end|>), END_OF_TEXT 3, THINK 4, THINK_END 5, NL 6,
USER 7, ASSISTANT 8; words are ids >= 100."""
import numpy as np

IM_START, END, END_OF_TEXT, THINK, THINK_END, NL, USER, ASSISTANT = 1, 2, 3, 4, 5, 6, 7, 8


def words(n, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(100, 50000, n)]


def simple_chat(user):
    """<|im_start|>user\\n{user}<|im_end|>\\n<|im_start|>assistant\\n<think>\\n\\n</think>\\n\\n"""
    return [IM_START, USER, NL] + list(user) + [END, NL, IM_START, ASSISTANT, NL, THINK, NL, NL, THINK_END, NL, NL]


def conversation(first, answer, second):
    """user / assistant / user turns; the assistant turn carries no think block, so the prompt
    departs from simple_chat(first) right after the first message's end."""
    return ([IM_START, USER, NL] + list(first) + [END, NL, IM_START, ASSISTANT, NL] + list(answer) + [END, NL]
            + [IM_START, USER, NL] + list(second) + [END, NL, IM_START, ASSISTANT, NL, THINK, NL, NL, THINK_END, NL,
                                                     NL])


def run_prompt(lineage, prompt, step, generated: int = 0):
    """One request: restore, prefill the rest in planned chunks (``step(position, rows)`` does the
    device work), save a checkpoint at each boundary reached, then consume ``generated`` decode
    tokens. Returns (cached tokens, plan)."""
    position, bounds = lineage.begin(prompt)
    cached = position
    plan = lineage.plan(len(prompt), position, bounds)
    for pos, rows, checkpoint in plan:
        step(pos, rows)
        lineage.cache.position = pos + rows
        if checkpoint:
            lineage.save(pos + rows, bounds)
    for i in range(generated):
        step(len(prompt) + i, 1)
        lineage.cache.position = len(prompt) + i + 1
    return cached, plan
