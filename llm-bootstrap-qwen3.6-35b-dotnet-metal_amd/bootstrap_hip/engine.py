"""Host-side KV policy and call sites of the INT8 full-attention path.

The reference engine keeps these in C# (QwenEngine.cs, DeviceAttention.cs,
ContextLimits.cs, PrefixCache.cs); this module restates exactly those lines over the
HIP shim so the device path can be driven the way the engine drives it:

* ``ContextLimits``            ContextLimits.cs:5-19
* ``Int8KvCache``              QwenEngine.cs:17-24,43,61 (allocation), 76-99 (grow by
                               doubling with a device copy), 122-132 (reset), and
                               PrefixCache.cs:45-77 (restore = truncate by position, no clear);
                               ``state_hash`` follows PrefixCacheSelfTest.cs:133-148 (KV part)
* ``DeviceAttentionWorkspace`` DeviceAttention.cs:14-20 (Prepare), 65-70 (EncodeInt8)
* ``append_rows`` / ``decode`` the INT8 lines of PrefillBlock (Prefill.cs:248-261) and
                               Forward (QwenEngine.cs:158-166)
* ``verify_attention_int8``    the verify-block reader of PrefillBlock (Prefill.cs:269-285)
* ``PrefixLineage``            checkpoint index of the single KV lineage (PrefixCache.cs:8-122,
                               QwenEngine.cs:195-233), KV part
"""
from __future__ import annotations

import hashlib
from typing import List, Optional

import numpy as np

from .native import Binding, Device, GpuBuffer, HipError, KernelArgs

# ContextLimits.cs:5-6
NATIVE_WINDOW = 262144
ATTENTION_WORKSPACE_FLOATS = 32 * 1024 * 1024
# QwenEngine.cs:58-61: layer l is full attention when (l + 1) % 4 == 0 -> 10 of 40
FULL_ATTENTION_LAYERS = tuple(l for l in range(40) if (l + 1) % 4 == 0)
KV_HEADS, HEAD_DIM, Q_HEADS, GROUP = 2, 256, 16, 8
ROPE_THETA = 10_000_000.0


class ContextLimits:
    """ContextLimits.cs:3-20."""

    NativeWindow = NATIVE_WINDOW
    AttentionWorkspaceFloats = ATTENTION_WORKSPACE_FLOATS

    @staticmethod
    def output_budget(prompt_tokens: int, requested: int, context_window: int) -> int:
        if prompt_tokens < 1 or prompt_tokens >= context_window or requested < 1:
            raise ValueError("Context window exceeded or invalid output budget")
        return min(requested, context_window - prompt_tokens)

    @staticmethod
    def prefill_count(position: int, remaining: int) -> int:
        count = min(512, remaining)
        return min(count, ATTENTION_WORKSPACE_FLOATS // 16 // (position + count))


def validate_context_window(context_window: int) -> int:
    """QwenEngine.cs:25."""
    if 1 <= context_window <= NATIVE_WINDOW:
        return context_window
    raise ValueError("Context window must fit the model's native 262144-token window")


def int8_value_capacity(capacity: int) -> int:
    """QwenEngine.cs:23: V is allocated in whole 256-token pages."""
    return (capacity + 255) // 256 * 256


def value_index(vector: int, dimension: int) -> int:
    """kernels.metal:126-128."""
    token, head = vector // 2, vector % 2
    return (token // 256 * 2 + head) * 65536 + dimension * 256 + token % 256


def grow_schedule(capacity: int, required: int, context: int) -> int:
    """QwenEngine.cs:85-88: double (capped at the window) until ``required`` fits."""
    if required <= capacity:
        return capacity
    if required > context:
        raise ValueError("required KV capacity exceeds the context window")
    while capacity < required:
        capacity = min(context, capacity * 2)
    return capacity


class Int8KvLayer:
    """One full-attention layer's INT8 cache: K codes, V pages, K/V scales."""

    def __init__(self, device: Device, capacity: int):
        self.key = device.allocate(capacity * 512)
        self.value = device.allocate(int8_value_capacity(capacity) * 512)
        self.key_scale = device.allocate(capacity * 2 * 4)
        self.value_scale = device.allocate(capacity * 2 * 4)

    def buffers(self) -> List[GpuBuffer]:
        return [self.key, self.value, self.key_scale, self.value_scale]


class Int8KvCache:
    """KV allocation / growth / reset / truncate policy of the INT8 target cache."""

    def __init__(self, device: Device, context_window: int = NATIVE_WINDOW, layers: int = 10):
        self.device = device
        self.context = validate_context_window(context_window)
        self.capacity = min(self.context, 4096)                  # QwenEngine.cs:43
        self.layers = [Int8KvLayer(device, self.capacity) for _ in range(layers)]
        self.scores = device.allocate(16 * self.capacity * 4)    # QwenEngine.cs:57 (Buffer(16*cap))
        self.position = 0                                        # consumed tokens of the live lineage
        self.growth_log: List[int] = []

    @property
    def target_kv_bytes(self) -> int:
        """QwenEngine.cs:24 for INT8, scaled to this cache's layer count."""
        n = len(self.layers)
        cap = self.capacity
        return cap * 512 * 2 * n + cap * 2 * 2 * n * 4 + (int8_value_capacity(cap) - cap) * 512 * n

    def _grow(self, buffer: GpuBuffer, nbytes: int) -> GpuBuffer:
        """QwenEngine.cs:76-82: allocate zero-filled, copy all old bytes, release."""
        if nbytes <= buffer.length:
            return buffer
        replacement = self.device.allocate(nbytes)
        self.device.copy(replacement, 0, buffer, 0, buffer.length)
        buffer.dispose()
        return replacement

    def ensure_capacity(self, required: int) -> None:
        """QwenEngine.cs:83-99. Must run with no command active (QwenEngine.cs:89)."""
        capacity = grow_schedule(self.capacity, required, self.context)
        if capacity == self.capacity:
            return
        for layer in self.layers:
            layer.key = self._grow(layer.key, capacity * 512)
            layer.value = self._grow(layer.value, int8_value_capacity(capacity) * 512)
            layer.key_scale = self._grow(layer.key_scale, capacity * 2 * 4)
            layer.value_scale = self._grow(layer.value_scale, capacity * 2 * 4)
        self.scores = self._grow(self.scores, capacity * 16 * 4)
        self.capacity = capacity
        self.growth_log.append(capacity)

    def reset(self) -> None:
        """QwenEngine.cs:122-132 (KV part): clear K, V and both scale buffers."""
        self.device.begin()
        for layer in self.layers:
            for buffer in layer.buffers():
                self.device.clear(buffer)
        self.device.end()
        self.position = 0

    def restore_prefix(self, position: int) -> int:
        """PrefixCache.cs:45-77, KV part: positions at/after the checkpoint are not cleared;
        causal masking and overwrite-before-read keep them unobservable (PrefixCache.cs:68-70)."""
        if position < 0 or position > self.position:
            raise ValueError("checkpoint beyond the live lineage")
        self.position = position
        return position

    def state_hash(self, consumed: Optional[int] = None) -> str:
        """KV part of PrefixTestStateHash (PrefixCacheSelfTest.cs:133-148): K bytes
        consumed*512, whole V pages plus the consumed prefix of the partial page per
        (head, d), and the K/V scales consumed*8 bytes; layer by layer."""
        consumed = self.position if consumed is None else consumed
        h = hashlib.sha256()
        pages, tail = consumed // 256, consumed % 256
        for layer in self.layers:
            h.update(layer.key.read(np.uint8, consumed * 512).tobytes())
            h.update(layer.value.read(np.uint8, pages * 256 * 512).tobytes())
            if tail:
                block = layer.value.read(np.uint8, 2 * 65536, pages * 2 * 65536).reshape(2, 256, 256)
                for head in range(2):
                    for d in range(256):
                        h.update(block[head, d, :tail].tobytes())
            h.update(layer.key_scale.read(np.uint8, consumed * 8).tobytes())
            h.update(layer.value_scale.read(np.uint8, consumed * 8).tobytes())
        return h.hexdigest()


# PrefixCache.cs:8
PREFIX_CHECKPOINT_LIMIT, PREFIX_CHECKPOINT_INTERVAL = 4, 4096


class PrefixLineage:
    """Checkpoint index of the single live KV lineage (PrefixCache.cs:8-122 and the prompt loop
    of QwenEngine.cs:195-233), KV part. A checkpoint is a position of that lineage: the codes and
    scales stay in place in the device store, and restoring one truncates the lineage by position
    (``Int8KvCache.restore_prefix``); nothing past it is cleared, since every position consumed
    later is overwritten before a causal read. The recurrent/conv/logit snapshot the reference
    stores with each checkpoint belongs to the model's other layers and is not kept here.
    ``end_token`` is the tokenizer's message-end id (Tokenizer.cs:19)."""

    def __init__(self, cache: Int8KvCache, end_token: int, limit: int = PREFIX_CHECKPOINT_LIMIT,
                 interval: int = PREFIX_CHECKPOINT_INTERVAL):
        self.cache = cache
        self.end_token = end_token
        self.limit, self.interval = limit, interval
        self.checkpoints: List[int] = []     # positions, in the order saved (PrefixCache.cs:12)
        self.tokens: List[int] = []          # the prompt the lineage was built from (PrefixCache.cs:14)
        self._enabled = True

    @property
    def enabled(self) -> bool:
        return self._enabled

    @enabled.setter
    def enabled(self, value: bool) -> None:
        """PrefixCache.cs:16-20: toggling drops every checkpoint."""
        if self._enabled != value:
            self.clear()
        self._enabled = value

    def clear(self) -> None:
        """ClearPrefixCache (PrefixCache.cs:28-32)."""
        self.checkpoints = []
        self.tokens = []

    def reset(self) -> None:
        """QwenEngine.cs:122-131, KV part: drop the checkpoints and clear the store."""
        self.clear()
        self.cache.reset()

    def find(self, prompt) -> Optional[int]:
        """FindPrefix (PrefixCache.cs:34-40): the last saved checkpoint inside the prompt's common
        prefix with the lineage's prompt."""
        if not self._enabled:
            return None
        common, limit = 0, min(len(prompt), len(self.tokens))
        while common < limit and prompt[common] == self.tokens[common]:
            common += 1
        hits = [c for c in self.checkpoints if c <= common]
        return hits[-1] if hits else None

    def cached_tokens(self, prompt) -> int:
        """CachedPrefixTokens (PrefixCache.cs:42)."""
        found = self.find(prompt)
        return 0 if found is None else found

    def restore(self, prompt) -> int:
        """RestorePrefix (PrefixCache.cs:45-77), KV part: no checkpoint resets the lineage;
        otherwise checkpoints past the one found are dropped before the first write and the
        lineage is truncated to it. Returns the position prefill resumes from."""
        checkpoint = self.find(prompt)
        if checkpoint is None:
            self.reset()
            return 0
        while self.checkpoints and self.checkpoints[-1] > checkpoint:
            self.checkpoints.pop()
        return self.cache.restore_prefix(checkpoint)

    def boundaries(self, prompt) -> List[int]:
        """PrefixBoundaries (PrefixCache.cs:107-122): prompt end, end of the first and of the
        last message, then whole checkpoint-interval blocks from the latest down, at most
        ``limit`` positions."""
        n = len(prompt)
        found = {n}
        ends = [i for i, t in enumerate(prompt) if t == self.end_token]
        first_message = ends[0] + 1 if ends else 0
        last_message = ends[-1] + 1 if ends else 0
        if first_message > 0:
            found.add(first_message)
        if last_message > 0:
            found.add(last_message)
        block = (n - 1) // self.interval * self.interval
        while block > 0 and len(found) < self.limit:
            found.add(block)
            block -= self.interval
        return sorted(found)

    def save(self, position: int, boundaries: List[int]) -> None:
        """SavePrefix (PrefixCache.cs:79-105), KV part: at the limit, evict the first checkpoint
        that is not one of this request's boundaries (else the oldest)."""
        if not self._enabled or position in self.checkpoints:
            return
        if len(self.checkpoints) == self.limit:
            victims = [i for i, c in enumerate(self.checkpoints) if c not in boundaries]
            del self.checkpoints[victims[0] if victims else 0]
        self.checkpoints.append(position)

    def begin(self, prompt) -> tuple:
        """The head of Generate (QwenEngine.cs:201-206): restore, then own a copy of the prompt
        as the lineage key. Returns (position, boundaries)."""
        position = self.restore(prompt)
        boundaries = self.boundaries(prompt)
        self.tokens = list(prompt) if self._enabled else []
        return position, boundaries

    @staticmethod
    def plan(prompt_length: int, position: int, boundaries: List[int]) -> List[tuple]:
        """The batched prompt loop of QwenEngine.cs:207-233 (WidePrefill off): chunks of
        ``ContextLimits.prefill_count`` rows that never cross a boundary; a chunk under 8 rows
        runs one token at a time. (position, rows, checkpoint-after) triples."""
        chunks = []
        while position < prompt_length:
            boundary = next(p for p in boundaries if p > position)
            count = ContextLimits.prefill_count(position, boundary - position)
            if count < 8:
                count = 1
            chunks.append((position, count, position + count == boundary))
            position += count
        return chunks


class DeviceAttentionWorkspace:
    """DeviceAttention.cs:5-72, INT8 part: grouped FP16 query scratch + EncodeInt8."""

    OnlineGroupHeads = 8

    def __init__(self, device: Device):
        self.device = device
        self.query: Optional[GpuBuffer] = None

    def prepare(self, rows: int) -> None:
        """DeviceAttention.cs:14-20 (INT8 needs only the packed query)."""
        need = rows * 4096 * 2
        if self.query is None or self.query.length < need:
            if self.query is not None:
                self.query.dispose()
            self.query = self.device.allocate(need)

    @property
    def packed_query(self) -> GpuBuffer:
        if self.query is None:
            raise HipError("Attention is not prepared")
        return self.query

    def encode_int8(self, q, k, v, ks, vs, gate, output, rows: int, position: int,
                    prepared_query: bool = False) -> None:
        """DeviceAttention.cs:65-70. Must be called inside a command."""
        p = KernelArgs(M=rows, K=position + rows, Position=position, A=self.OnlineGroupHeads)
        if not prepared_query:
            self.device.dispatch("attention_query_grouped_half", p, rows * 1024, 128, q, self.packed_query)
        self.device.dispatch2d("attention_online_int8_q32_k256_r2", p, (rows * 8 + 31) // 32 * 256, 2, 256,
                               self.packed_query, k, v, gate, output, ks, vs)

    def dispose(self) -> None:
        if self.query is not None:
            self.query.dispose()
            self.query = None


def append_rows(device: Device, layer: Int8KvLayer, q, k, v, rotated, rows: int, position: int,
                theta: float = ROPE_THETA) -> None:
    """Unfused INT8 append of Prefill.cs:257 / QwenEngine.cs:162: rotate Q into ``rotated``,
    rotate K and store K/V codes and scales at ``position``. Inside a command."""
    p = KernelArgs(M=rows, Position=position, K=position + rows, Theta=theta)
    device.dispatch("batch_rope_int8", p, rows * 4096, 256, q, k, v, rotated,
                    layer.key, layer.value, layer.key_scale, layer.value_scale)


def prepare_fused(device: Device, layer: Int8KvLayer, qkv, k, v, q_norm, k_norm, packed, gate, rows: int,
                  position: int, theta: float = ROPE_THETA, epsilon: float = 1e-6) -> None:
    """Fused INT8 preparation of Prefill.cs:250 (attention_prepare_fused_int8): Q/K RMS norm with
    (w + 1), RoPE, grouped FP16 Q + gate split, INT8 K/V append. Inside a command."""
    p = KernelArgs(M=rows, Position=position, K=position + rows, Theta=theta, Epsilon=epsilon, A=GROUP)
    device.dispatch("attention_prepare_fused_int8", p, rows * 18 * 256, 256, qkv, k, v, q_norm, k_norm, packed,
                    gate, layer.key, layer.value, layer.key_scale, layer.value_scale)


def prepare_fused_fp16(device: Device, layer: "Fp16KvLayer", qkv, k, v, q_norm, k_norm, packed, gate, rows: int,
                       position: int, theta: float = ROPE_THETA, epsilon: float = 1e-6) -> None:
    """Fused FP16-KV preparation of Prefill.cs:252 (attention_prepare_fused): Q/K RMS norm with
    (w + 1), RoPE, grouped FP16 Q + gate split, FP16 K/V append. Inside a command."""
    p = KernelArgs(M=rows, Position=position, K=position + rows, Theta=theta, Epsilon=epsilon, A=GROUP)
    device.dispatch("attention_prepare_fused", p, rows * 18 * 256, 256, qkv, k, v, q_norm, k_norm, packed, gate,
                    layer.key, layer.value)


def store_rows(device: Device, layer: Int8KvLayer, k, v, rows: int, position: int) -> None:
    """Append already-rotated FP32 K/V rows (store_kv_int8 alone). Inside a command."""
    device.dispatch("kv_store_int8", KernelArgs(M=rows, Position=position), rows * 512, 256,
                    k, v, layer.key, layer.value, layer.key_scale, layer.value_scale)


class Fp16KvLayer:
    """FP16 control cache of one layer: token-major K and V [cap][2][256] halves
    (kernels.metal:16-21 with flags bit 256; QwenEngine.cs:61 with KvElementBytes = 2)."""

    def __init__(self, device: Device, capacity: int):
        self.key = device.allocate(capacity * 512 * 2)
        self.value = device.allocate(capacity * 512 * 2)

    def buffers(self) -> List[GpuBuffer]:
        return [self.key, self.value]


def append_rows_fp16(device: Device, layer: Fp16KvLayer, q, k, v, rotated, rows: int, position: int,
                     theta: float = ROPE_THETA) -> None:
    """Unfused FP16 append (batch_rope with KvFlags = 256, Prefill.cs:258). Inside a command."""
    p = KernelArgs(M=rows, Position=position, K=position + rows, Theta=theta, Flags=256)
    device.dispatch("batch_rope", p, rows * 4096, 128, q, k, v, rotated, layer.key, layer.value)


def encode_online_fp16(workspace: "DeviceAttentionWorkspace", q, layer: Fp16KvLayer, gate, output, rows: int,
                       position: int, prepared_query: bool = False) -> None:
    """DeviceAttention.cs:50-63 (EncodeOnline, FP16 KV): grouped FP16 query, then the FP16 online
    kernel. The reference routes fewer than 32 rows to its non-online path; the gfx950 online
    kernel serves every row count. Inside a command."""
    device = workspace.device
    p = KernelArgs(M=rows, K=position + rows, Position=position, A=GROUP)
    if not prepared_query:
        device.dispatch("attention_query_grouped_half", p, rows * 1024, 128, q, workspace.packed_query)
    device.dispatch2d("attention_online_q32_k256_s8_g8_r2", p, (rows * 8 + 31) // 32 * 256, 2, 256,
                      workspace.packed_query, layer.key, layer.value, gate, output)


def decode(device: Device, layer: Int8KvLayer, rotated, gate, output, position: int, rows: int = 1) -> None:
    """Fused split-K decode over keys [0, position + row] for each row. Inside a command."""
    p = KernelArgs(M=rows, K=position + rows, Position=position)
    device.dispatch("attention_decode_int8", p, rows * 4096, 256, rotated, layer.key, layer.value,
                    gate, output, layer.key_scale, layer.value_scale)


def decode_append(device: Device, layer: Int8KvLayer, q, k, v, rotated, gate, output, position: int,
                  theta: float = ROPE_THETA) -> None:
    """One decode step of QwenEngine.cs:161-165 in one dispatch: batch_rope_int8 with M = 1
    (rotate q into ``rotated``, rotate k and append k/v at ``position``) followed by attention
    of the rotated query over keys [0, position]. Same bytes as ``append_rows`` then ``decode``.
    Inside a command."""
    p = KernelArgs(M=1, K=position + 1, Position=position, Theta=theta)
    device.dispatch("attention_decode_append_int8", p, 4096, 256, q, k, v, rotated, layer.key, layer.value,
                    layer.key_scale, layer.value_scale, gate, output)


def decode_reference_path(device: Device, layer: Int8KvLayer, rotated, gate, output, scores: GpuBuffer,
                          position: int, rows: int = 1) -> None:
    """The engine's three-kernel INT8 reader (QwenEngine.cs:163-165, Prefill.cs:280-283)."""
    length = position + rows
    p = KernelArgs(M=rows, K=length, Position=position)
    device.dispatch2d("batch_attention_scores_int8", p, length * 32, rows * 16, 128, rotated, layer.key, scores,
                      layer.key_scale)
    soft = KernelArgs(M=rows, K=length, Position=length - 1)
    device.dispatch("attention_softmax", soft, rows * 16 * 256, 256, scores)
    device.dispatch("batch_attention_values_int8", p, rows * 4096, 128, scores, layer.value, gate, output,
                    layer.value_scale)


def verify_slices(rows: int, position: int,
                  workspace_floats: int = ATTENTION_WORKSPACE_FLOATS) -> List[tuple]:
    """Query slices of a verify block (Prefill.cs:273-276): as many rows per slice as keep
    rows*16*(position+rows_total) score floats inside the workspace; (first, count) pairs."""
    length = position + rows
    capacity = workspace_floats // 16 // length
    if rows < 1 or capacity < 1:
        raise ValueError("Attention workspace budget exceeded")
    return [(first, min(capacity, rows - first)) for first in range(0, rows, capacity)]


def verify_attention_int8(device: Device, layer: Int8KvLayer, rotated: GpuBuffer, gate: GpuBuffer,
                          scores: GpuBuffer, rows: int, position: int,
                          workspace_floats: int = ATTENTION_WORKSPACE_FLOATS) -> None:
    """INT8 attention of a speculative verify block (Prefill.cs:269-285, ``verify`` true): the
    scalar reader over query slices. Each slice keeps its absolute causal position and the whole
    block's key count as the score stride, and writes its output over its own rotated query rows.
    Inside a command."""
    length = position + rows
    for first, count in verify_slices(rows, position, workspace_floats):
        if scores.length < count * 16 * length * 4:
            raise ValueError("score workspace smaller than one slice")
        p = KernelArgs(M=count, K=length, Position=position + first)
        query, g = rotated.at(first * 4096 * 4), gate.at(first * 4096 * 4)
        device.dispatch2d("batch_attention_scores_int8", p, length * 32, count * 16, 128, query, layer.key, scores,
                          layer.key_scale)
        soft = KernelArgs(M=count, K=length, Position=length - 1)
        device.dispatch("attention_softmax", soft, count * 16 * 256, 256, scores)
        device.dispatch("batch_attention_values_int8", p, count * 4096, 128, scores, layer.value, g, query,
                        layer.value_scale)
