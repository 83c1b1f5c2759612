"""Empty dispatches on the GPU: a dispatch with no rows (M = 0; for attention_softmax, no 256-thread
row groups) is accepted the way the reference's Metal encoder accepts a zero-thread dispatch
(Metal.cs:96-104), launches nothing and leaves every binding's bytes as they were. The fused
single-token step attention_decode_append_int8 serves exactly one row and refuses M = 0."""
import numpy as np
import pytest

from bootstrap_hip import HipError, KernelArgs

pytestmark = pytest.mark.gpu

GUARD, SIZE = 0x5A, 65536

# (kernel, arguments, bindings, dispatched threads, threads per group)
CASES = [
    ("kv_store_int8", KernelArgs(M=0, Position=100), 6, 0, 256),
    ("batch_rope_int8", KernelArgs(M=0, Position=100, Theta=1e7), 8, 0, 256),
    ("attention_query_grouped_half", KernelArgs(M=0, A=8), 2, 0, 128),
    ("attention_prepare_fused_int8", KernelArgs(M=0, Position=100, K=100, Theta=1e7, Epsilon=1e-6, A=8), 11, 0, 256),
    ("rmsnorm", KernelArgs(N=256, M=0, Flags=1, Epsilon=1e-6), 4, 0, 256),
    ("batch_split_q", KernelArgs(M=0), 3, 0, 128),
    ("attention_online_int8_q32_k256_r2", KernelArgs(M=0, K=100, Position=100, A=8), 7, 0, 256),
    ("attention_online_int8", KernelArgs(M=0, K=100, Position=100, A=8), 7, 0, 256),
    ("attention_online_int8_q32_k128", KernelArgs(M=0, K=100, Position=100, A=8), 7, 0, 256),
    ("attention_decode_int8", KernelArgs(M=0, K=100, Position=100), 7, 0, 256),
    ("attention_online_q32_k256_s8_g8_r2", KernelArgs(M=0, K=100, Position=100, A=8, Flags=256), 5, 0, 256),
    ("batch_rope", KernelArgs(M=0, Position=100, Theta=1e7, Flags=256), 6, 0, 128),
    ("attention_prepare_fused", KernelArgs(M=0, Position=100, K=100, Theta=1e7, Epsilon=1e-6, A=8, Flags=256), 9, 0,
     256),
    ("batch_attention_scores_int8", KernelArgs(M=0, K=100, Position=100), 4, 0, 128),
    ("attention_softmax", KernelArgs(M=0, K=100, Position=99), 1, 0, 256),
    ("batch_attention_values_int8", KernelArgs(M=0, K=100, Position=100), 5, 0, 128),
]


@pytest.mark.parametrize("noalloc", [False, True])
def test_empty_dispatches_leave_memory_untouched(device, noalloc):
    buffers = [device.allocate(SIZE) for _ in range(11)]
    for b in buffers:
        b.write(np.full(SIZE, GUARD, np.uint8))
    before = device.allocated_bytes
    device.begin()
    for kernel, args, count, threads, group in CASES:
        device.dispatch(kernel, args, threads, group, *buffers[:count], noalloc=noalloc)
    device.end()
    assert device.allocated_bytes == before, "an empty dispatch allocated device memory"
    for i, b in enumerate(buffers):
        assert np.all(b.read(np.uint8, SIZE) == GUARD), f"binding {i} was written"
    for b in buffers:
        b.dispose()


def test_decode_append_refuses_no_rows(device):
    buffers = [device.allocate(SIZE) for _ in range(10)]
    device.begin()
    with pytest.raises(HipError, match="M = 1"):
        device.dispatch("attention_decode_append_int8", KernelArgs(M=0, K=100, Position=100), 0, 256, *buffers)
    device.end()
    for b in buffers:
        b.dispose()
