"""MI355X (gfx950) INT8 KV-cache path: host mirror of the engine's KV policy over the
libbootstrap_hip.so C ABI. See native.py (P/Invoke twin) and engine.py (KV policy)."""
from .native import Binding, Device, GpuBuffer, HipError, KernelArgs, library_path, load_library  # noqa: F401
from .engine import (  # noqa: F401
    ContextLimits, DeviceAttentionWorkspace, Int8KvCache, Int8KvLayer, PrefixLineage, append_rows, decode, prepare_fused,
    decode_reference_path, grow_schedule, Fp16KvLayer, append_rows_fp16, encode_online_fp16, int8_value_capacity, store_rows, validate_context_window, value_index,
)

PACKAGE_DIR = __path__[0]
