"""CPU-side checks: the C ABI library loads and exports every declared symbol, and the
host KV policy mirrors the engine's constants and rules (Program.cs:307-320)."""
import ctypes
import os
import re
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for header in os.listdir(os.path.join(ROOT, "include")):
        if header.endswith(".h"):
            text = open(os.path.join(ROOT, "include", header)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"\b(boot_[a-z_0-9]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    from bootstrap_hip import native
    lib = ctypes.CDLL(native.library_path())
    declared = declared_functions()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), name
    assert set(native.SIGNATURES) == set(declared)


def test_kernel_args_layout():
    from bootstrap_hip import KernelArgs
    assert ctypes.sizeof(KernelArgs) == 64
    assert KernelArgs.Epsilon.offset == 32 and KernelArgs.C.offset == 48


def test_context_limits_rules():
    from bootstrap_hip import ContextLimits, validate_context_window
    for valid in (1, 512, 4096, 8192, 32768, 32769, 262144):                   # Program.cs:307
        assert validate_context_window(valid) == valid
    for invalid in (-1, 0, 262145, 2 ** 31 - 1):                               # Program.cs:308-312
        with pytest.raises(ValueError):
            validate_context_window(invalid)
    for position in (0, 4090, 32760, 65530, 262144 - 513):                     # Program.cs:313-318
        count = ContextLimits.prefill_count(position, 512)
        assert 1 <= count <= 512 and count * 16 * (position + count) <= ContextLimits.AttentionWorkspaceFloats
    assert ContextLimits.output_budget(10, 65536, 262144) == 65536             # Program.cs:319
    assert ContextLimits.output_budget(10, 2 ** 31 - 1, 32768) == 32758
    assert ContextLimits.output_budget(32767, 99999, 32768) == 1


def test_grow_schedule_doubles_to_window():
    from bootstrap_hip import grow_schedule
    cap, seen = 4096, []
    while cap < 262144:
        cap = grow_schedule(cap, cap + 1, 262144)
        seen.append(cap)
    assert seen == [8192, 16384, 32768, 65536, 131072, 262144]
    assert grow_schedule(4096, 131073, 262144) == 262144
    assert grow_schedule(4096, 5000, 6000) == 6000                             # capped at the window
    with pytest.raises(ValueError):
        grow_schedule(4096, 262145, 262144)


def test_target_kv_bytes_full_window():
    from bootstrap_hip import int8_value_capacity
    cap, layers = 262144, 10
    # QwenEngine.cs:24 for INT8: K and V codes + FP32 K/V scales + V page padding
    total = cap * 512 * 2 * layers + cap * 2 * 2 * layers * 4 + (int8_value_capacity(cap) - cap) * 512 * layers
    assert total == 2_726_297_600
    assert int8_value_capacity(4097) == 4352 and int8_value_capacity(4096) == 4096


def test_verify_slices_follow_the_workspace_budget():
    from bootstrap_hip import engine
    # Prefill.cs:273-276: rows per slice = AttentionWorkspaceFloats / 16 / (position + count)
    assert engine.verify_slices(8, 262136) == [(0, 8)]                        # full window: 8 rows fit
    slices = engine.verify_slices(512, 30208)                                 # 2097152 // 30720 = 68
    assert [n for _, n in slices] == [68] * 7 + [36]
    assert [f for f, _ in slices] == list(range(0, 512, 68))
    assert engine.verify_slices(5, 0, workspace_floats=16 * 5 * 2) == [(0, 2), (2, 2), (4, 1)]
    with pytest.raises(ValueError):
        engine.verify_slices(8, 100, workspace_floats=16 * 100)               # not one row fits
    with pytest.raises(ValueError):
        engine.verify_slices(0, 100)


class _RecordingLibrary:
    """Stands in for libbootstrap_hip.so: hands out handles and records release/destroy calls."""

    def __init__(self):
        self.calls, self.next = [], 100

    def boot_buffer(self, ctx, nbytes):
        self.next += 1
        return self.next

    def boot_release_buffer(self, handle):
        self.calls.append(("release", handle))

    def boot_destroy(self, ctx):
        self.calls.append(("destroy", ctx))

    def boot_error(self, ctx):
        return b"error"


def test_buffer_dispose_after_device_close_does_not_release():
    """boot_destroy frees every buffer the context owns (shim.cpp boot_destroy), so a buffer
    disposed after Device.close must not reach boot_release_buffer (freed memory)."""
    import weakref
    from bootstrap_hip.native import Device
    device = Device.__new__(Device)
    device.lib, device.handle, device._live = _RecordingLibrary(), 7, weakref.WeakSet()
    kept, released = device.allocate(64), device.allocate(64)
    released.dispose()
    released.dispose()                                   # a second dispose is a no-op
    device.close()
    kept.dispose()                                       # after close: handle forgotten only
    assert device.lib.calls == [("release", 102), ("destroy", 7)]
    assert kept.handle == 0 and released.handle == 0


def test_rope_frequencies_are_correctly_rounded():
    """The launchers evaluate the RoPE frequencies pow(theta, -float(2j)/64) (kernels.metal:123)
    as (float)pow((double)theta, ...) on the host; for the thetas in use that is the correctly
    rounded FP32 value of the exact power (checked here with 60-digit decimal arithmetic)."""
    import math
    from decimal import Decimal, getcontext
    import numpy as np
    getcontext().prec = 60
    for theta in (10_000_000.0, 1_000_000.0, 10_000.0):
        for j in range(32):
            exact = (Decimal(theta).ln() * (Decimal(-2 * j) / Decimal(64))).exp()
            host = np.float32(math.pow(theta, float(np.float32(-(2 * j)) / np.float32(64.0))))
            f = np.float32(float(exact))
            nearest = min((np.nextafter(f, np.float32(-1)), f, np.nextafter(f, np.float32(2))),
                          key=lambda c: abs(Decimal(float(c)) - exact))
            assert host == nearest, (theta, j)


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 exits with status 2 and says why, before touching a device."""
    import json
    import subprocess
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert out.returncode == 2
    line = json.loads(out.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]
