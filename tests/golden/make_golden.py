#!/usr/bin/env python3
"""Writes tests/golden/kv_golden.json: the known answers the tests check the CPU oracle and
the GPU path against. Run from the repository root after building oracle/libkvref.so.

Contents and where each comes from:
* splitmix64: the published first outputs of splitmix64 seeded with 1234567 (Vigna's
  reference splitmix64.c test vector). They are typed in here, not computed by the oracle.
* reference_cases: the (history, rows) attention cases of Int8KvTests.cs:24 and the
  tolerances the reference asserts (Int8KvTests.cs:54,59,156,169,178; KvStorageTests.cs:55).
* config1: SHA-256 of the oracle's INT8 cache for config 1 (512 tokens of N(0,1) K seed 0 /
  V seed 1 at position 0, capacity 513). A regression anchor: once the oracle is pinned by
  the checks in tests/test_oracle.py, every later build must reproduce these bytes.
"""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from oracle_lib import Oracle  # noqa: E402

SPLITMIX64_1234567 = [6457827717110365317, 3203168211198807973, 9817491932198370423,
                      4593380528125082431, 16408922859458223821]


def config1_digests(oracle):
    k = oracle.normal(512 * 512, 0).reshape(512, 2, 256)
    v = oracle.normal(512 * 512, 1).reshape(512, 2, 256)
    kc, vc, ks, vs = oracle.empty_cache(513, fill=0)
    oracle.store(k, v, 0, kc, vc, ks, vs)
    return {name: hashlib.sha256(a.tobytes()).hexdigest()
            for name, a in (("key_codes", kc), ("value_pages", vc), ("key_scales", ks), ("value_scales", vs))}


def main():
    oracle = Oracle()
    golden = {
        "splitmix64": {"seed": 1234567, "outputs": [str(x) for x in SPLITMIX64_1234567]},
        "reference_cases": {
            "attention_history_rows": [[0, 1], [17, 7], [127, 31], [127, 32], [257, 33], [4093, 7],
                                       [8192, 128], [30000, 33]],
            "store": {"rows": 33, "position": 4093, "theta": 1e7, "epsilon": 1e-6,
                      "scale_abs_tol": 2e-5, "code_abs_tol": "amax/254 + 3e-3"},
            "attention_abs_tol": "sum|p*v*vs| / gate / 256 + 1e-4",
            "scalar_reader_abs_tol": 4.1e-3,
            "small_value_scale": {"factor": 1e-6, "rel_tol": 0.008},
            "rope_abs_tol": 6e-4,
        },
        "config1": {"tokens": 512, "k_seed": 0, "v_seed": 1, "position": 0, "capacity": 513,
                    "sha256": config1_digests(oracle)},
    }
    with open(os.path.join(HERE, "kv_golden.json"), "w") as f:
        json.dump(golden, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
