"""The CPU oracle against the committed known answers in tests/golden/kv_golden.json:
published splitmix64 outputs (the seeded generator every synthetic config uses) and the
config-1 INT8 cache digests. CPU only."""
import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kv_golden.json")


def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def test_splitmix64_published_outputs(oracle):
    g = golden()["splitmix64"]
    got = oracle.splitmix64(g["seed"], len(g["outputs"]))
    assert [int(x) for x in got] == [int(x) for x in g["outputs"]]


def test_config1_cache_digests(oracle):
    g = golden()["config1"]
    k = oracle.normal(g["tokens"] * 512, g["k_seed"]).reshape(g["tokens"], 2, 256)
    v = oracle.normal(g["tokens"] * 512, g["v_seed"]).reshape(g["tokens"], 2, 256)
    kc, vc, ks, vs = oracle.empty_cache(g["capacity"], fill=0)
    oracle.store(k, v, g["position"], kc, vc, ks, vs)
    for name, a in (("key_codes", kc), ("value_pages", vc), ("key_scales", ks), ("value_scales", vs)):
        assert hashlib.sha256(a.tobytes()).hexdigest() == g["sha256"][name], name


def test_reference_cases_recorded():
    cases = golden()["reference_cases"]["attention_history_rows"]
    assert len(cases) == 8 and all(h >= 0 and r >= 1 and h + r <= 262144 for h, r in cases)
    assert np.array_equal(np.array(cases)[:, 1], [1, 7, 31, 32, 33, 7, 128, 33])
