"""Write the committed fixtures of tests/golden/ (run from the repository root).

* known_answer_update.json -- the reference's own known-answer case
  (tests/test_kv_cache.py:24-47 of BarqTrain): a layer with max_batch_size=1, max_cache_len=8,
  page_size=4 receives arange-valued K/V of 3 then 2 tokens (the second append crosses the
  page boundary at slot 4); the expected returns are the concatenations the test asserts.
* config1_digests.json -- for configuration 1 (2 layers, batch 1, 4 heads x 64, page 16, fp32,
  prefill 32 + 128 decode steps, inputs from tests/kvgen.py seed 1001): per layer and step the
  first 16 hex digits of SHA-256 over the gathered K bytes then V bytes, computed with the
  slot-history model (tests/slot_history.py), which shares nothing with the oracle.

Neither file is produced by running the reference.
"""

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from kvgen import C1, config1_steps, to_bits  # noqa: E402
from slot_history import SlotHistory  # noqa: E402


def known_answer():
    k1 = np.arange(24, dtype=np.float32).reshape(1, 2, 3, 4)
    v1 = k1 + 100.0
    k2 = np.arange(16, dtype=np.float32).reshape(1, 2, 2, 4) + 1000.0
    v2 = k2 + 100.0
    return {
        "source": "BarqTrain tests/test_kv_cache.py:24-47",
        "layer": {"max_batch_size": 1, "max_cache_len": 8, "page_size": 4},
        "dtype": "float32",
        "calls": [
            {"keys": k1.tolist(), "values": v1.tolist(),
             "expect_keys": k1.tolist(), "expect_values": v1.tolist(), "expect_seq_length": 3},
            {"keys": k2.tolist(), "values": v2.tolist(),
             "expect_keys": np.concatenate([k1, k2], axis=2).tolist(),
             "expect_values": np.concatenate([v1, v2], axis=2).tolist(), "expect_seq_length": 5},
        ],
    }


def config1_digests():
    models = [SlotHistory(C1["batch"]) for _ in range(C1["layers"])]
    out = {"config": {k: (str(v) if k == "dtype" else v) for k, v in C1.items()}, "layers": []}
    digests = [[] for _ in models]
    for step in config1_steps():
        for layer, (k, v) in enumerate(step):
            m = models[layer]
            m.append(to_bits(k), to_bits(v))
            gk, gv = m.gather(C1["heads"], C1["dim"], np.uint32)
            h = hashlib.sha256(gk.tobytes() + gv.tobytes()).hexdigest()[:16]
            digests[layer].append(h)
    out["layers"] = digests
    return out


if __name__ == "__main__":
    with open(os.path.join(HERE, "known_answer_update.json"), "w") as f:
        json.dump(known_answer(), f, indent=1)
    with open(os.path.join(HERE, "config1_digests.json"), "w") as f:
        json.dump(config1_digests(), f, indent=1)
    print("fixtures written")
