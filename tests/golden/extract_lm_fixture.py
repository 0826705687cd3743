"""Write tests/golden/qwen3_tts_lm_fixture.npz from the reference's own fixture
tests/data/infer-ref/qwen3-tts-lm/{manifest.json,tensors.bin} (data captured
from PyTorch with the real model weights). Only the tensors the offline tests
can use are kept: talker.logits_last [3072], predictor.logits [15][2048],
predictor.codes [16], predictor.embed [16][1024] and the last row of
talker.norm [1024]. Each tensor's sha256 is checked against the manifest
first.

Run in the build container: python tests/golden/extract_lm_fixture.py
"""
import hashlib
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = "/root/reference/tests/data/infer-ref/qwen3-tts-lm"
KEEP = ("talker.logits_last", "predictor.logits", "predictor.codes", "predictor.embed",
        "talker.norm")


def main():
    with open(os.path.join(SRC, "manifest.json"), encoding="utf-8") as f:
        man = json.load(f)
    with open(os.path.join(SRC, man["blob"]["file"]), "rb") as f:
        blob = f.read()
    assert hashlib.sha256(blob).hexdigest() == man["blob"]["sha256"]
    out = {}
    for t in man["tensors"]:
        if t["name"] not in KEEP:
            continue
        raw = blob[t["offset"]:t["offset"] + t["bytes"]]
        assert hashlib.sha256(raw).hexdigest() == t["sha256"], t["name"]
        dt = {"f32": "<f4", "i32": "<i4"}[t["dtype"]]
        a = np.frombuffer(raw, dtype=dt).reshape(t["shape"])
        key = t["name"].replace(".", "_")
        if t["name"] == "talker.norm":
            a = a[-1]
            key = "talker_norm_last"
        out[key] = a.copy()
    np.savez(os.path.join(HERE, "qwen3_tts_lm_fixture.npz"), **out)
    print({k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
