"""The back part of the 12 Hz decoder on the GPU (TQwenCodecVulkan.Back,
codec.vulkan.pas:568-652) through the C ABI, against the oracle (pinned to a
float64 PyTorch composition, tests/test_oracle_codec.py). Bars from the
reference's own GPU codec test (tests/test.tts.qwen.codec.vulkan.pas:46-49,
143-165): the wav within 2e-5 absolute, and chunks of 1, 4 and all frames
giving the same samples, bit for bit."""
import numpy as np
import pytest

import q3h
import q3o
import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def weights():
    return synth.codec_weights(1)


def _gpu(device, w, x, chunks, max_frames=16):
    c = q3h.Codec(device, w, max_frames=max_frames)
    out, f = [], 0
    try:
        for n in chunks:
            print(f"codec back: {n} frame(s)", flush=True)
            out.append(c.back(x[f:f + n]))
            f += n
    finally:
        c.destroy()
    return np.concatenate(out)


def test_codec_matches_oracle(device, weights):
    x = synth.prompt(3, 6)
    gpu = _gpu(device, weights, x, [1, 2, 3])
    oc = q3o.Codec(weights)
    ref = np.concatenate([oc.back(x[:3]), oc.back(x[3:])])
    oc.destroy()
    d = np.abs(gpu - ref).max()
    print(f"max |gpu - oracle| = {d:.3g}, peak {np.abs(ref).max():.3g}")
    assert d <= 2e-5, d


def test_codec_chunks_give_the_same_samples(device, weights):
    x = synth.prompt(4, 8)
    one = _gpu(device, weights, x, [1] * 8)
    four = _gpu(device, weights, x, [4, 4])
    all_ = _gpu(device, weights, x, [8])
    passes = _gpu(device, weights, x, [8], max_frames=3)  # passes of 3, 3, 2 inside
    assert np.array_equal(one, four) and np.array_equal(one, all_)
    assert np.array_equal(one, passes)


def test_codec_reset_and_errors(device, weights):
    x = synth.prompt(5, 2)
    c = q3h.Codec(device, weights, max_frames=4)
    try:
        a = c.back(x)
        b = c.back(x)
        assert not np.array_equal(a, b)  # the histories carry the first call
        c.reset()
        assert np.array_equal(c.back(x), a)
        assert c.back(np.zeros((0, 1024), np.float32)).shape == (0,)
        assert c.bytes > 100 * 1024 * 1024
    finally:
        c.destroy()
    bad = dict(weights)
    bad["conv0_w"] = None
    with pytest.raises(q3h.Q3HError) as e:
        q3h.Codec(device, bad)
    assert e.value.code == q3h.E_ARG and "NULL" in str(e.value)
    with pytest.raises(q3h.Q3HError) as e:
        q3h.Codec(device, weights, max_frames=0)
    assert e.value.code == q3h.E_ARG
