"""Pins the oracle's back part of the 12 Hz decoder (TQwenCodec.Back,
codec.pas:1040-1083) on the CPU.

The reference's codec tests compare against PyTorch outputs of the real model
(tests/test.tts.qwen.codec.pas: stages within 1e-4 relative, the wav within
1e-5), which are absent here (no model weights). The oracle is pinned instead
against a float64 PyTorch composition of the same modules over the whole
sequence (tests/codec_torch.py: torch conv1d with causal padding,
conv_transpose1d truncated to T stride samples, layer_norm, erf GELU, the
SnakeBeta formula), on seeded weights, decoded here in chunks with the
histories carried from call to call; and by the reference's own chunking
property (tests/test.tts.qwen.codec.pas:221-242: chunks of 1, 4 and all
frames give the same samples)."""
import numpy as np

import codec_torch


def _decode(q3o, w, x, chunks):
    c = q3o.Codec(w)
    out, f = [], 0
    for n in chunks:
        out.append(c.back(x[f:f + n]))
        f += n
    c.destroy()
    return np.concatenate(out)


def test_codec_back_matches_torch(q3o, synth):
    w = synth.codec_weights(1)
    x = synth.prompt(3, 6)
    stages = {}
    ref = codec_torch.back(w, x, stages)
    assert np.abs(stages["out"]).max() < 1.0  # no clipping: the comparison sees every sample
    pcm = _decode(q3o, w, x, [1, 2, 3])
    assert pcm.shape == (6 * 1920,)
    assert np.abs(pcm - ref).max() < 1e-5, np.abs(pcm - ref).max()


def test_codec_chunks_give_the_same_samples(q3o, synth):
    w = synth.codec_weights(2)
    x = synth.prompt(4, 5)
    one = _decode(q3o, w, x, [1] * 5)
    two = _decode(q3o, w, x, [2, 3])
    all_ = _decode(q3o, w, x, [5])
    assert np.array_equal(one, two) and np.array_equal(one, all_)


def test_codec_reset(q3o, synth):
    w = synth.codec_weights(2)
    x = synth.prompt(5, 2)
    c = q3o.Codec(w)
    a = c.back(x)
    c.back(x)  # histories now hold this sentence
    c.reset()
    b = c.back(x)
    c.destroy()
    assert np.array_equal(a, b)
