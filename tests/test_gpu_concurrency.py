"""The reference's threading on one device: the talker steps frames on the
producer thread (TQwenTtsProducer.Execute, src/tts/mormot.ai.tts.qwen.pas:
276-319) while the speaking thread decodes earlier frames through the codec's
back part on the same GPU (TQwenCodecVulkan.Back under GpuLock,
src/tts/mormot.ai.tts.qwen.codec.vulkan.pas:633-652). Here both run through
the C ABI from two Python threads at once (ctypes releases the interpreter
lock during each call), and their outputs must equal those of serial runs, bit
for bit."""
import threading

import numpy as np
import pytest

import q3h
from models import Model

pytestmark = pytest.mark.gpu


def _both(fa, fb, timeout=120):
    out, err = {}, []

    def wrap(name, fn):
        try:
            out[name] = fn()
        except BaseException as e:  # reported by the main thread
            err.append(e)
    ta = threading.Thread(target=wrap, args=("a", fa))
    tb = threading.Thread(target=wrap, args=("b", fb))
    ta.start()
    tb.start()
    ta.join(timeout)
    tb.join(timeout)
    assert not ta.is_alive() and not tb.is_alive(), "a thread did not finish"
    if err:
        raise err[0]
    return out["a"], out["b"]


def test_frame_and_codec_from_two_threads(device, synth):
    m = Model(device, seed=21, talker_layers=2, cp_layers=1, max_positions=128)
    w = synth.codec_weights(2)
    rows = synth.prompt(33, 24)
    pre = synth.prompt(34, 20)
    fr = m.frame(n_streams=1, max_positions=128)
    codec = q3h.Codec(device, w, max_frames=4)

    def frames():
        fr.start(0, pre)
        return np.stack([fr.step()[0][0].copy() for _ in range(12)])

    def decode():
        codec.reset()
        return np.concatenate([codec.back(rows[i:i + 2]) for i in range(0, 24, 2)])

    try:
        want_codes, want_pcm = frames(), decode()
        for r in range(3):
            print(f"concurrent round {r}", flush=True)
            codes, pcm = _both(frames, decode)
            assert np.array_equal(codes, want_codes), r
            assert np.array_equal(pcm, want_pcm), r
    finally:
        fr.destroy()
        codec.destroy()
        m.destroy()


def test_two_frames_from_two_threads(device, synth):
    """Two sentences on two frames over the same stacks, stepped by two
    threads at once (each frame, with its contexts, used by one thread at a
    time: talker.pas:77)."""
    m = Model(device, seed=22, talker_layers=2, cp_layers=1, max_positions=128)
    fa = m.frame(n_streams=1, max_positions=128)
    fb = m.frame(n_streams=2, max_positions=128)
    pa, pb = synth.prompt(35, 17), synth.prompt(36, 29)

    def run_a():
        fa.start(0, pa)
        return np.stack([fa.step()[0][0].copy() for _ in range(10)])

    def run_b():
        fb.start(0, pb)
        fb.start(1, pa)
        return np.stack([fb.step()[0].copy() for _ in range(10)])

    try:
        want_a, want_b = run_a(), run_b()
        for r in range(3):
            print(f"concurrent round {r}", flush=True)
            got_a, got_b = _both(run_a, run_b)
            assert np.array_equal(got_a, want_a) and np.array_equal(got_b, want_b), r
    finally:
        fa.destroy()
        fb.destroy()
        m.destroy()
