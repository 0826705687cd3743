"""The device frame step's composition against the closed form of marker
tables through zero-weight stacks (tests/markers.py), independently of the
oracle: for every frame and stream the 16 codes follow the chain of the
tables and heads, and the talker's normed state (q3h_frame_state) decodes to
the 16 markers of the frame's codes plus the stream's trailing row, then
tts_pad (TQwenTalker.NextFrame, mormot.ai.tts.qwen.talker.pas:649-677).

Each kernel path of the frame runs: one stream on the fused code-predictor
kernels with the greedy argmax inside the next product (graph and direct
launches), several streams on the general path, f32 weights, and the int8
path (Q8_0 activations)."""
import numpy as np
import pytest

import q3h
import synth
from markers import GROUPS, Markers, decode_state, zero_stack

pytestmark = pytest.mark.gpu

FRAMES = 12

VARIANTS = {
    "q8_b1_graph": dict(dtype=q3h.Q8_0, act_q8=0, n=1, use_graph=True),
    "q8_b1_direct": dict(dtype=q3h.Q8_0, act_q8=0, n=1, use_graph=False),
    "q8_b3": dict(dtype=q3h.Q8_0, act_q8=0, n=3, use_graph=True),
    "f32_b1": dict(dtype=q3h.F32, act_q8=0, n=1, use_graph=True),
    "int8_b1": dict(dtype=q3h.Q8_0, act_q8=1, n=1, use_graph=True),
    "int8_b4": dict(dtype=q3h.Q8_0, act_q8=1, n=4, use_graph=True),
}


@pytest.mark.parametrize("name", list(VARIANTS))
def test_frame_markers(device, name):
    v = VARIANTS[name]
    print(f"markers frame {name}", flush=True)
    mk = Markers(seed=5)
    tdims = dict(synth.TALKER, layers=2)
    cdims = dict(synth.PREDICTOR, layers=5)
    tl, tf = zero_stack(tdims)
    cl, cf = zero_stack(cdims)
    ts = q3h.Stack(device, dict(tdims, dtype=v["dtype"], kv_f16=0, act_q8=v["act_q8"],
                                max_positions=64), tl, tf, q3h.F32)
    cs = q3h.Stack(device, dict(cdims, dtype=v["dtype"], kv_f16=0, act_q8=v["act_q8"],
                                max_positions=16), cl, cf, q3h.F32)
    ts.add_head(mk.talker_head, q3h.F32)
    for h in mk.cp_heads:
        cs.add_head(h, q3h.F32)
    n = v["n"]
    fr = q3h.Frame(ts, cs, mk.codec_emb, mk.pred_emb, mk.tts_pad, n_streams=n, eos=2150,
                   max_positions=64, max_frames=32, use_graph=v["use_graph"])
    try:
        starts = [int(mk.sets[GROUPS - 1][(3 + 2 * s) % 8]) for s in range(n)]
        ntrail = [(s % 4) + 1 for s in range(n)]
        for s in range(n):
            fr.start(s, mk.prefill(5 + s, starts[s]), mk.trailing[:ntrail[s]])
        expect = [mk.chain(starts[s], FRAMES) for s in range(n)]
        for i in range(FRAMES):
            codes, alive = fr.step()
            for s in range(n):
                assert alive[s] == 1
                assert np.array_equal(codes[s], expect[s][i]), (name, s, i, codes[s],
                                                                expect[s][i])
                _, past = fr.state(s)
                assert np.array_equal(decode_state(past),
                                      mk.state_columns(codes[s], i, ntrail[s])), (name, s, i)
    finally:
        fr.destroy()
        ts.destroy()
        cs.destroy()


def marker_frame(device, mk, v, max_frames=32):
    tdims = dict(synth.TALKER, layers=2)
    cdims = dict(synth.PREDICTOR, layers=5)
    tl, tf = zero_stack(tdims)
    cl, cf = zero_stack(cdims)
    ts = q3h.Stack(device, dict(tdims, dtype=v["dtype"], kv_f16=0, act_q8=v["act_q8"],
                                max_positions=64), tl, tf, q3h.F32)
    cs = q3h.Stack(device, dict(cdims, dtype=v["dtype"], kv_f16=0, act_q8=v["act_q8"],
                                max_positions=16), cl, cf, q3h.F32)
    ts.add_head(mk.talker_head, q3h.F32)
    for h in mk.cp_heads:
        cs.add_head(h, q3h.F32)
    fr = q3h.Frame(ts, cs, mk.codec_emb, mk.pred_emb, mk.tts_pad, n_streams=v["n"], eos=2150,
                   max_positions=64, max_frames=max_frames, use_graph=v["use_graph"])
    return fr, ts, cs


@pytest.mark.parametrize("name", ["q8_b1_graph", "q8_b3", "int8_b4"])
def test_frame_repetition_penalty_decides(device, name):
    """Code 0 decided by the repetition penalty (tests/markers.py
    add_alternatives): the device's seen-code flags against the reference's
    ChooseCode0 loop, frame by frame."""
    v = VARIANTS[name]
    print(f"penalty frame {name}", flush=True)
    mk = Markers(seed=6)
    mk.add_alternatives(0.97)
    n = v["n"]
    starts = [int(mk.sets[GROUPS - 1][(1 + s) % 8]) for s in range(n)]
    want = [mk.run(st, 16, eos=2150) for st in starts]
    plain = Markers(seed=6)
    assert any(not np.array_equal(a, b) for a, b in zip(want[0], plain.run(starts[0], 16)))
    fr, ts, cs = marker_frame(device, mk, v)
    try:
        for s in range(n):
            fr.start(s, mk.prefill(4, starts[s]), mk.trailing)
        for i in range(16):
            codes, alive = fr.step()
            for s in range(n):
                assert alive[s] == 1 and np.array_equal(codes[s], want[s][i]), (name, s, i)
    finally:
        fr.destroy()
        ts.destroy()
        cs.destroy()


@pytest.mark.parametrize("name", ["q8_b1_graph", "q8_b1_direct", "q8_b3", "int8_b1", "int8_b4"])
def test_frame_eos_then_restart(device, name):
    """eos ends stream 0 (codes -1, alive 0) in the frame the reference's
    NextFrame returns false; at batch 1 the step that meets eos runs its whole
    captured graph with the stream dead. Then the stream starts again and its
    frames follow the chain from the new prefill."""
    v = VARIANTS[name]
    print(f"eos frame {name}", flush=True)
    mk = Markers(seed=7)
    start15 = int(mk.sets[GROUPS - 1][2])
    trigger = int(mk.chain(start15, 1)[0][-1])
    mk.add_eos(2150, trigger)
    want = mk.run(start15, 12, eos=2150)
    assert want[-1] is None
    n = v["n"]
    fr, ts, cs = marker_frame(device, mk, v)
    try:
        other = int(mk.sets[GROUPS - 1][5])
        other_want = mk.run(other, 12, eos=2150)
        for s in range(n):
            fr.start(s, mk.prefill(4, start15 if s == 0 else other), mk.trailing)
        for i, w in enumerate(want):
            codes, alive = fr.step()
            if w is None:
                assert alive[0] == 0 and np.all(codes[0] == -1), (name, i)
            else:
                assert alive[0] == 1 and np.array_equal(codes[0], w), (name, i)
            for s in range(1, n):
                ow = other_want[i] if i < len(other_want) else None
                if ow is None:
                    assert alive[s] == 0
                else:
                    assert alive[s] == 1 and np.array_equal(codes[s], ow), (name, s, i)
        # the ended stream starts again
        fr.start(0, mk.prefill(3, start15), mk.trailing)
        for i in range(3):
            codes, alive = fr.step()
            assert alive[0] == 1 and np.array_equal(codes[0], want[i]), (name, "restart", i)
    finally:
        fr.destroy()
        ts.destroy()
        cs.destroy()
