"""The oracle's NextFrame composition (q3o_frame_next, a restatement of
mormot.ai.tts.qwen.talker.pas:640-681) pinned by marker tables through
zero-weight stacks (tests/markers.py): the codes of every frame follow the
closed-form chain of the tables and heads, and the talker's normed state
decodes to the 16 markers of the frame's codes plus trailing row `frame`
(then tts_pad). Nothing of the oracle is used to compute the expectation."""
import numpy as np
import pytest

import q3o
import synth
from markers import GROUPS, Markers, decode_state, zero_stack

FRAMES = 12  # > 4: code 0 repeats (4-cycles), so the repetition penalty runs


def oracle_markers_frame(mk, dtype, act_q8, talker_layers=2, cp_layers=1):
    tdims = dict(synth.TALKER, layers=talker_layers)
    cdims = dict(synth.PREDICTOR, layers=cp_layers)
    q = q3o.quantize_q8_0 if dtype == q3o.Q8_0 else (lambda a: a)

    def stack(dims):
        layers, final = zero_stack(dims)
        for L in layers:
            for k in synth.MATRICES:
                L[k] = q(L[k])
        return q3o.Stack(dims, layers, final, dtype, act_q8=act_q8)
    ot, oc = stack(tdims), stack(cdims)
    fr = q3o.Frame(ot, oc, q(mk.talker_head), [q(h) for h in mk.cp_heads], mk.codec_emb,
                   mk.pred_emb, mk.tts_pad, eos=2150, max_positions=64)
    return fr, ot, oc


@pytest.mark.parametrize("dtype,act_q8", [(q3o.F32, 0), (q3o.Q8_0, 0), (q3o.Q8_0, 1)],
                         ids=["f32", "q8_0", "q8_0_int8_act"])
def test_oracle_frame_composition_markers(dtype, act_q8):
    mk = Markers(seed=5)
    start15 = int(mk.sets[GROUPS - 1][3])
    expect = mk.chain(start15, FRAMES)
    fr, ot, oc = oracle_markers_frame(mk, dtype, act_q8)
    fr.start(mk.prefill(6, start15), mk.trailing)
    try:
        for i in range(FRAMES):
            codes = fr.next()
            assert codes is not None
            assert np.array_equal(codes, expect[i]), (i, codes, expect[i])
            _, past = fr.state()
            assert np.array_equal(decode_state(past), mk.state_columns(codes, i)), i
    finally:
        for o in (fr, ot, oc):
            o.destroy()


def test_markers_detect_a_wrong_composition():
    """The marker expectation is not vacuous: with pred_emb shifted by one
    table (pred_emb[g] gathered where pred_emb[g - 1] belongs) the chain breaks
    at code 2, and with the trailing rows swapped the decoded state differs."""
    mk = Markers(seed=5)
    start15 = int(mk.sets[GROUPS - 1][3])
    expect = mk.chain(start15, 2)
    wrong = Markers(seed=5)
    wrong.pred_emb = mk.pred_emb[1:] + mk.pred_emb[:1]
    fr, ot, oc = oracle_markers_frame(wrong, q3o.F32, 0)
    fr.start(mk.prefill(6, start15), mk.trailing)
    codes = fr.next()
    for o in (fr, ot, oc):
        o.destroy()
    assert codes[0] == expect[0][0] and codes[1] == expect[0][1]
    assert codes[2] != expect[0][2]
    fr, ot, oc = oracle_markers_frame(mk, q3o.F32, 0)
    fr.start(mk.prefill(6, start15), mk.trailing[::-1].copy())
    codes = fr.next()
    _, past = fr.state()
    for o in (fr, ot, oc):
        o.destroy()
    assert np.array_equal(codes, expect[0])
    assert not np.array_equal(decode_state(past), mk.state_columns(codes, 0))


def test_oracle_frame_matches_a_transformers_composition():
    """The oracle's frame with random f32 weights against NextFrame composed
    over transformers' Qwen3 decoder (tests/frame_torch.py): identical codes
    for every frame, the talker logits and normed state within 1e-4 (the
    reference's f32 bar). This pins what the zero-weight markers cannot see:
    the past state as row 0 of the code predictor (it reaches row 1 only
    through attention), the code-predictor context reset per frame and the
    talker K/V carried across frames."""
    from frame_torch import TorchFrame, TorchStack
    seed = 31
    tdims = dict(synth.TALKER, layers=2)
    cdims = dict(synth.PREDICTOR, layers=2)
    tl, tf = synth.stack_weights(seed, "talker.model.", tdims, norm_std=0.1)
    cl, cf = synth.stack_weights(seed, "talker.code_predictor.model.", cdims, norm_std=0.1)
    th = synth.talker_head(seed)
    ch = [synth.cp_head(seed, g) for g in range(15)]
    ce = synth.codec_embedding(seed)
    pe = [synth.pred_embedding(seed, g) for g in range(15)]
    pad = synth.tts_pad(seed)
    pre = synth.prompt(seed, 10)
    trailing = synth.normal(seed, "trailing", (3, 1024), 0.02)
    tf_ = TorchFrame(TorchStack(tdims, tl, tf), TorchStack(cdims, cl, cf), th, ch, ce, pe, pad,
                     eos=2150)
    ot = q3o.Stack(tdims, tl, tf, q3o.F32)
    oc = q3o.Stack(cdims, cl, cf, q3o.F32)
    of = q3o.Frame(ot, oc, th, ch, ce, pe, pad, eos=2150, max_positions=64)
    try:
        tf_.start(pre, trailing)
        of.start(pre, trailing)
        for i in range(6):
            want = tf_.next()
            got = of.next()
            assert np.array_equal(got, want), (i, got, want)
            lg, past = of.state()
            assert np.max(np.abs(lg - tf_.logits)) <= 1e-4 * np.max(np.abs(tf_.logits)), i
            assert np.max(np.abs(past - tf_.past)) <= 1e-4 * np.max(np.abs(tf_.past)), i
    finally:
        for o in (of, ot, oc):
            o.destroy()


def run_oracle(mk, frames, start15, eos, dtype=q3o.F32, act_q8=0):
    fr, ot, oc = oracle_markers_frame(mk, dtype, act_q8)
    fr.start(mk.prefill(6, start15), mk.trailing)
    out = []
    try:
        for _ in range(frames):
            c = fr.next()
            out.append(None if c is None else np.array(c, np.int64))
            if c is None:
                break
    finally:
        for o in (fr, ot, oc):
            o.destroy()
    return out


def same(a, b):
    return len(a) == len(b) and all((x is None and y is None) or
                                    (x is not None and y is not None and np.array_equal(x, y))
                                    for x, y in zip(a, b))


@pytest.mark.parametrize("dtype,act_q8", [(q3o.F32, 0), (q3o.Q8_0, 1)], ids=["f32", "int8"])
def test_oracle_frame_repetition_penalty_decides(dtype, act_q8):
    """A second talker-head row per marker at 0.97 of the first: once the
    first code was returned, the penalty (x / 1.05 < 0.97 x) hands code 0 to
    the alternative. The oracle follows the reference's ChooseCode0 loop."""
    mk = Markers(seed=6)
    mk.add_alternatives(0.97)
    start15 = int(mk.sets[GROUPS - 1][1])
    want = mk.run(start15, 20, eos=2150)
    plain = Markers(seed=6).run(start15, 20, eos=2150)
    assert not same(want, plain)  # the penalty changed some code 0
    assert same(run_oracle(mk, 20, start15, 2150, dtype, act_q8), want)


def test_oracle_frame_eos_ends_the_sentence():
    """eos wins the code 0 after a frame ending in a given code 15, but not
    before two frames were returned (ChooseCode0's processors)."""
    mk = Markers(seed=7)
    start15 = int(mk.sets[GROUPS - 1][2])
    plain = mk.chain(start15, 12)
    trigger = int(plain[0][-1])  # frame 0's code 15: eos still forbidden after it
    mk.add_eos(2150, trigger)
    want = mk.run(start15, 12, eos=2150)
    assert want[-1] is None and len(want) > 2
    assert same(run_oracle(mk, 12, start15, 2150), want)
