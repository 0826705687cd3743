"""Pins the oracle's text projection and Start row layout (CPU only).

TQwenTalker.TextProject (talker.pas:390-421) has no golden vector in the
reference (its fixture starts from the summed prefill rows, talker.embed), so
the oracle's q3o_text_project is pinned by:
- torch in float64 (F.linear, F.silu, torch's own bfloat16 widening) on
  random tables: a dropped bias, a transposed weight or a wrong SiLU fails;
- the clamp's closed form: with fc1 = 0 the SiLU input is the bias, so an
  entry below -80 contributes exactly 0 while one just above it contributes
  v e^v != 0 (F.silu gives a tiny nonzero value at -100: the clamp is the
  reference's own rule);
- BF16 widening: a BF16 table and the f32 table of the same values (bits
  shifted in numpy) give identical outputs;
- out-of-range ids raise, as EQwenTalker does (talker.pas:405-406).

The Start row layout (talker.pas:520-580) is pinned with marker projections:
every projected text id and codec id is a one-hot column, so each row decodes
to the (text id, codec id) pair it holds; the expected sequence is written
out from the layout Start documents (role; tts_pad x (codec - 2) + tts_bos
over the codec ids but the last; then the text over codec_pad, tts_eos over
codec_pad, tts_pad over codec_bos - or the first text token over codec_bos
and the rest as trailing rows ending with tts_eos).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F


def _bf16_table(rng, vocab, cols, scale=1.0):
    x = torch.from_numpy((rng.standard_normal((vocab, cols)) * scale).astype(np.float32))
    b = x.to(torch.bfloat16)
    bits = b.view(torch.int16).numpy().view(np.uint16).copy()
    return bits, b.to(torch.float64)


def _weights(rng, th, h, scale1=None, scale2=None):
    s1 = scale1 if scale1 is not None else 1.0 / np.sqrt(th)
    s2 = scale2 if scale2 is not None else 1.0 / np.sqrt(th)
    w1 = (rng.standard_normal((th, th)) * s1).astype(np.float32)
    b1 = (rng.standard_normal(th) * 0.5).astype(np.float32)
    w2 = (rng.standard_normal((h, th)) * s2).astype(np.float32)
    b2 = (rng.standard_normal(h) * 0.5).astype(np.float32)
    return w1, b1, w2, b2


def test_text_project_matches_torch_float64(q3o):
    rng = np.random.default_rng(3)
    vocab, th, h = 50, 128, 64
    bits, emb64 = _bf16_table(rng, vocab, th, 2.0)
    w1, b1, w2, b2 = _weights(rng, th, h, scale1=4.0 / np.sqrt(th))
    ids = np.array([0, 7, 49, 7, 13, 2, 31], np.int32)
    y = q3o.text_project(bits, w1, b1, w2, b2, ids)
    e = emb64[torch.from_numpy(ids.astype(np.int64))]
    t = lambda a: torch.from_numpy(a).to(torch.float64)
    hid = F.linear(e, t(w1), t(b1))
    ref = F.linear(F.silu(hid), t(w2), t(b2)).numpy()
    # some SiLU inputs are far below zero, none below -80 here
    assert hid.min().item() < -5 and hid.min().item() > -80
    assert np.abs(y - ref).max() <= 2e-5 * max(1.0, np.abs(ref).max())


def test_silu_clamp_closed_form(q3o):
    th, h = 64, 32
    w1 = np.zeros((th, th), np.float32)
    b1 = np.zeros(th, np.float32)
    b1[:6] = [-100.0, -80.5, -80.0, -79.5, 0.0, 5.0]
    w2 = np.zeros((h, th), np.float32)
    w2[np.arange(h), np.arange(h)] = 1.0  # y[j] = silu(b1[j]) + b2[j]
    b2 = np.zeros(h, np.float32)
    emb = np.ones((3, th), np.float32)
    y = q3o.text_project(emb, w1, b1, w2, b2, [1])[0]
    assert y[0] == 0.0 and y[1] == 0.0  # below -80: exactly 0
    # -80 itself is not below -80: v / (1 + e^80) (tiny, nonzero, negative)
    for j, v in ((2, -80.0), (3, -79.5), (5, 5.0)):
        exact = v / (1.0 + np.exp(-v))
        assert y[j] < 0 or v > 0
        assert abs(y[j] - exact) <= 1e-6 * abs(exact), (j, y[j], exact)
    assert y[4] == 0.0
    # torch's SiLU at -100 is not 0: the clamp is a rule of its own
    assert F.silu(torch.tensor(-100.0, dtype=torch.float64)).item() != 0.0


def test_bf16_table_equals_widened_f32_table(q3o):
    rng = np.random.default_rng(5)
    vocab, th, h = 20, 64, 32
    x = (rng.standard_normal((vocab, th)) * np.exp(rng.uniform(-20, 5, (vocab, th))))
    bits = (x.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    f32 = (bits.astype(np.uint32) << 16).view(np.float32)  # the same values in f32
    w1, b1, w2, b2 = _weights(rng, th, h)
    ids = np.arange(vocab, dtype=np.int32)[::-1].copy()
    a = q3o.text_project(bits, w1, b1, w2, b2, ids)
    b = q3o.text_project(f32, w1, b1, w2, b2, ids)
    assert np.array_equal(a, b)


def test_text_project_errors_and_empty(q3o):
    rng = np.random.default_rng(6)
    w1, b1, w2, b2 = _weights(rng, 64, 32)
    emb = np.zeros((4, 64), np.float32)
    assert q3o.text_project(emb, w1, b1, w2, b2, []).shape == (0, 32)
    for bad in ([4], [-1], [0, 1, 5]):
        with pytest.raises(IndexError):
            q3o.text_project(emb, w1, b1, w2, b2, bad)


# ---- the Start row layout ----

TV, CV = 40, 24  # text ids and codec ids of the marker tables
H = TV + CV


def _marker_project(ids):
    out = np.zeros((len(ids), H), np.float32)
    for r, i in enumerate(ids):
        out[r, i] = 1.0
    return out


def _decode(rows):
    got = []
    for r in rows:
        t = np.nonzero(r[:TV])[0]
        c = np.nonzero(r[TV:])[0]
        assert len(t) == 1 and len(c) <= 1
        got.append((int(t[0]), int(c[0]) if len(c) else None))
    return got


@pytest.mark.parametrize("non_streaming", [True, False])
@pytest.mark.parametrize("n_text,codec", [(1, [3, 4, 5, 6, 7]), (4, [3, 4, 9, 5, 6, 7]),
                                          (6, [8, 4, 10, 5, 11, 6, 7])])
def test_start_rows_layout(q3o, non_streaming, n_text, codec):
    codec_emb = np.zeros((CV, H), np.float32)
    codec_emb[np.arange(CV), TV + np.arange(CV)] = 1.0
    role = [30, 31, 32]
    text = list(range(10, 10 + n_text))
    tail = [33, 34, 30, 31, 32]
    ids = role + text + tail
    bos, eos, pad, cpad, cbos = 1, 2, 0, 6, 7
    pre, trail = q3o.start_rows(_marker_project, codec_emb, ids, codec, bos, eos, pad, cpad,
                                cbos, non_streaming)
    nc = len(codec)
    expect = [(30, None), (31, None), (32, None)]
    expect += [(pad, codec[i]) for i in range(nc - 2)] + [(bos, codec[nc - 2])]
    if non_streaming:
        expect += [(t, cpad) for t in text] + [(eos, cpad), (pad, cbos)]
        expect_trail = [(pad, None)]
        assert len(pre) == 3 + (nc - 1) + (n_text + 1) + 1  # talker.pas:531-532
    else:
        expect += [(text[0], cbos)]
        expect_trail = [(t, None) for t in text[1:]] + [(eos, None)]
        assert len(pre) == 3 + (nc - 1) + 1  # talker.pas:533-534
    assert _decode(pre) == expect
    assert _decode(trail) == expect_trail


def test_start_rows_rejects_empty_text(q3o):
    with pytest.raises(ValueError):
        q3o.start_rows(_marker_project, np.zeros((CV, H), np.float32), [1] * 8, [6, 7],
                       1, 2, 0, 6, 7, True)
